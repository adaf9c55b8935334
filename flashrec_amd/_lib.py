"""ctypes binding of ``libflashrec_amd.so`` (declared in ``include/flashrec_amd.h``).

The library is loaded lazily on first use and there is no fallback: if it is
missing or a call reports an error, the caller gets an exception.  Tensors
cross the boundary as raw ``data_ptr()`` integers plus strides; the stream is
``torch.cuda.current_stream().cuda_stream``.
"""

from __future__ import annotations

import ctypes
import os
from pathlib import Path
from typing import Optional

import torch

LIB_PATH = Path(os.environ.get("FLASHREC_AMD_LIB") or Path(__file__).resolve().parent / "libflashrec_amd.so")

FR_OK = 0
FR_EINVAL = 1
FR_EUNSUPPORTED = 2
FR_ELAUNCH = 3
FR_ETOOLARGE = 4
GENREC_NOALLOC_SCRATCH_BYTES = 4 << 20  # FR_GENREC_NOALLOC_SCRATCH_BYTES

DTYPE_CODE = {
    torch.bfloat16: 0,
    torch.float16: 1,
    torch.float32: 2,
    torch.float8_e4m3fn: 3,
}

_P = ctypes.c_void_p
_I64 = ctypes.c_int64
_I32 = ctypes.c_int
_F32 = ctypes.c_float

# name -> argtypes; every symbol here is declared in include/flashrec_amd.h
SIGNATURES = {
    "fr_abi_version": [],
    "fr_per_token_quant_fp8": [_P, _I32, _I64, _I64, _I64, _P, _P, _P],
    "fr_quantize_weight_fp8": [_P, _I32, _I64, _I64, _I64, _P, _P, _P],
    "fr_rms_quant_fp8": [_P, _I32, _I64, _P, _I64, _P, _I64, _I64, _F32, _P, _P, _P],
    "fr_rmsnorm": [_P, _I32, _I64, _P, _I64, _P, _P, _I64, _I64, _I64, _F32, _P],
    "fr_silu_quant_fp8": [_P, _I32, _I64, _I64, _I64, _P, _P, _P],
    "fr_silu_and_mul": [_P, _I32, _I64, _P, _I64, _I64, _I64, _P],
    "fr_fp8_scaled_mm": [_P, _I64, _P, _I64, _P, _I64, _P, _I64, _P, _I64, _P, _I64, _I64, _I64, _I64, _I32, _P],
    "fr_fp8_scaled_mm_residual": [_P, _I64, _P, _I64, _P, _I64, _P, _I64, _P, _I64, _P, _I64, _I64, _I64, _I64,
                                  _I32, _P],
    "fr_fp8_scaled_mm_silu": [_P, _I64, _P, _I64, _P, _I64, _P, _I64, _P, _I64, _I64, _I64, _I64, _P],
    "fr_fp8_weight_prearranged_bytes": [_I64, _I64],
    "fr_fp8_weight_prearrange": [_P, _I64, _I64, _I64, _P, _P],
    "fr_fp8_scaled_mm_prearranged": [_P, _I64, _P, _P, _I64, _P, _I64, _P, _I64, _P, _I64, _I64, _I64, _I64, _I32,
                                     _I32, _P],
    "fr_qk_norm_rope_store_fp8": [
        _P, _I64, _I64, _P, _I64, _I64, _P, _I64, _I64,  # q, k, v + strides
        _P, _P, _P, _P, _F32, _P, _I64,  # pos, loc, qw, kw, eps, cos_sin, rows
        _P, _I64, _I64, _P, _I64, _I64, _I64,  # caches + strides, num_slots
        _I64, _I64, _I64, _I64, _P,  # T, Hq, Hk, D, stream
    ],
    "fr_rope_inplace": [_P, _I64, _I64, _P, _I64, _I64, _P, _P, _I64, _I64, _I64, _I64, _I64, _P],
    "fr_rope_inplace_any": [_P, _I64, _I64, _I64, _P, _I64, _I64, _I64, _I32, _P, _P, _I64, _I64, _I64, _I64, _I64,
                            _P],
    "fr_store_kv_fp8": [_P, _I64, _P, _I64, _I32, _P, _P, _I64, _P, _I64, _I64, _I64, _I64, _P],
    "fr_store_kv_bf16": [_P, _I64, _P, _I64, _P, _P, _I64, _P, _I64, _I64, _I64, _I64, _P],
    "fr_rope_store_kv_bf16": [
        _P, _I64, _I64, _P, _I64, _I64, _P, _I64, _I64,  # q, k, v + strides
        _P, _P, _P, _I64,  # positions, loc, cos_sin, rows
        _P, _I64, _I64, _P, _I64, _I64, _I64,  # caches + strides, num_slots
        _I64, _I64, _I64, _I64, _P,  # T, Hq, Hk, D, stream
    ],
    "fr_log_softmax_f32": [_P, _I64, _P, _I64, _I64, _I64, _P],
    "fr_genrec_scratch_bytes": [_I64, _I64, _I64],
    "fr_genrec_mask_topk_expand": [
        _P, _P, _P, _P, _P, _I64,  # outputs, scratch + bytes
        _P, _P, _P, _P, _P,  # cum, top_logprobs, top_tokens, node_ids, allow_table
        _P, _P, _P, _P, _P, _P,  # token_ids in/out, next_node, node_ids_out, do_expand, col
        _I64, _I64, _I64, _I64,  # token_base, n_nodes, vsz, invalid_node
        _I64, _I64, _I64, _I64, _I64,  # N, BW, C, K, L
        _I32, _I32, _I32, _I32, _P,  # apply flags, next_node is int32, stream
    ],
    "fr_genrec_mask_topk_expand_noalloc": [
        _P, _P, _P, _P,  # outputs
        _P, _P, _P, _P, _P,  # cum, top_logprobs, top_tokens, node_ids, allow_table
        _P, _P, _P, _P, _P, _P,  # token_ids in/out, next_node, node_ids_out, do_expand, col
        _I64, _I64, _I64, _I64,  # token_base, n_nodes, vsz, invalid_node
        _I64, _I64, _I64, _I64, _I64,  # N, BW, C, K, L
        _I32, _I32, _I32, _I32, _P,  # apply flags, next_node is int32, stream
    ],
    "fr_trie_mask_candidates": [_P, _P, _P, _P, _P, _I64, _I64, _I64, _I64, _I64, _F32, _P],
    "fr_trie_advance_nodes": [_P, _P, _P, _P, _P, _I32, _I64, _I64, _I64, _I64, _I64, _I64, _I64, _P],
    "fr_beam_expand_token_ids": [_P, _P, _P, _P, _I64, _I64, _I64, _I64, _P],
    "fr_row_topk": [_P, _I64, _I64, _I64, _I64, _P, _P, _P, _P, _P],
    "fr_log_softmax_row_topk": [_P, _I64, _I64, _I64, _I64, _P, _P, _P, _P, _P],
    "fr_paged_attention_fp8": [
        _P, _I64, _I64, _P, _I64, _I64, _P, _I64, _I64,  # q, k_cache, v_cache + strides
        _I64, _P, _P, _P,  # num_slots, kv_indices, kv_start, kv_len
        _P, _I64, _I64, _I64, _I64, _I64, _I64, _F32, _P, _P,  # out + strides, T, Hq, Hk, D, scale, plan, stream
    ],
    "fr_paged_attention_quant_fp8": [
        _P, _I64, _I64, _P, _I64, _I64, _P, _I64, _I64,  # q, k_cache, v_cache + strides
        _I64, _P, _P, _P,  # num_slots, kv_indices, kv_start, kv_len
        _P, _I64, _P, _I64, _I64, _I64, _I64, _F32, _P, _P,  # codes, ldq, scales, T, Hq, Hk, D, scale, plan, stream
    ],
    "fr_paged_attention_plan_size": [_I64, _I64, _I64],
    "fr_calib_mfma_ceiling": [_I64, _I64, _I32, _P, _P, _P],
    "fr_paged_attention_plan": [_P, _P, _P, _I64, _I64, _I64, _P, _P],
}

_LIB: Optional[ctypes.CDLL] = None


class FlashRecKernelError(RuntimeError):
    """A C-ABI call returned a nonzero status."""

    def __init__(self, name: str, code: int):
        self.code = code
        super().__init__(f"{name} failed with status {code}")


class Unsupported(FlashRecKernelError):
    """FR_EUNSUPPORTED: the kernels do not handle this (valid) request."""


def load() -> ctypes.CDLL:
    global _LIB
    if _LIB is not None:
        return _LIB
    if not LIB_PATH.exists():
        raise RuntimeError(
            f"flashrec_amd native library not built: {LIB_PATH} is missing "
            "(run `python -m flashrec_amd.build`); there is no non-HIP path"
        )
    lib = ctypes.CDLL(str(LIB_PATH))
    for name, argtypes in SIGNATURES.items():
        fn = getattr(lib, name)
        fn.argtypes = argtypes
        fn.restype = ctypes.c_int
    lib.fr_paged_attention_plan_size.restype = ctypes.c_int64
    lib.fr_fp8_weight_prearranged_bytes.restype = ctypes.c_int64
    _LIB = lib
    return lib


def call(name: str, *args) -> None:
    rc = getattr(load(), name)(*args)
    if rc == FR_OK:
        return
    if rc == FR_EUNSUPPORTED:
        raise Unsupported(name, rc)
    raise FlashRecKernelError(name, rc)


def stream_of(t: torch.Tensor) -> int:
    return torch.cuda.current_stream(t.device).cuda_stream


def require_device(*tensors: torch.Tensor) -> None:
    """The FP8 path runs only on ROCm device tensors; no CPU fallback exists."""
    for t in tensors:
        if t is not None and not t.is_cuda:
            raise RuntimeError(
                "flashrec_amd kernels take ROCm device tensors only "
                f"(got a {t.device} tensor); there is no CPU path"
            )


def ptr(t: Optional[torch.Tensor]) -> Optional[int]:
    return None if t is None else t.data_ptr()
