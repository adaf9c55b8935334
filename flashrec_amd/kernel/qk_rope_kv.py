"""Fused Q/K RMSNorm + NeoX RoPE + unscaled e4m3 KV scatter, signature of
``flashrec.kernel.qk_rope_kv``.

Reference: python/flashrec/kernel/qk_rope_kv.py:164-250.  Arithmetic is the
reference's unfused sequence (python/flashrec/models/qwen3.py:108-128): per-head
RMSNorm to bf16, rotate-half RoPE in fp32 rounded to bf16, then
``.to(float8_e4m3fn)`` for K and V (python/flashrec/kvcache/pool.py:130-132).
"""

from __future__ import annotations

import torch

from flashrec_amd._lib import Unsupported, call, require_device, stream_of


@torch.compiler.disable
def fused_qk_norm_rope_store_fp8(
    q: torch.Tensor,
    k: torch.Tensor,
    v: torch.Tensor,
    positions: torch.Tensor,
    loc: torch.Tensor,
    q_weight: torch.Tensor,
    k_weight: torch.Tensor,
    eps: float,
    cos_sin_cache: torch.Tensor,
    k_cache: torch.Tensor,
    v_cache: torch.Tensor,
) -> bool:
    """Per-head RMSNorm of q and k, rotate-half RoPE, q written back in
    place, K and V stored as e4m3 (scale 1) into their slots ``loc``.

    Heads are ``[T, H, D]`` views whose last dimension is contiguous (views
    into the fused qkv output need no copy); the pools are ``[slots, H_kv, D]``
    e4m3.  A layout this kernel does not take returns False before any work,
    so the caller can run the unfused steps, the reference's contract.
    """
    require_device(q, k, v, k_cache, v_cache)
    if q.numel() == 0:
        return False
    if k_cache.dtype != torch.float8_e4m3fn or v_cache.dtype != torch.float8_e4m3fn:
        return False
    if q.dim() != 3 or k.dim() != 3 or v.dim() != 3:
        return False
    if q.dtype != torch.bfloat16 or k.dtype != torch.bfloat16 or v.dtype != torch.bfloat16:
        return False
    t, n_q, d = int(q.shape[0]), int(q.shape[1]), int(q.shape[2])
    n_kv = int(k.shape[1])
    if k.shape[0] != t or v.shape[0] != t or v.shape[1] != n_kv:
        return False
    if d > 128 or d % 2 != 0:
        return False
    if int(cos_sin_cache.shape[-1]) != d:
        return False
    if k_cache.dim() != 3 or v_cache.dim() != 3 or k_cache.shape[-1] != d or v_cache.shape[-1] != d:
        return False
    if k_cache.stride(-1) != 1 or v_cache.stride(-1) != 1:
        return False
    q_src = q
    if q.stride(-1) != 1:
        q = q.contiguous()
    if k.stride(-1) != 1:
        k = k.contiguous()
    if v.stride(-1) != 1:
        v = v.contiguous()
    pos = positions.view(-1)[:t].to(dtype=torch.int64).contiguous()
    loc64 = loc.view(-1)[:t].to(dtype=torch.int64).contiguous()
    qw = q_weight.reshape(-1).to(device=q.device, dtype=torch.bfloat16).contiguous()
    kw = k_weight.reshape(-1).to(device=q.device, dtype=torch.bfloat16).contiguous()
    cs = cos_sin_cache.to(device=q.device, dtype=torch.float32).contiguous()
    if int(qw.numel()) != d or int(kw.numel()) != d:
        return False
    try:
        call("fr_qk_norm_rope_store_fp8",
             q.data_ptr(), q.stride(0), q.stride(1),
             k.data_ptr(), k.stride(0), k.stride(1),
             v.data_ptr(), v.stride(0), v.stride(1),
             pos.data_ptr(), loc64.data_ptr(), qw.data_ptr(), kw.data_ptr(), float(eps),
             cs.data_ptr(), cs.shape[0],
             k_cache.data_ptr(), k_cache.stride(0), k_cache.stride(1),
             v_cache.data_ptr(), v_cache.stride(0), v_cache.stride(1), k_cache.shape[0],
             t, n_q, n_kv, d, stream_of(q))
    except Unsupported:
        return False
    if q_src.data_ptr() != q.data_ptr():
        q_src.copy_(q)
    return True
