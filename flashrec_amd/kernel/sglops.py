"""Operator wrappers with the signatures of ``flashrec.kernel.sglops``.

Reference: python/flashrec/kernel/sglops.py.  Each function keeps the
reference's name, arguments, return convention and in-place behaviour, but
runs a hand-written HIP kernel through the C ABI.  Unlike the reference there
is no CPU branch: CPU tensors raise (a silent torch fallback would hide a
missing or broken native library).
"""

from __future__ import annotations

from typing import NamedTuple, Optional

import torch

from flashrec_amd._lib import DTYPE_CODE, call, load, ptr, require_device, stream_of

_FP8_MAX = 448.0


_HALF = (torch.bfloat16, torch.float16)
# activation dtypes of the row kernels (rmsnorm, fused_add_rmsnorm,
# silu_and_mul and their fp8-quantizing forms): intermediates are rounded to
# the activation dtype, fp32 rows keep them in fp32
_ACT = (torch.bfloat16, torch.float16, torch.float32)


def _vec(weight: torch.Tensor, x: torch.Tensor) -> torch.Tensor:
    """The norm weight as a contiguous vector in the activations' dtype."""
    return weight.reshape(-1).to(device=x.device, dtype=x.dtype).contiguous()


def _rows(x: torch.Tensor, width: int) -> torch.Tensor:
    """[..., width] -> [rows, width] with unit inner stride (copy only if needed)."""
    x2 = x.reshape(-1, width)
    if x2.stride(-1) != 1 or (x2.shape[0] > 1 and x2.stride(0) < width):
        x2 = x2.contiguous()
    return x2


@torch.compiler.disable
def rmsnorm(x: torch.Tensor, weight: torch.Tensor, eps: float) -> torch.Tensor:
    """``(x * rsqrt(mean(x^2) + eps)) * weight`` per row (sglops.py:33-45)."""
    require_device(x)
    if x.dtype not in _ACT:
        raise TypeError(f"rmsnorm takes bf16/fp16/fp32 activations, got {x.dtype}")
    orig = x.shape
    hidden = int(weight.numel())
    x2 = _rows(x, hidden)
    w = _vec(weight, x)
    out = torch.empty(x2.shape, dtype=x.dtype, device=x.device)
    call("fr_rmsnorm", x2.data_ptr(), DTYPE_CODE[x.dtype], x2.stride(0), None, 0, w.data_ptr(), out.data_ptr(),
         out.stride(0), x2.shape[0], hidden, float(eps), stream_of(x))
    return out.view(orig)


@torch.compiler.disable
def fused_add_rmsnorm(
    x: torch.Tensor, residual: torch.Tensor, weight: torch.Tensor, eps: float
) -> tuple[torch.Tensor, torch.Tensor]:
    """``residual += x`` then RMSNorm(residual). Mutates both (sglops.py:48-61)."""
    require_device(x, residual)
    if x.dtype not in _ACT or residual.dtype != x.dtype:
        raise TypeError("fused_add_rmsnorm takes bf16, fp16 or fp32 x and a residual of the same dtype")
    hidden = int(weight.numel())
    x2 = x.reshape(-1, hidden).contiguous()
    r2 = residual.reshape(-1, hidden).contiguous()
    w = _vec(weight, x)
    call("fr_rmsnorm", x2.data_ptr(), DTYPE_CODE[x.dtype], x2.stride(0), r2.data_ptr(), r2.stride(0), w.data_ptr(),
         x2.data_ptr(), x2.stride(0), x2.shape[0], hidden, float(eps), stream_of(x))
    return x2.reshape(x.shape), r2.reshape(residual.shape)


@torch.compiler.disable
def apply_rope_inplace(
    positions: torch.Tensor,
    query: torch.Tensor,
    key: torch.Tensor,
    head_size: int,
    cos_sin_cache: torch.Tensor,
) -> bool:
    """NeoX RoPE of ``query`` [T, Hq*D] and ``key`` [T, Hk*D] in place (sglops.py:64-81).

    Returns True when the kernel ran; False for layouts it does not take
    (the reference returns False when its backend is absent).
    """
    require_device(query, key)
    d = int(head_size)
    t = int(positions.numel())
    if query.dtype != torch.bfloat16 or key.dtype != torch.bfloat16:
        return False
    if d <= 0 or d > 128 or d % 2 or int(cos_sin_cache.shape[-1]) != d:
        return False
    q3 = query.view(t, -1, d)
    k3 = key.view(t, -1, d)
    if q3.stride(-1) != 1 or k3.stride(-1) != 1:
        return False
    pos = positions.view(-1).to(dtype=torch.int64).contiguous()
    cs = cos_sin_cache.to(device=query.device, dtype=torch.float32).contiguous()
    call("fr_rope_inplace", q3.data_ptr(), q3.stride(0), q3.stride(1), k3.data_ptr(),
         k3.stride(0), k3.stride(1), pos.data_ptr(), cs.data_ptr(), cs.shape[0], t,
         q3.shape[1], k3.shape[1], d, stream_of(query))
    return True


def _heads(x: torch.Tensor, t: int, d: int) -> torch.Tensor:
    """[T, H*D] or [T, H, D] -> a [T, H, D] view (any strides)."""
    return x.unflatten(-1, (-1, d)) if x.dim() == 2 else x.reshape(t, -1, d)


@torch.compiler.disable
def rope_inplace_any(
    positions: torch.Tensor,
    query: torch.Tensor,
    key: torch.Tensor,
    head_size: int,
    cos_sin_cache: torch.Tensor,
) -> None:
    """NeoX RoPE in place for the layouts ``apply_rope_inplace`` declines
    (fp16 / fp32 heads, D > 128, strided head elements): the torch branch of
    ``RotaryEmbedding.forward`` (python/flashrec/layers/rotary.py:55-71),
    fp32 products and sums rounded once to the head's dtype."""
    require_device(query, key)
    d = int(head_size)
    if d <= 0 or d % 2 or int(cos_sin_cache.shape[-1]) != d:
        raise ValueError(f"RoPE needs an even head size matching the cos/sin cache, got {d}")
    if query.dtype not in _ACT or key.dtype != query.dtype:
        raise TypeError(f"RoPE takes bf16, fp16 or fp32 heads of one dtype, got {query.dtype} / {key.dtype}")
    t = int(positions.numel())
    q3, k3 = _heads(query, t, d), _heads(key, t, d)
    pos = positions.reshape(-1).to(dtype=torch.int64).contiguous()
    cs = cos_sin_cache.to(device=query.device, dtype=torch.float32).contiguous()
    call("fr_rope_inplace_any", q3.data_ptr(), q3.stride(0), q3.stride(1), q3.stride(2), k3.data_ptr(),
         k3.stride(0), k3.stride(1), k3.stride(2), DTYPE_CODE[query.dtype], pos.data_ptr(), cs.data_ptr(),
         cs.shape[0], t, q3.shape[1], k3.shape[1], d, stream_of(query))


@torch.compiler.disable
def per_token_quant_fp8(x: torch.Tensor) -> tuple[torch.Tensor, torch.Tensor]:
    """Per-row absmax e4m3 quant: ``(q [M,K] e4m3, scale [M,1] fp32)`` (sglops.py:84-96)."""
    require_device(x)
    if x.dtype not in (torch.bfloat16, torch.float16, torch.float32):
        raise TypeError(f"per_token_quant_fp8 takes bf16/fp16/fp32, got {x.dtype}")
    x2 = _rows(x, x.shape[-1])
    q = torch.empty(x2.shape, dtype=torch.float8_e4m3fn, device=x2.device)
    s = torch.empty((x2.shape[0], 1), dtype=torch.float32, device=x2.device)
    call("fr_per_token_quant_fp8", x2.data_ptr(), DTYPE_CODE[x2.dtype], x2.shape[0],
         x2.shape[1], x2.stride(0), q.data_ptr(), s.data_ptr(), stream_of(x2))
    return q, s


def _mfma_operands(a: torch.Tensor, b: torch.Tensor, m: int, n: int, k: int):
    """Operands the MFMA kernel takes: rows of a multiple of 16 bytes, 16-byte
    aligned, K a multiple of 16.  Anything else is repacked here, with K
    zero-padded (zeros add nothing to the products), instead of leaving it to
    the library's scalar fallback kernel (a per-output VALU loop)."""
    lda = a.stride(0) if m > 1 else k
    ldb = b.stride(1) if n > 1 else k
    ok = (k % 16 == 0 and lda % 16 == 0 and ldb % 16 == 0 and a.data_ptr() % 16 == 0
          and b.data_ptr() % 16 == 0)
    if ok or k == 0:
        return a, b, k
    k16 = (k + 15) // 16 * 16
    a16 = torch.zeros((m, k16), dtype=torch.uint8, device=a.device)
    a16[:, :k] = a.view(torch.uint8)
    b16 = torch.zeros((n, k16), dtype=torch.uint8, device=b.device)
    b16[:, :k] = b.t().view(torch.uint8)
    return a16.view(a.dtype), b16.view(b.dtype).t(), k16


@torch.compiler.disable
def fp8_scaled_mm(
    a_fp8: torch.Tensor,
    b_fp8: torch.Tensor,
    scale_a: torch.Tensor,
    scale_b: torch.Tensor,
    out_dtype: torch.dtype,
    bias: Optional[torch.Tensor] = None,
) -> torch.Tensor:
    """a: [M,K] fp8, b: [K,N] fp8 (column-major), scale_a: [M,1], scale_b: [N] (sglops.py:99-140)."""
    if a_fp8.dtype != torch.float8_e4m3fn or b_fp8.dtype != torch.float8_e4m3fn:
        raise TypeError("fp8_scaled_mm takes float8_e4m3fn operands")
    if out_dtype not in (torch.bfloat16, torch.float16, torch.float32):
        raise TypeError(f"unsupported out_dtype {out_dtype}")
    if a_fp8.dim() != 2 or b_fp8.dim() != 2 or a_fp8.shape[1] != b_fp8.shape[0]:
        raise ValueError(f"shape mismatch: a {tuple(a_fp8.shape)} b {tuple(b_fp8.shape)}")
    m, k = int(a_fp8.shape[0]), int(a_fp8.shape[1])
    n = int(b_fp8.shape[1])
    if bias is not None and bias.numel() != n:
        raise ValueError(f"bias has {bias.numel()} values, the output has {n} columns")
    require_device(a_fp8, b_fp8)
    a = a_fp8 if a_fp8.stride(1) == 1 and (m <= 1 or a_fp8.stride(0) >= k) else a_fp8.contiguous()
    b = b_fp8
    if not (b.stride(0) == 1 and (n <= 1 or b.stride(1) >= k)):
        b = b.t().contiguous().t()  # column-major copy
    a, b, k = _mfma_operands(a, b, m, n, k)
    sa = scale_a.reshape(-1).to(device=a.device, dtype=torch.float32).contiguous()
    sb = scale_b.reshape(-1).to(device=a.device, dtype=torch.float32).contiguous()
    if sa.numel() not in (1, m) or sb.numel() not in (1, n):
        raise ValueError("scale_a must have 1 or M values and scale_b 1 or N values")
    bias_t = None
    if bias is not None:
        bias_t = bias.reshape(-1).to(device=a.device, dtype=out_dtype).contiguous()
    out = torch.empty((m, n), dtype=out_dtype, device=a.device)
    lda = a.stride(0) if m > 1 else k
    ldb = b.stride(1) if n > 1 else k
    call("fr_fp8_scaled_mm", a.data_ptr(), lda, b.data_ptr(), ldb, sa.data_ptr(), sa.numel(),
         sb.data_ptr(), sb.numel(), ptr(bias_t), 0 if bias_t is None else n, out.data_ptr(), out.stride(0), m, n, k,
         DTYPE_CODE[out_dtype], stream_of(a))
    return out


@torch.compiler.disable
def fp8_scaled_mm_residual(
    a_fp8: torch.Tensor,
    b_fp8: torch.Tensor,
    scale_a: torch.Tensor,
    scale_b: torch.Tensor,
    residual: torch.Tensor,
    out: Optional[torch.Tensor] = None,
) -> torch.Tensor:
    """``residual + fp8_scaled_mm(a, b, scale_a, scale_b, residual.dtype)`` in
    one kernel, both roundings as the two steps (the product to the residual's
    dtype, then the sum; sglops.py:53-55).  ``out`` defaults to ``residual``
    itself (updated in place, as fused_add_rmsnorm updates it); returns it.
    residual: [M, N] bf16 or fp16 with a unit inner stride."""
    if a_fp8.dtype != torch.float8_e4m3fn or b_fp8.dtype != torch.float8_e4m3fn:
        raise TypeError("fp8_scaled_mm_residual takes float8_e4m3fn operands")
    if residual.dtype not in _HALF:
        raise TypeError(f"the residual must be bf16 or fp16, got {residual.dtype}")
    if a_fp8.dim() != 2 or b_fp8.dim() != 2 or a_fp8.shape[1] != b_fp8.shape[0]:
        raise ValueError(f"shape mismatch: a {tuple(a_fp8.shape)} b {tuple(b_fp8.shape)}")
    m, k = int(a_fp8.shape[0]), int(a_fp8.shape[1])
    n = int(b_fp8.shape[1])
    if residual.dim() != 2 or tuple(residual.shape) != (m, n) or residual.stride(1) != 1:
        raise ValueError(f"residual must be [{m}, {n}] with a unit inner stride, got {tuple(residual.shape)}")
    if out is None:
        out = residual
    if out.dtype != residual.dtype or tuple(out.shape) != (m, n) or out.stride(1) != 1:
        raise ValueError("out must match the residual's dtype and shape with a unit inner stride")
    if out.data_ptr() == residual.data_ptr() and out.stride(0) != residual.stride(0):
        raise ValueError("an aliased out must share the residual's row stride")
    require_device(a_fp8, b_fp8, residual, out)
    a = a_fp8 if a_fp8.stride(1) == 1 and (m <= 1 or a_fp8.stride(0) >= k) else a_fp8.contiguous()
    b = b_fp8
    if not (b.stride(0) == 1 and (n <= 1 or b.stride(1) >= k)):
        b = b.t().contiguous().t()
    a, b, k = _mfma_operands(a, b, m, n, k)
    sa = scale_a.reshape(-1).to(device=a.device, dtype=torch.float32).contiguous()
    sb = scale_b.reshape(-1).to(device=a.device, dtype=torch.float32).contiguous()
    if sa.numel() not in (1, m) or sb.numel() not in (1, n):
        raise ValueError("scale_a must have 1 or M values and scale_b 1 or N values")
    lda = a.stride(0) if m > 1 else k
    ldb = b.stride(1) if n > 1 else k
    ldr = residual.stride(0) if m > 1 else n
    ldo = out.stride(0) if m > 1 else n
    call("fr_fp8_scaled_mm_residual", a.data_ptr(), lda, b.data_ptr(), ldb, sa.data_ptr(), sa.numel(),
         sb.data_ptr(), sb.numel(), residual.data_ptr(), ldr, out.data_ptr(), ldo, m, n, k,
         DTYPE_CODE[residual.dtype], stream_of(a))
    return out


class PrearrangedFp8Weight(NamedTuple):
    """e4m3 weight codes of an ``[N, K]`` matrix rearranged once for
    ``fp8_scaled_mm_prearranged``: blocks of 32 rows x 64 bytes of K, each
    stored in the order a wave's MFMA operand registers hold it, so the GEMM
    loads weights as contiguous 1 KB runs straight into registers."""

    data: torch.Tensor  # uint8 [fr_fp8_weight_prearranged_bytes(N, K)]
    n: int
    k: int


def prearrange_fp8_weight(b_fp8: torch.Tensor) -> PrearrangedFp8Weight:
    """``b_fp8``: the ``[K, N]`` e4m3 weight of ``fp8_scaled_mm`` (any strides;
    ``Linear`` keeps it as the column-major view of ``[N, K]`` codes).  A new
    buffer; the codes are copied bit for bit."""
    if b_fp8.dtype != torch.float8_e4m3fn or b_fp8.dim() != 2:
        raise TypeError("prearrange_fp8_weight takes a 2-D float8_e4m3fn [K, N] weight")
    require_device(b_fp8)
    k, n = int(b_fp8.shape[0]), int(b_fp8.shape[1])
    rows = b_fp8.t()
    if not (rows.stride(1) == 1 and (n <= 1 or rows.stride(0) >= k)):
        rows = rows.contiguous()
    nbytes = int(load().fr_fp8_weight_prearranged_bytes(n, k))
    if nbytes < 0:
        raise ValueError(f"cannot prearrange a [{n}, {k}] weight")
    data = torch.empty(nbytes, dtype=torch.uint8, device=b_fp8.device)
    if nbytes:
        call("fr_fp8_weight_prearrange", rows.data_ptr(), rows.stride(0) if n > 1 else k, n, k, data.data_ptr(),
             stream_of(b_fp8))
    return PrearrangedFp8Weight(data, n, k)


@torch.compiler.disable
def fp8_scaled_mm_prearranged(
    a_fp8: torch.Tensor,
    w: PrearrangedFp8Weight,
    scale_a: torch.Tensor,
    scale_b: torch.Tensor,
    out_dtype: torch.dtype = torch.bfloat16,
    residual: Optional[torch.Tensor] = None,
    out: Optional[torch.Tensor] = None,
    silu: bool = False,
) -> torch.Tensor:
    """``fp8_scaled_mm(a, b, scale_a, scale_b, out_dtype)`` with ``b`` given
    as ``prearrange_fp8_weight(b)``: the same results bit for bit.  With
    ``residual`` the product (rounded to the residual's dtype) is added into
    it, as ``fp8_scaled_mm_residual`` (``out`` defaults to the residual);
    with ``silu`` the weight must be gate/up interleaved (``interleave_gate_up``)
    and the output is ``[M, N / 2]`` bf16, as ``fp8_scaled_mm_silu``."""
    if a_fp8.dtype != torch.float8_e4m3fn or a_fp8.dim() != 2:
        raise TypeError("fp8_scaled_mm_prearranged takes a 2-D float8_e4m3fn activation")
    m, k = int(a_fp8.shape[0]), int(a_fp8.shape[1])
    n = w.n
    if k != w.k:
        raise ValueError(f"activation K {k} does not match the weight's {w.k}")
    if silu:
        if residual is not None or n % 16:
            raise ValueError("the SiLU form takes no residual and N a multiple of 16")
        out_dtype = torch.bfloat16
    if residual is not None:
        if residual.dtype not in _HALF or tuple(residual.shape) != (m, n) or residual.stride(1) != 1:
            raise ValueError(f"residual must be bf16/fp16 [{m}, {n}] with a unit inner stride")
        out_dtype = residual.dtype
        if out is None:
            out = residual
    if out_dtype not in (torch.bfloat16, torch.float16, torch.float32):
        raise TypeError(f"unsupported out_dtype {out_dtype}")
    n_out = n // 2 if silu else n
    if out is None:
        out = torch.empty((m, n_out), dtype=out_dtype, device=a_fp8.device)
    if out.dtype != out_dtype or tuple(out.shape) != (m, n_out) or out.stride(1) != 1:
        raise ValueError(f"out must be {out_dtype} [{m}, {n_out}] with a unit inner stride")
    require_device(a_fp8, w.data, out)
    a = a_fp8 if a_fp8.stride(1) == 1 and (m <= 1 or a_fp8.stride(0) >= k) else a_fp8.contiguous()
    lda = a.stride(0) if m > 1 else k
    if k % 16 or lda % 16 or a.data_ptr() % 16:
        # the activation ring takes 16-byte rows: zero-pad K (the weight's
        # prearranged K steps already hold zeros there)
        k16 = (k + 15) // 16 * 16
        a16 = torch.zeros((m, k16), dtype=torch.uint8, device=a.device)
        a16[:, :k] = a.view(torch.uint8)
        a, k, lda = a16.view(a_fp8.dtype), k16, k16
    sa = scale_a.reshape(-1).to(device=a.device, dtype=torch.float32).contiguous()
    sb = scale_b.reshape(-1).to(device=a.device, dtype=torch.float32).contiguous()
    if sa.numel() not in (1, m) or sb.numel() not in (1, n):
        raise ValueError("scale_a must have 1 or M values and scale_b 1 or N values")
    ldr = 0 if residual is None else (residual.stride(0) if m > 1 else n)
    ldo = out.stride(0) if m > 1 else n_out
    call("fr_fp8_scaled_mm_prearranged", a.data_ptr(), lda, w.data.data_ptr(), sa.data_ptr(), sa.numel(),
         sb.data_ptr(), sb.numel(), ptr(residual), ldr, out.data_ptr(), ldo, m, n, k, DTYPE_CODE[out_dtype],
         int(silu), stream_of(a))
    return out


def interleave_gate_up(t: torch.Tensor, dim: int = 0) -> torch.Tensor:
    """The gate half then the up half of ``t`` along ``dim`` (2n entries, n a
    multiple of 8) reordered into chunks of 16: 8 gate entries followed by
    the 8 up entries of the same output columns, the order
    ``fp8_scaled_mm_silu`` takes its weight rows and scales in.  A copy."""
    size = int(t.shape[dim])
    if size % 16:
        raise ValueError(f"gate/up interleave needs a multiple of 16 rows, got {size}")
    shape = list(t.shape)
    split = shape[:dim] + [2, size // 16, 8] + shape[dim + 1:]
    return t.reshape(split).transpose(dim, dim + 1).reshape(shape).contiguous()


@torch.compiler.disable
def fp8_scaled_mm_silu(
    a_fp8: torch.Tensor,
    b_fp8: torch.Tensor,
    scale_a: torch.Tensor,
    scale_b: torch.Tensor,
    out: Optional[torch.Tensor] = None,
) -> torch.Tensor:
    """``silu_and_mul(fp8_scaled_mm(a, b, scale_a, scale_b, bf16))`` in one
    GEMM, for weights whose gate/up columns were put in the order of
    ``interleave_gate_up`` (``b`` ``[K, N]`` column-major and ``scale_b`` both
    interleaved).  Bit-for-bit the two steps on the un-interleaved weights
    (sglops.py:99-151): the product rounded to bf16, torch's silu in fp32
    rounded to bf16, the product with up rounded to bf16.  Returns (or writes
    into ``out``) ``[M, N / 2]`` bf16."""
    if a_fp8.dtype != torch.float8_e4m3fn or b_fp8.dtype != torch.float8_e4m3fn:
        raise TypeError("fp8_scaled_mm_silu takes float8_e4m3fn operands")
    if a_fp8.dim() != 2 or b_fp8.dim() != 2 or a_fp8.shape[1] != b_fp8.shape[0]:
        raise ValueError(f"shape mismatch: a {tuple(a_fp8.shape)} b {tuple(b_fp8.shape)}")
    m, k = int(a_fp8.shape[0]), int(a_fp8.shape[1])
    n = int(b_fp8.shape[1])
    if n % 16:
        raise ValueError(f"fp8_scaled_mm_silu needs N a multiple of 16, got {n}")
    require_device(a_fp8, b_fp8)
    if out is None:
        out = torch.empty((m, n // 2), dtype=torch.bfloat16, device=a_fp8.device)
    elif out.dtype != torch.bfloat16 or tuple(out.shape) != (m, n // 2) or out.stride(1) != 1:
        raise ValueError(f"out must be [{m}, {n // 2}] bf16 with a unit inner stride")
    require_device(out)
    if k == 0:  # an empty product: silu(0) * 0
        return out.zero_()
    a = a_fp8 if a_fp8.stride(1) == 1 and (m <= 1 or a_fp8.stride(0) >= k) else a_fp8.contiguous()
    b = b_fp8
    if not (b.stride(0) == 1 and (n <= 1 or b.stride(1) >= k)):
        b = b.t().contiguous().t()
    a, b, k = _mfma_operands(a, b, m, n, k)
    sa = scale_a.reshape(-1).to(device=a.device, dtype=torch.float32).contiguous()
    sb = scale_b.reshape(-1).to(device=a.device, dtype=torch.float32).contiguous()
    if sa.numel() not in (1, m) or sb.numel() not in (1, n):
        raise ValueError("scale_a must have 1 or M values and scale_b 1 or N values")
    lda = a.stride(0) if m > 1 else k
    ldb = b.stride(1) if n > 1 else k
    ldo = out.stride(0) if m > 1 else n // 2
    call("fr_fp8_scaled_mm_silu", a.data_ptr(), lda, b.data_ptr(), ldb, sa.data_ptr(), sa.numel(),
         sb.data_ptr(), sb.numel(), out.data_ptr(), ldo, m, n, k, stream_of(a))
    return out


@torch.compiler.disable
def silu_and_mul(x: torch.Tensor) -> torch.Tensor:
    """SwiGLU: ``silu(x[..., :d]) * x[..., d:]`` with ``d = last_dim // 2`` (sglops.py:143-151)."""
    require_device(x)
    if x.dtype not in _ACT:
        raise TypeError(f"silu_and_mul takes bf16/fp16/fp32, got {x.dtype}")
    last = int(x.shape[-1])
    if last % 2:
        raise ValueError("silu_and_mul needs an even last dimension")
    d = last // 2
    x2 = _rows(x, last)
    out = torch.empty((x2.shape[0], d), dtype=x.dtype, device=x.device)
    call("fr_silu_and_mul", x2.data_ptr(), DTYPE_CODE[x.dtype], x2.stride(0), out.data_ptr(), out.stride(0),
         x2.shape[0], d, stream_of(x))
    return out.view(*x.shape[:-1], d)


@torch.compiler.disable
def apply_rope_and_store_kv(
    positions: torch.Tensor,
    query: torch.Tensor,
    key: torch.Tensor,
    value: torch.Tensor,
    loc: torch.Tensor,
    k_cache: torch.Tensor,
    v_cache: torch.Tensor,
    head_size: int,
    cos_sin_cache: torch.Tensor,
) -> bool:
    """RoPE of ``query`` / ``key`` in place, then ``k_cache[loc] = key``,
    ``v_cache[loc] = value``, in one kernel (sglops.py:154-204).

    As in the reference this is the matching-dtype path: it returns False
    when a cache's dtype differs from the activations' (an fp8 pool goes
    through ``fused_qk_norm_rope_store_fp8`` or ``TokenToKVPool.store``), and
    for layouts the kernel does not take (head dim > 128 or odd, non-unit
    inner strides, a cache whose rows are not ``[H_kv, head_size]``).
    """
    require_device(query, key, value, k_cache, v_cache)
    if key.dtype != k_cache.dtype or value.dtype != v_cache.dtype:
        return False
    if not (query.dtype == key.dtype == value.dtype == torch.bfloat16):
        return False
    d = int(head_size)
    t = int(positions.numel())
    if d <= 0 or d > 128 or d % 2 or int(cos_sin_cache.shape[-1]) != d:
        return False
    q3 = query.view(t, -1, d)
    k3 = key.view(t, -1, d)
    v3 = value.view(t, -1, d)
    hk = int(k3.shape[1])
    if int(v3.shape[1]) != hk or q3.stride(-1) != 1 or k3.stride(-1) != 1 or v3.stride(-1) != 1:
        return False
    slots = int(k_cache.shape[0])
    if k_cache.numel() != slots * hk * d or v_cache.shape != k_cache.shape:
        return False
    kc = k_cache.view(slots, hk, d)
    vc = v_cache.view(slots, hk, d)
    if kc.stride(-1) != 1 or vc.stride(-1) != 1:
        return False
    pos = positions.reshape(-1).to(dtype=torch.int64).contiguous()
    loc64 = loc.reshape(-1).to(dtype=torch.int64).contiguous()
    if int(loc64.numel()) != t:
        raise ValueError(f"loc has {loc64.numel()} slots for {t} tokens")
    cs = cos_sin_cache.to(device=query.device, dtype=torch.float32).contiguous()
    call("fr_rope_store_kv_bf16", q3.data_ptr(), q3.stride(0), q3.stride(1), k3.data_ptr(),
         k3.stride(0), k3.stride(1), v3.data_ptr(), v3.stride(0), v3.stride(1), pos.data_ptr(),
         loc64.data_ptr(), cs.data_ptr(), cs.shape[0], kc.data_ptr(), kc.stride(0), kc.stride(1),
         vc.data_ptr(), vc.stride(0), vc.stride(1), slots, t, q3.shape[1], hk, d, stream_of(query))
    return True


@torch.compiler.disable
def store_kv_cache(
    k_cache: torch.Tensor,
    v_cache: torch.Tensor,
    loc: torch.Tensor,
    k: torch.Tensor,
    v: torch.Tensor,
) -> None:
    """``k_cache[loc] = k; v_cache[loc] = v`` on rows of width row_dim (sglops.py:207-222).

    e4m3 caches take e4m3 k/v (copied) or bf16 k/v (converted with torch's
    ``.to(float8_e4m3fn)`` rounding); bf16 caches take bf16 k/v.  Slots
    outside ``[0, slots)`` are skipped instead of raising an IndexError.
    """
    require_device(k_cache, v_cache, k, v)
    if k_cache.dtype != v_cache.dtype or k_cache.dtype not in (torch.float8_e4m3fn, torch.bfloat16):
        raise TypeError("store_kv_cache writes float8_e4m3fn or bfloat16 caches")
    slots = int(k_cache.shape[0])
    row_dim = int(k_cache[0].numel()) if slots else int(k.shape[-1])
    kc = k_cache.view(slots, row_dim)
    vc = v_cache.view(slots, row_dim)
    loc64 = loc.view(-1).to(dtype=torch.int64).contiguous()
    n = int(loc64.numel())
    k2 = k.reshape(n, row_dim)
    v2 = v.reshape(n, row_dim)
    if k2.stride(-1) != 1:
        k2 = k2.contiguous()
    if v2.stride(-1) != 1:
        v2 = v2.contiguous()
    if k_cache.dtype == torch.bfloat16:
        if k2.dtype != torch.bfloat16 or v2.dtype != torch.bfloat16:
            raise TypeError("a bf16 cache takes bf16 k/v")
        call("fr_store_kv_bf16", k2.data_ptr(), k2.stride(0), v2.data_ptr(), v2.stride(0),
             loc64.data_ptr(), kc.data_ptr(), kc.stride(0), vc.data_ptr(), vc.stride(0), slots, n,
             row_dim, stream_of(k_cache))
        return
    if k2.dtype != v2.dtype or k2.dtype not in (torch.bfloat16, torch.float8_e4m3fn):
        raise TypeError("k/v must both be bf16 or both float8_e4m3fn")
    call("fr_store_kv_fp8", k2.data_ptr(), k2.stride(0), v2.data_ptr(), v2.stride(0),
         DTYPE_CODE[k2.dtype], loc64.data_ptr(), kc.data_ptr(), kc.stride(0), vc.data_ptr(),
         vc.stride(0), slots, n, row_dim, stream_of(k_cache))


@torch.compiler.disable
def log_softmax_f32(logits: torch.Tensor, out: Optional[torch.Tensor] = None) -> torch.Tensor:
    """Row-wise ``log_softmax`` of fp32 logits (the tail of logits.py:118-120).

    ``out`` (default: a new tensor) may be ``logits`` itself; it must be fp32
    of the logits' shape and device with unit inner stride."""
    if logits.dtype != torch.float32 or logits.dim() != 2 or logits.stride(1) != 1:
        raise TypeError("log_softmax_f32 takes 2-D fp32 logits with unit inner stride")
    if out is not None and (out.dtype != torch.float32 or tuple(out.shape) != tuple(logits.shape)
                            or out.stride(1) != 1 or out.device != logits.device):
        raise ValueError("log_softmax_f32: out must be fp32 on the logits' device, of the logits' "
                         f"shape {tuple(logits.shape)}, with unit inner stride")
    require_device(logits)
    if out is None:
        out = torch.empty_like(logits)
    call("fr_log_softmax_f32", logits.data_ptr(), logits.stride(0), out.data_ptr(),
         out.stride(0), logits.shape[0], logits.shape[1], stream_of(logits))
    return out


__all__ = [
    "rmsnorm",
    "fused_add_rmsnorm",
    "apply_rope_inplace",
    "rope_inplace_any",
    "per_token_quant_fp8",
    "fp8_scaled_mm",
    "fp8_scaled_mm_silu",
    "prearrange_fp8_weight",
    "fp8_scaled_mm_prearranged",
    "PrearrangedFp8Weight",
    "interleave_gate_up",
    "silu_and_mul",
    "apply_rope_and_store_kv",
    "store_kv_cache",
    "log_softmax_f32",
]
