"""Torch-CPU restatement of the reference's CPU arithmetic for the FP8 path.

TEST INFRASTRUCTURE ONLY (see ``oracle/__init__.py``).  Every function states
the reference file:line whose CPU behaviour it restates; all inputs and
outputs are CPU tensors.  The HIP kernels are required to match these
bit-for-bit (codes, scales, bf16 outputs, slot layout), except for the
documented rounding-boundary flips caused by a different fp32 summation order
(RMS variance) or exp implementation (SiLU), and the GEMM, which is checked
against ``fp8_scaled_mm`` below (an fp32 matmul of dequantised operands) to a
max-abs-normalised relative tolerance.
"""

from __future__ import annotations

from typing import Optional

import torch
import torch.nn.functional as F

FP8_MAX = 448.0
E4M3 = torch.float8_e4m3fn


# --------------------------------------------------------------- quantisation
def per_token_quant_fp8(x: torch.Tensor) -> tuple[torch.Tensor, torch.Tensor]:
    """python/flashrec/kernel/sglops.py:86, :92-96 (CPU branch)."""
    x2 = x.reshape(-1, x.shape[-1]).contiguous()
    x_f = x2.float()
    amax = x_f.abs().amax(dim=-1, keepdim=True).clamp(min=1e-12)
    scale = (amax / FP8_MAX).to(dtype=torch.float32)
    q = (x_f / scale).clamp(-FP8_MAX, FP8_MAX).to(E4M3)
    return q, scale


def quantize_weight_fp8(weight: torch.Tensor) -> tuple[torch.Tensor, torch.Tensor]:
    """python/flashrec/layers/linear.py:26-32."""
    w = weight.float()
    amax = w.abs().amax(dim=-1).clamp(min=1e-12)
    scale = (amax / FP8_MAX).to(dtype=torch.float32)
    q = (w / scale.unsqueeze(-1)).clamp(-FP8_MAX, FP8_MAX).to(E4M3)
    return q, scale


# --------------------------------------------------------------- norms / act
def rmsnorm(x: torch.Tensor, weight: torch.Tensor, eps: float) -> torch.Tensor:
    """python/flashrec/kernel/sglops.py:35-39 (CPU branch)."""
    x_f = x.float()
    var = x_f.pow(2).mean(dim=-1, keepdim=True)
    y = x_f * torch.rsqrt(var + eps)
    return (y * weight.float()).to(x.dtype)


def fused_add_rmsnorm(
    x: torch.Tensor, residual: torch.Tensor, weight: torch.Tensor, eps: float
) -> tuple[torch.Tensor, torch.Tensor]:
    """python/flashrec/kernel/sglops.py:53-55 (CPU branch): bf16 add, then rmsnorm."""
    residual = residual + x
    return rmsnorm(residual, weight, eps), residual


def silu_and_mul(x: torch.Tensor) -> torch.Tensor:
    """python/flashrec/kernel/sglops.py:146, :151 (CPU branch)."""
    d = int(x.shape[-1]) // 2
    return F.silu(x[..., :d]) * x[..., d:]


def rmsnorm_per_token_quant_fp8(x, weight, eps):
    """python/flashrec/kernel/rms_fp8.py:128-130 (fallback composition)."""
    return per_token_quant_fp8(rmsnorm(x, weight, eps))


def fused_add_rmsnorm_per_token_quant_fp8(x, residual, weight, eps):
    """python/flashrec/kernel/rms_fp8.py:141-145 (fallback composition)."""
    hidden, residual = fused_add_rmsnorm(x, residual, weight, eps)
    q, scale = per_token_quant_fp8(hidden)
    return q, scale, residual


def silu_and_mul_per_token_quant_fp8(x):
    """python/flashrec/kernel/silu_fp8.py:79-82 (fallback composition)."""
    return per_token_quant_fp8(silu_and_mul(x))


# --------------------------------------------------------------- GEMM
def fp8_scaled_mm(
    a_fp8: torch.Tensor,
    b_fp8: torch.Tensor,
    scale_a: torch.Tensor,
    scale_b: torch.Tensor,
    out_dtype: torch.dtype = torch.bfloat16,
    bias: Optional[torch.Tensor] = None,
) -> torch.Tensor:
    """W8A8 reference product: fp32 matmul of dequantised operands.

    This is the acceptance oracle for python/flashrec/kernel/sglops.py:99-140:
    a [M,K] e4m3, b [K,N] e4m3, scale_a [M,1] (or 1), scale_b [N] (or 1).
    Returned in fp32 (callers round to ``out_dtype`` when comparing storage).
    """
    a = a_fp8.float() * scale_a.reshape(-1, 1).float()
    b = b_fp8.float() * scale_b.reshape(1, -1).float()
    out = a @ b
    if bias is not None:
        out = out + bias.float()
    return out


def fp8_scaled_mm_torch_cpu(a_fp8, b_fp8, scale_a, scale_b, out_dtype, bias=None):
    """The reference's literal CPU branch (sglops.py:111-139): ``torch._scaled_mm``
    in bf16 with unit scales, then the per-row/per-channel rescale in fp32 and
    a second bf16 rounding.  Kept to show the acceptance oracle above agrees
    with it to bf16 precision."""
    one = torch.ones(1, dtype=torch.float32)
    out = torch._scaled_mm(
        a_fp8,
        b_fp8,
        scale_a=scale_a.flatten()[:1] if scale_a.numel() == 1 else one,
        scale_b=scale_b.flatten()[:1] if scale_b.numel() == 1 else one,
        out_dtype=out_dtype,
        use_fast_accum=True,
    )
    if isinstance(out, tuple):
        out = out[0]
    if scale_a.numel() > 1 or scale_b.numel() > 1:
        out = out.float() * scale_a.float() * scale_b.view(1, -1).float()
        out = out.to(out_dtype)
        if bias is not None:
            out = out + bias.to(dtype=out_dtype)
    elif bias is not None:
        out = out + bias.to(dtype=out.dtype)
    return out


# --------------------------------------------------------------- RoPE / KV
def cos_sin_cache(head_dim: int, max_position: int, base: float) -> torch.Tensor:
    """python/flashrec/layers/rotary.py:21-34: [max_pos, D] fp32, cos half then sin half."""
    inv_freq = 1.0 / (base ** (torch.arange(0, head_dim, 2, dtype=torch.float32) / head_dim))
    t = torch.arange(max_position, dtype=torch.float32)
    freqs = torch.einsum("i,j->ij", t, inv_freq)
    return torch.cat((freqs.cos(), freqs.sin()), dim=-1)


def _rotate_half(x: torch.Tensor) -> torch.Tensor:
    """python/flashrec/layers/rotary.py:11-14."""
    x1 = x[..., : x.shape[-1] // 2]
    x2 = x[..., x.shape[-1] // 2 :]
    return torch.cat((-x2, x1), dim=-1)


def apply_rope(positions: torch.Tensor, x: torch.Tensor, cache: torch.Tensor) -> torch.Tensor:
    """NeoX rotate-half RoPE of bf16 ``x`` [T, H, D]; bf16 result.

    Restates python/flashrec/layers/rotary.py:69-71 (``x*cos + rotate_half(x)*sin``
    in fp32, then ``.to(x.dtype)``).  The reference's torch branch
    (rotary.py:55-58) takes ``cos, sin = cache.chunk(2)`` of width D/2 and
    multiplies them into the width-D head directly, which does not broadcast
    for D > 2; the cos/sin halves are therefore repeated over both halves of
    the head here, which is the NeoX formula the reference's GPU backends
    (sgl-kernel, FlashInfer, and its own Triton kernel at
    python/flashrec/kernel/qk_rope_kv.py:185-186, :216-217) evaluate.
    """
    c = cache[positions.long()]
    cos, sin = c.chunk(2, dim=-1)
    cos = torch.cat((cos, cos), dim=-1).unsqueeze(1)
    sin = torch.cat((sin, sin), dim=-1).unsqueeze(1)
    return ((x * cos) + (_rotate_half(x) * sin)).to(x.dtype)


def store_kv(k_cache, v_cache, loc, k, v) -> None:
    """python/flashrec/kvcache/pool.py:124-139 + sglops.py:221-222 (CPU branch).

    k/v [n, H, D] are converted to the cache dtype, then ``cache[loc] = rows``.
    """
    loc = loc.view(-1).to(dtype=torch.int64)
    n = int(loc.numel())
    if n == 0:
        return
    h, d = int(k_cache.shape[1]), int(k_cache.shape[2])
    k = k.reshape(n, h, d).to(k_cache.dtype)
    v = v.reshape(n, h, d).to(v_cache.dtype)
    k_cache.view(-1, h * d)[loc] = k.reshape(n, h * d)
    v_cache.view(-1, h * d)[loc] = v.reshape(n, h * d)


def qk_norm_rope_store_fp8(q, k, v, positions, loc, q_weight, k_weight, eps, cache, k_cache,
                           v_cache) -> torch.Tensor:
    """The unfused sequence of python/flashrec/models/qwen3.py:108-128 that
    python/flashrec/kernel/qk_rope_kv.py:164-250 replaces: per-head RMSNorm
    (bf16), rotate-half RoPE (bf16), e4m3 store of K and V at ``loc``.
    Mutates the caches; returns the rotated q (bf16, same shape as q)."""
    qn = rmsnorm(q, q_weight, eps)
    kn = rmsnorm(k, k_weight, eps)
    qr = apply_rope(positions, qn, cache)
    kr = apply_rope(positions, kn, cache)
    store_kv(k_cache, v_cache, loc, kr, v)
    return qr


# --------------------------------------------------------------- lm head
def restricted_logprobs_fp8(hidden: torch.Tensor, weight: torch.Tensor) -> torch.Tensor:
    """SID-restricted lm_head with the north star's fp8 upgrade of
    python/flashrec/logits.py:118-120: quantise the weight slice per channel
    and the hidden rows per token, fp32 product of the dequantised operands,
    fp32 log_softmax."""
    qw, sw = quantize_weight_fp8(weight)
    qa, sa = per_token_quant_fp8(hidden)
    logits = fp8_scaled_mm(qa, qw.t(), sa, sw)
    return F.log_softmax(logits, dim=-1)


# --------------------------------------------------------------- attention
def paged_attention(q: torch.Tensor, k_cache: torch.Tensor, v_cache: torch.Tensor,
                    kv_indices: torch.Tensor, kv_start: torch.Tensor, kv_len: torch.Tensor,
                    scale: float) -> torch.Tensor:
    """python/flashrec/attention/flashinfer.py:380-431 (_sdpa), per query token.

    Token t gathers rows kv_indices[kv_start[t]:kv_start[t]+kv_len[t]] of the
    e4m3 caches (cast exactly, as ``k_all.to(q.dtype)`` at :386-389 is exact
    for e4m3), repeats kv heads for grouped queries (:33-37, :406-407) and
    takes softmax(q k^T * scale) v — here in fp32, rounded to bf16 once (the
    reference's bf16 SDPA rounds its probabilities to bf16 on the way, so the
    two differ by bf16 rounding only).  No visible slot: zeros.
    """
    T, Hq, D = q.shape
    Hk = k_cache.shape[1]
    rep = Hq // Hk
    out = torch.zeros(T, Hq, D, dtype=torch.float32)
    kf = k_cache.float()
    vf = v_cache.float()
    for t in range(T):
        n = int(kv_len[t])
        if n == 0:
            continue
        s0 = int(kv_start[t])
        idx = kv_indices[s0:s0 + n].long()
        k = kf[idx].repeat_interleave(rep, dim=1)  # [n, Hq, D]
        v = vf[idx].repeat_interleave(rep, dim=1)
        qt = q[t].float()  # [Hq, D]
        sc = torch.einsum("hd,nhd->hn", qt, k) * scale
        p = torch.softmax(sc, dim=-1)
        out[t] = torch.einsum("hn,nhd->hd", p, v)
    return out.to(torch.bfloat16)


def sdpa_reference_style(q: torch.Tensor, k_cache: torch.Tensor, v_cache: torch.Tensor,
                         kv_indices: torch.Tensor, kv_indptr: torch.Tensor) -> torch.Tensor:
    """The decode branch of flashinfer.py:380-431 as its own sequence of torch
    calls (gather, cast to bf16, NHD -> BHSD permute, repeat_kv,
    F.scaled_dot_product_attention with scale D^-0.5), one query per row."""
    rows, Hq, D = q.shape
    Hk = k_cache.shape[1]
    rep = Hq // Hk
    k_all = k_cache.to(q.dtype)
    v_all = v_cache.to(q.dtype)
    outs = []
    for i in range(rows):
        idx = kv_indices[int(kv_indptr[i]):int(kv_indptr[i + 1])].long()
        k_t = k_all[idx].permute(1, 0, 2).unsqueeze(0)
        v_t = v_all[idx].permute(1, 0, 2).unsqueeze(0)
        q_t = q[i:i + 1].permute(1, 0, 2).unsqueeze(0)
        b, h, s, d = k_t.shape
        k_t = k_t[:, :, None].expand(b, h, rep, s, d).reshape(b, h * rep, s, d)
        v_t = v_t[:, :, None].expand(b, h, rep, s, d).reshape(b, h * rep, s, d)
        attn = F.scaled_dot_product_attention(q_t, k_t, v_t, scale=D ** -0.5)
        outs.append(attn.squeeze(0).permute(1, 0, 2))
    return torch.cat(outs, dim=0)
