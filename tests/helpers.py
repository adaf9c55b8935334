"""Comparison helpers shared by the parity tests."""

from __future__ import annotations

import torch


def codes(t: torch.Tensor) -> torch.Tensor:
    """e4m3 tensor -> int16 codes on the CPU."""
    return t.detach().cpu().contiguous().view(torch.uint8).to(torch.int16)


def code_flip_stats(q_got: torch.Tensor, q_ref: torch.Tensor):
    """(fraction of differing codes, max distance between differing codes of the same sign)."""
    a, b = codes(q_got), codes(q_ref)
    diff = a != b
    frac = diff.float().mean().item()
    if not diff.any():
        return 0.0, 0
    same_sign = ((a ^ b) & 0x80) == 0
    dist = torch.where(diff & same_sign, (a - b).abs(), torch.full_like(a, 255))
    # zero may be encoded with either sign when the value rounds to 0
    zero_pair = diff & ((a & 0x7F) == 0) & ((b & 0x7F) <= 1) | diff & ((b & 0x7F) == 0) & ((a & 0x7F) <= 1)
    dist = torch.where(zero_pair, torch.ones_like(dist), dist)
    return frac, int(dist[diff].max().item())


def assert_fp8_parity(q_got, s_got, q_ref, s_ref, max_flip_frac=1e-3, label=""):
    """The bar for quantised outputs whose pre-quant value is summed or passed
    through exp in a different order than torch's CPU: codes and scales
    bit-exact except <= 1-ULP flips on < 0.1% of elements (codes) and of rows
    (scales).  Prints the flip counts; returns (code flips, scale flips)."""
    s_got = s_got.detach().cpu().float().reshape(-1)
    s_ref = s_ref.detach().cpu().float().reshape(-1)
    sdiff = s_got != s_ref
    n_sflip = int(sdiff.sum().item())
    if n_sflip:
        rel = ((s_got - s_ref).abs() / s_ref.abs().clamp(min=1e-30))[sdiff]
        # amax is a 16-bit float value: a flip moves it by one ULP (<= 2^-7 relative)
        assert rel.max().item() <= 2.0 ** -7, f"scale off by {rel.max().item()}"
    frac, dist = code_flip_stats(q_got, q_ref)
    n_codes = q_ref.numel()
    n_cflip = int(round(frac * n_codes))
    print(f"parity{(' ' + label) if label else ''}: {n_cflip}/{n_codes} codes flipped, "
          f"{n_sflip}/{s_ref.numel()} scales changed")
    assert n_sflip < max_flip_frac * s_ref.numel() or n_sflip == 0, \
        f"{n_sflip} of {s_ref.numel()} rows changed scale (bar: < {max_flip_frac:.1%})"
    assert dist <= 1, f"codes differ by {dist} ULP"
    assert frac < max_flip_frac, f"{frac:.2e} of codes flipped"
    return n_cflip, n_sflip


def assert_bf16_parity(got, ref, max_flip_frac=1e-3):
    """bf16 outputs: bit-exact except 1-ULP flips on < 0.1% of elements."""
    a = got.detach().cpu().contiguous().view(torch.int16).to(torch.int32)
    b = ref.detach().cpu().contiguous().view(torch.int16).to(torch.int32)
    diff = a != b
    if not diff.any():
        return
    dist = (a - b).abs()[diff].max().item()
    frac = diff.float().mean().item()
    assert dist <= 1, f"bf16 values differ by {dist} ULP"
    assert frac < max_flip_frac, f"{frac:.2e} of bf16 values flipped"


def max_abs_rel(got: torch.Tensor, ref: torch.Tensor) -> float:
    """max |got - ref| / max |ref|  (the GEMM acceptance metric)."""
    got = got.detach().cpu().float()
    ref = ref.detach().cpu().float()
    return ((got - ref).abs().max() / ref.abs().max().clamp(min=1e-30)).item()


def assert_rope_parity(got, ref, n_ref, max_flip_frac=1e-3):
    """Rotated heads (bf16 q, or decoded e4m3 K pages via ``decoded=True``
    callers): bit-exact except where the per-head RMS normalisation flipped
    one bf16 ULP (different fp32 summation order than torch's CPU).  Such a
    flip moves an input of the rotation by <= 2^-8 |n|, so each output of the
    pair (n_i, n_partner) may move by <= 2^-7 (|n_i| + |n_partner|)."""
    got = got.detach().cpu().float()
    ref = ref.detach().cpu().float()
    n = n_ref.detach().cpu().float()
    half = n.shape[-1] // 2
    partner = torch.cat([n[..., half:], n[..., :half]], dim=-1)
    bound = 2.0 ** -7 * (n.abs() + partner.abs())
    diff = got != ref
    frac = diff.float().mean().item()
    assert frac < max_flip_frac, f"{frac:.2e} of rotated values differ"
    if diff.any():
        excess = ((got - ref).abs() - bound)[diff].max().item()
        assert excess <= 0, f"rotated value off by {excess} beyond the one-ULP-norm-flip bound"
