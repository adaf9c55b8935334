"""The W8A8 GEMM with SiLU-and-mul in its epilogue
(``fp8_scaled_mm_silu`` -> ``fr_fp8_scaled_mm_silu``), the MLP's gate_up
projection and the SiLU-and-mul half of silu_and_mul_per_token_quant_fp8.

Bars:
* bit-exact against the two steps it replaces on the un-interleaved weights:
  ``fp8_scaled_mm`` to bf16 (held to the fp32 dequantised oracle in
  test_gpu_gemm.py) then ``silu_and_mul`` (held to torch's CPU silu in
  test_gpu_quant.py);
* against the oracle composition (torch CPU silu on the GPU's bf16 gate_up
  output): bit-exact but for 1-ULP flips on < 0.1 % of values, also with
  gates far outside [-80, 80] (the epilogue's exact-formula branch);
* the full chain (epilogue + per-token quant) against the oracle's
  silu_and_mul_per_token_quant_fp8 of the GPU's gate_up output, at the fp8
  parity bar.
Shapes: the decode step's gate_up (256 x 256 tile), M = 512 (256 x 128),
small N (128 x 128), ragged M and N (the bounds-checked path), M = 1, K not
a multiple of 16 (operands repacked by the wrapper), and several tiles per
workgroup on the 256 x 128 and 128 x 128 tiles."""

import pytest
import torch

from helpers import assert_bf16_parity, assert_fp8_parity
from oracle import ops

pytestmark = pytest.mark.gpu


def _operands(m, n, k, seed, x_scale=1.0):
    g = torch.Generator().manual_seed(seed)
    x = (torch.randn(m, k, generator=g) * x_scale).to(torch.bfloat16)
    w = (0.02 * torch.randn(n, k, generator=g)).to(torch.bfloat16)
    qa, sa = ops.per_token_quant_fp8(x)
    qw, sw = ops.quantize_weight_fp8(w)
    return qa, sa, qw, sw


def _fused(dev, qa, sa, qw, sw, out=None):
    from flashrec_amd.kernel.sglops import fp8_scaled_mm_silu, interleave_gate_up

    qwi = interleave_gate_up(qw.to(dev))
    swi = interleave_gate_up(sw.to(dev))
    return fp8_scaled_mm_silu(qa.to(dev), qwi.t(), sa.to(dev), swi, out)


def _gate_up(dev, qa, sa, qw, sw):
    from flashrec_amd.kernel.sglops import fp8_scaled_mm

    return fp8_scaled_mm(qa.to(dev), qw.to(dev).t(), sa.to(dev), sw.to(dev), torch.bfloat16)


def _assert_same(got, ref, label=""):
    g = got.contiguous().view(torch.int16).cpu()
    r = ref.contiguous().view(torch.int16).cpu()
    bad = (g != r).nonzero()
    if bad.numel():
        idx = [tuple(int(v) for v in bad[i]) for i in range(min(5, bad.shape[0]))]
        gf, rf = got.float().cpu(), ref.float().cpu()
        raise AssertionError(f"{label}: {bad.shape[0]} of {g.numel()} differ, e.g. "
                             f"{[(i, float(gf[i]), float(rf[i])) for i in idx]}")


@pytest.mark.parametrize("m,n,k", [(4096, 12288, 2048), (512, 12288, 2048), (256, 2048, 1024),
                                   (300, 1040, 384), (4096 + 100, 2048 + 64, 2048), (33, 96, 256),
                                   (1, 256, 2048), (64, 512, 1000), (2624, 6144, 2048), (3648, 2112, 1024)])
def test_silu_epilogue_matches_two_steps(dev, m, n, k):
    from flashrec_amd.kernel.sglops import silu_and_mul

    qa, sa, qw, sw = _operands(m, n, k, seed=m + n + k)
    gu = _gate_up(dev, qa, sa, qw, sw)
    ref = silu_and_mul(gu)
    got = _fused(dev, qa, sa, qw, sw)
    assert got.shape == (m, n // 2) and got.dtype == torch.bfloat16
    _assert_same(got, ref, f"{m}x{n}x{k}")
    # and against torch's CPU silu on the same bf16 gate_up output
    assert_bf16_parity(got, ops.silu_and_mul(gu.cpu()))


def test_silu_epilogue_wide_gates(dev):
    """Gates up to several hundred (and below -88, where exp(-g) overflows):
    the epilogue's torch-formula branch, checked against torch's CPU silu."""
    qa, sa, qw, sw = _operands(512, 2048, 2048, seed=7, x_scale=300.0)
    gu = _gate_up(dev, qa, sa, qw, sw)
    g = gu[:, :1024].float()
    assert (g.abs() > 80).float().mean().item() > 0.3 and (g < -88).any()
    got = _fused(dev, qa, sa, qw, sw)
    assert_bf16_parity(got, ops.silu_and_mul(gu.cpu()))


def test_silu_epilogue_into_strided_out(dev):
    """``out`` a column slice of a wider buffer: the columns around it are untouched."""
    qa, sa, qw, sw = _operands(384, 1024, 512, seed=3)
    buf = torch.full((384, 1024), 7.0, dtype=torch.bfloat16, device=dev)
    got = _fused(dev, qa, sa, qw, sw, out=buf[:, 256:768])
    ref = _fused(dev, qa, sa, qw, sw)
    _assert_same(got, ref, "strided out")
    assert (buf[:, :256] == 7.0).all() and (buf[:, 768:] == 7.0).all()


def test_silu_chain_matches_oracle_quant(dev):
    """Epilogue + per-token quant = silu_and_mul_per_token_quant_fp8 of the
    gate_up output (the decode step's MLP middle), at the decode shape."""
    from flashrec_amd.kernel.sglops import per_token_quant_fp8

    qa, sa, qw, sw = _operands(4096, 12288, 2048, seed=11)
    gu = _gate_up(dev, qa, sa, qw, sw).cpu()
    q, s = per_token_quant_fp8(_fused(dev, qa, sa, qw, sw))
    q_ref, s_ref = ops.silu_and_mul_per_token_quant_fp8(gu)
    assert_fp8_parity(q, s, q_ref, s_ref, label="gate_up silu epilogue + quant")


def test_linear_forward_fp8_silu(dev):
    """Linear.forward_fp8_silu (interleaved copy built on first use) equals
    forward_fp8 then silu_and_mul; a reload drops the interleaved copy."""
    from flashrec_amd.kernel.sglops import per_token_quant_fp8, silu_and_mul
    from flashrec_amd.layers.linear import Linear

    g = torch.Generator(device=dev).manual_seed(2)
    lin = Linear(1024, 2 * 768)
    lin.load((0.02 * torch.randn(1536, 1024, generator=g, device=dev)).to(torch.bfloat16), quantize_fp8=True)
    x = torch.randn(200, 1024, generator=g, device=dev).to(torch.bfloat16)
    q, s = per_token_quant_fp8(x)
    ref = silu_and_mul(lin.forward_fp8(q, s, (200, 1024), torch.bfloat16))
    _assert_same(lin.forward_fp8_silu(q, s), ref, "Linear")
    lin.load((0.02 * torch.randn(1536, 1024, generator=g, device=dev)).to(torch.bfloat16), quantize_fp8=True)
    ref2 = silu_and_mul(lin.forward_fp8(q, s, (200, 1024), torch.bfloat16))
    _assert_same(lin.forward_fp8_silu(q, s), ref2, "Linear after reload")

