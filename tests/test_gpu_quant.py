"""Parity of the HIP row kernels (quant, RMSNorm, SiLU) with the CPU oracle.

Inputs are generated on the CPU, the same tensors are copied to the GPU, and
outputs are compared with ``oracle.ops`` (the reference's CPU arithmetic).
"""

import pytest
import torch

from helpers import assert_bf16_parity, assert_fp8_parity, code_flip_stats, codes
from oracle import inputs, ops

pytestmark = pytest.mark.gpu


def _bf16(shape, seed, scale=1.0, outliers=0):
    g = torch.Generator().manual_seed(seed)
    x = torch.randn(*shape, generator=g) * scale
    if outliers:
        cols = torch.randperm(shape[-1], generator=g)[:outliers]
        x[..., cols] *= 20.0
    return x.to(torch.bfloat16)


def test_e4m3_conversion_all_bf16_patterns(dev):
    """Every bf16 bit pattern through the KV-store conversion == torch's `.to(e4m3)`."""
    from flashrec_amd.kernel.sglops import store_kv_cache

    bits = torch.arange(65536, dtype=torch.int32).to(torch.int16)
    x = bits.view(torch.bfloat16).reshape(512, 128)
    loc = torch.arange(512, dtype=torch.int64)
    kc = torch.zeros(512, 128, dtype=torch.float8_e4m3fn, device=dev)
    vc = torch.zeros_like(kc)
    store_kv_cache(kc, vc, loc.to(dev), x.to(dev), x.to(dev))
    torch.cuda.synchronize()
    ref = codes(x.to(torch.float8_e4m3fn))
    assert torch.equal(codes(kc), ref)
    assert torch.equal(codes(vc), ref)


@pytest.mark.parametrize("m,k", [(1, 2048), (7, 2048), (512, 2048), (64, 6144), (3, 96), (5, 100),
                                 (4, 8200), (33, 512)])
def test_per_token_quant_bitexact(dev, m, k):
    from flashrec_amd.kernel.sglops import per_token_quant_fp8

    x = _bf16((m, k), seed=m * 1000 + k, outliers=max(1, k // 100))
    q, s = per_token_quant_fp8(x.to(dev))
    q_ref, s_ref = ops.per_token_quant_fp8(x)
    assert q.shape == (m, k) and s.shape == (m, 1)
    assert torch.equal(s.cpu(), s_ref)
    assert torch.equal(codes(q), codes(q_ref))


@pytest.mark.parametrize("dtype", [torch.float32, torch.float16])
def test_per_token_quant_other_dtypes(dev, dtype):
    from flashrec_amd.kernel.sglops import per_token_quant_fp8

    g = torch.Generator().manual_seed(11)
    x = (torch.randn(37, 300, generator=g) * 3).to(dtype)
    q, s = per_token_quant_fp8(x.to(dev))
    q_ref, s_ref = ops.per_token_quant_fp8(x)
    assert torch.equal(s.cpu(), s_ref)
    assert torch.equal(codes(q), codes(q_ref))


def test_per_token_quant_edge_rows(dev):
    """Zero rows (scale floor 1e-12/448), a single spike, ties and tiny values."""
    from flashrec_amd.kernel.sglops import per_token_quant_fp8

    x = torch.zeros(6, 1024)
    x[1, 5] = 3.0
    x[2] = torch.linspace(-1, 1, 1024)
    x[3] = 1e-30
    x[4, ::2] = 448.0
    x[4, 1::2] = 464.0 * 448.0 / 464.0
    x[5] = torch.randn(1024, generator=torch.Generator().manual_seed(5)) * 1e-3
    x[5, :64] = -0.0  # signed zeros keep their sign (code 0x80)
    x[2, 100:110] = -0.0
    for dtype in (torch.float32, torch.bfloat16):
        xd = x.to(dtype)
        q, s = per_token_quant_fp8(xd.to(dev))
        q_ref, s_ref = ops.per_token_quant_fp8(xd)
        assert torch.equal(s.cpu(), s_ref)
        assert torch.equal(codes(q), codes(q_ref))


def test_per_token_quant_strided_rows(dev):
    from flashrec_amd.kernel.sglops import per_token_quant_fp8

    big = _bf16((64, 4096), seed=3)
    view = big[:, 1024:3072]  # row stride 4096, width 2048
    q, s = per_token_quant_fp8(view.to(dev))
    q_ref, s_ref = ops.per_token_quant_fp8(view)
    assert torch.equal(s.cpu(), s_ref)
    assert torch.equal(codes(q), codes(q_ref))


def test_quantize_weight_bitexact(dev):
    from flashrec_amd.layers.linear import quantize_weight_fp8

    w = inputs.weight(1024, 2048, seed=9)
    q, s = quantize_weight_fp8(w.to(dev))
    q_ref, s_ref = ops.quantize_weight_fp8(w)
    assert s.shape == (1024,)
    assert torch.equal(s.cpu(), s_ref)
    assert torch.equal(codes(q), codes(q_ref))


@pytest.mark.parametrize("m", [16, 512, 4096])
def test_rms_quant_config0(dev, m):
    from flashrec_amd.kernel.rms_fp8 import rmsnorm_per_token_quant_fp8

    x, gamma, eps = inputs.config0(m=m)
    q, s = rmsnorm_per_token_quant_fp8(x.to(dev), gamma.to(dev), eps)
    q_ref, s_ref = ops.rmsnorm_per_token_quant_fp8(x, gamma, eps)
    assert_fp8_parity(q, s, q_ref, s_ref)


def test_rms_quant_reference_case(dev):
    """Shape/seed of the reference's tests/test_rms_fp8.py:12-24."""
    from flashrec_amd.kernel.rms_fp8 import rmsnorm_per_token_quant_fp8

    torch.manual_seed(0)
    x = torch.randn(16, 2048, dtype=torch.bfloat16)
    w = torch.randn(2048, dtype=torch.bfloat16)
    q, s = rmsnorm_per_token_quant_fp8(x.to(dev), w.to(dev), 1e-6)
    q_ref, s_ref = ops.rmsnorm_per_token_quant_fp8(x, w, 1e-6)
    assert_fp8_parity(q, s, q_ref, s_ref)
    deq = q.float().cpu() * s.cpu()
    torch.testing.assert_close(deq, q_ref.float() * s_ref, atol=2e-1, rtol=2e-1)


@pytest.mark.parametrize("m,h", [(8, 2048), (4096, 2048), (5, 96), (3, 100)])
def test_fused_add_rms_quant(dev, m, h):
    from flashrec_amd.kernel.rms_fp8 import fused_add_rmsnorm_per_token_quant_fp8

    x = _bf16((m, h), seed=1)
    r = _bf16((m, h), seed=2)
    w = (1.0 + 0.1 * torch.randn(h, generator=torch.Generator().manual_seed(3))).to(torch.bfloat16)
    r_dev = r.to(dev)
    q, s, res = fused_add_rmsnorm_per_token_quant_fp8(x.to(dev), r_dev, w.to(dev), 1e-6)
    q_ref, s_ref, res_ref = ops.fused_add_rmsnorm_per_token_quant_fp8(x, r, w, 1e-6)
    assert torch.equal(res.cpu().view(torch.int16), res_ref.view(torch.int16))
    assert res.data_ptr() == r_dev.data_ptr()  # updated in place
    assert_fp8_parity(q, s, q_ref, s_ref)


@pytest.mark.parametrize("m,h", [(16, 2048), (512, 2048), (7, 128), (3, 100)])
def test_rmsnorm_bf16(dev, m, h):
    from flashrec_amd.kernel.sglops import rmsnorm

    x = _bf16((m, h), seed=m + h, outliers=2)
    w = (1.0 + 0.1 * torch.randn(h, generator=torch.Generator().manual_seed(4))).to(torch.bfloat16)
    out = rmsnorm(x.to(dev), w.to(dev), 1e-6)
    assert_bf16_parity(out, ops.rmsnorm(x, w, 1e-6))


def test_fused_add_rmsnorm_bf16_inplace(dev):
    from flashrec_amd.kernel.sglops import fused_add_rmsnorm

    x = _bf16((64, 2048), seed=7)
    r = _bf16((64, 2048), seed=8)
    w = torch.ones(2048, dtype=torch.bfloat16)
    xd, rd = x.to(dev), r.to(dev)
    y, res = fused_add_rmsnorm(xd, rd, w.to(dev), 1e-6)
    y_ref, res_ref = ops.fused_add_rmsnorm(x, r, w, 1e-6)
    assert y.data_ptr() == xd.data_ptr() and res.data_ptr() == rd.data_ptr()
    assert torch.equal(res.cpu().view(torch.int16), res_ref.view(torch.int16))
    assert_bf16_parity(y, y_ref)


@pytest.mark.parametrize("m,two_d", [(12, 96), (64, 12288), (4096, 12288), (5, 100), (3, 20000), (33, 4096), (7, 16384)])
def test_silu_quant(dev, m, two_d):
    from flashrec_amd.kernel.silu_fp8 import silu_and_mul_per_token_quant_fp8

    x = _bf16((m, two_d), seed=two_d + m)
    q, s = silu_and_mul_per_token_quant_fp8(x.to(dev))
    q_ref, s_ref = ops.silu_and_mul_per_token_quant_fp8(x)
    assert q.shape == (m, two_d // 2)
    assert_fp8_parity(q, s, q_ref, s_ref)


def test_silu_and_mul_bf16(dev):
    from flashrec_amd.kernel.sglops import silu_and_mul

    x = _bf16((33, 2 * 1536), seed=5, scale=3.0)
    out = silu_and_mul(x.to(dev))
    assert_bf16_parity(out, ops.silu_and_mul(x))


@pytest.mark.parametrize("scale", [1.0, 4.0, 20.0])
def test_silu_wide_gate_range(dev, scale):
    """Gates over a wide range (|g| up to ~80 at scale 20, where the
    exponent's fp32 argument is least exact): the bf16 silu(g) * u and the
    e4m3 codes match the reference composition (flip bar as elsewhere; none
    were observed on these inputs)."""
    from flashrec_amd.kernel.sglops import silu_and_mul
    from flashrec_amd.kernel.silu_fp8 import silu_and_mul_per_token_quant_fp8

    x = _bf16((256, 2 * 6144), seed=int(scale) + 40, scale=scale)
    assert_bf16_parity(silu_and_mul(x.to(dev)), ops.silu_and_mul(x))
    q, s = silu_and_mul_per_token_quant_fp8(x.to(dev))
    q_ref, s_ref = ops.silu_and_mul_per_token_quant_fp8(x)
    assert_fp8_parity(q, s, q_ref, s_ref)


def test_empty_batch(dev):
    from flashrec_amd.kernel.sglops import per_token_quant_fp8

    q, s = per_token_quant_fp8(torch.empty(0, 2048, dtype=torch.bfloat16, device=dev))
    assert q.shape == (0, 2048) and s.shape == (0, 1)


@pytest.mark.parametrize("m,h", [(512, 2048), (7, 100)])
def test_fp16_rms_quant_and_residual(dev, m, h):
    """fp16 activations (reference rms_fp8.py:86 takes x.dtype): intermediates
    round to fp16 as the reference's CPU composition does."""
    from flashrec_amd.kernel.rms_fp8 import (fused_add_rmsnorm_per_token_quant_fp8,
                                             rmsnorm_per_token_quant_fp8)
    from flashrec_amd.kernel.sglops import rmsnorm

    g = torch.Generator().manual_seed(m + h)
    x = torch.randn(m, h, generator=g).to(torch.float16)
    r = torch.randn(m, h, generator=g).to(torch.float16)
    w = (1.0 + 0.1 * torch.randn(h, generator=g)).to(torch.bfloat16)
    q, s = rmsnorm_per_token_quant_fp8(x.to(dev), w.to(dev), 1e-6)
    q_ref, s_ref = ops.rmsnorm_per_token_quant_fp8(x, w, 1e-6)
    assert_fp8_parity(q, s, q_ref, s_ref, label=f"fp16 rms {m}x{h}")
    rd = r.to(dev)
    q, s, res = fused_add_rmsnorm_per_token_quant_fp8(x.to(dev), rd, w.to(dev), 1e-6)
    q_ref, s_ref, res_ref = ops.fused_add_rmsnorm_per_token_quant_fp8(x, r, w, 1e-6)
    assert res.dtype == torch.float16 and torch.equal(res.cpu(), res_ref)
    assert_fp8_parity(q, s, q_ref, s_ref, label=f"fp16 add+rms {m}x{h}")
    y = rmsnorm(x.to(dev), w.to(dev), 1e-6)
    assert y.dtype == torch.float16
    assert_bf16_parity(y, ops.rmsnorm(x, w, 1e-6))  # 16-bit patterns: same bar


@pytest.mark.parametrize("m,two_d", [(64, 12288), (5, 100)])
def test_fp16_silu_quant(dev, m, two_d):
    from flashrec_amd.kernel.sglops import silu_and_mul
    from flashrec_amd.kernel.silu_fp8 import silu_and_mul_per_token_quant_fp8

    g = torch.Generator().manual_seed(two_d)
    x = (3 * torch.randn(m, two_d, generator=g)).to(torch.float16)
    q, s = silu_and_mul_per_token_quant_fp8(x.to(dev))
    q_ref, s_ref = ops.silu_and_mul_per_token_quant_fp8(x)
    assert_fp8_parity(q, s, q_ref, s_ref, label=f"fp16 silu {m}x{two_d}")
    y = silu_and_mul(x.to(dev))
    assert y.dtype == torch.float16
    assert_bf16_parity(y, ops.silu_and_mul(x))


def _assert_fp32_row_parity(q, s, q_ref, s_ref, label):
    """fp32 activations: the rows are never rounded to 16 bits, so a different
    fp32 summation order (the RMS variance) or exp moves amax, and with it the
    scale, by a few fp32 ulps on many rows; the bar is then scales within
    1e-6 relative and codes equal but for 1-ULP flips on < 0.1 % of elements."""
    s, s_ref = s.detach().cpu().reshape(-1), s_ref.reshape(-1)
    rel = ((s - s_ref).abs() / s_ref.abs()).max().item()
    frac, dist = code_flip_stats(q, q_ref)
    print(f"parity {label}: scales within {rel:.2e}, {frac:.2e} of codes flipped")
    assert rel <= 1e-6 and dist <= 1 and frac < 1e-3


@pytest.mark.parametrize("m,h", [(512, 2048), (7, 100)])
def test_fp32_rms_quant_and_residual(dev, m, h):
    """fp32 activations (the reference's fused op takes any x.dtype,
    rms_fp8.py:84-86; its CPU composition keeps fp32 rows unrounded)."""
    from flashrec_amd.kernel.rms_fp8 import (fused_add_rmsnorm_per_token_quant_fp8,
                                             rmsnorm_per_token_quant_fp8)
    from flashrec_amd.kernel.sglops import fused_add_rmsnorm, rmsnorm

    g = torch.Generator().manual_seed(7 * m + h)
    x = torch.randn(m, h, generator=g)
    r = torch.randn(m, h, generator=g)
    w = (1.0 + 0.1 * torch.randn(h, generator=g)).to(torch.bfloat16)
    q, s = rmsnorm_per_token_quant_fp8(x.to(dev), w.to(dev), 1e-6)
    q_ref, s_ref = ops.rmsnorm_per_token_quant_fp8(x, w, 1e-6)
    _assert_fp32_row_parity(q, s, q_ref, s_ref, f"fp32 rms {m}x{h}")
    rd = r.to(dev)
    q, s, res = fused_add_rmsnorm_per_token_quant_fp8(x.to(dev), rd, w.to(dev), 1e-6)
    q_ref, s_ref, res_ref = ops.fused_add_rmsnorm_per_token_quant_fp8(x, r, w, 1e-6)
    assert res.dtype == torch.float32 and torch.equal(res.cpu(), res_ref)  # one fp32 add: exact
    _assert_fp32_row_parity(q, s, q_ref, s_ref, f"fp32 add+rms {m}x{h}")
    # unquantized fp32 outputs: only the variance's summation order differs,
    # which moves rsqrt by a few fp32 ulps
    y = rmsnorm(x.to(dev), w.to(dev), 1e-6)
    assert y.dtype == torch.float32
    torch.testing.assert_close(y.cpu(), ops.rmsnorm(x, w, 1e-6), rtol=4e-6, atol=0)
    xd, rd = x.to(dev), r.to(dev)
    y, res = fused_add_rmsnorm(xd, rd, w.to(dev), 1e-6)
    y_ref, res_ref = ops.fused_add_rmsnorm(x, r, w, 1e-6)
    assert torch.equal(res.cpu(), res_ref)
    torch.testing.assert_close(y.cpu(), y_ref, rtol=4e-6, atol=0)


@pytest.mark.parametrize("m,two_d", [(64, 12288), (5, 100)])
def test_fp32_silu_quant(dev, m, two_d):
    from flashrec_amd.kernel.sglops import silu_and_mul
    from flashrec_amd.kernel.silu_fp8 import silu_and_mul_per_token_quant_fp8

    g = torch.Generator().manual_seed(two_d + 1)
    x = 3 * torch.randn(m, two_d, generator=g)
    q, s = silu_and_mul_per_token_quant_fp8(x.to(dev))
    q_ref, s_ref = ops.silu_and_mul_per_token_quant_fp8(x)
    _assert_fp32_row_parity(q, s, q_ref, s_ref, f"fp32 silu {m}x{two_d}")
    # fp32 outputs: exp differs from torch's vectorised CPU exp by an ulp or so
    y = silu_and_mul(x.to(dev))
    assert y.dtype == torch.float32
    torch.testing.assert_close(y.cpu(), ops.silu_and_mul(x), rtol=4e-6, atol=1e-30)


def test_silu_unaligned_rows_match_aligned(dev):
    """A row that the vector kernel takes and the same row through the generic
    kernel (a strided, unaligned view) give the same bits: both use one SiLU
    arithmetic."""
    from flashrec_amd.kernel.sglops import silu_and_mul
    from flashrec_amd.kernel.silu_fp8 import silu_and_mul_per_token_quant_fp8

    g = torch.Generator().manual_seed(11)
    x = (4 * torch.randn(96, 2048, generator=g)).to(torch.bfloat16)
    x[3, 5] = 100.0  # a gate beyond the in-range form in one row
    aligned = x.to(dev)
    holder = torch.zeros(96, 2048 + 1, dtype=torch.bfloat16, device=dev)
    holder[:, 1:] = aligned
    unaligned = holder[:, 1:]  # rows start 2 bytes into a 16-byte line
    assert unaligned.data_ptr() % 16 != 0
    assert torch.equal(silu_and_mul(unaligned).cpu().view(torch.int16),
                       silu_and_mul(aligned).cpu().view(torch.int16))
    qa, sa = silu_and_mul_per_token_quant_fp8(aligned)
    qu, su = silu_and_mul_per_token_quant_fp8(unaligned)
    assert torch.equal(codes(qa), codes(qu)) and torch.equal(sa.cpu(), su.cpu())
