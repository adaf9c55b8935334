"""Pins for the oracle (oracle/ops.py) that do not restate its formulas:
exact rational arithmetic, float64 closed forms, integer-exact products,
complex-number rotation for RoPE, and layout/permutation invariants."""

from fractions import Fraction

import numpy as np
import pytest
import torch

from oracle import e4m3, inputs, ops


def _f32(v) -> float:
    return float(np.float32(v))


def _rn_f32(fr: Fraction) -> float:
    """Round an exact rational to the nearest fp32 (ties to even) via float64
    neighbours: exact for the magnitudes used here."""
    lo = np.float32(float(fr))
    cands = [np.nextafter(lo, np.float32(-np.inf)), lo, np.nextafter(lo, np.float32(np.inf))]
    best = min(cands, key=lambda c: (abs(Fraction(float(c)) - fr),
                                      int(np.float32(c).view(np.uint32)) & 1))
    return float(best)


def test_per_token_quant_exact_rational():
    """q = e4m3(RN(x / RN(amax/448))) computed with exact rationals, element by element."""
    g = torch.Generator().manual_seed(0)
    x = (torch.randn(6, 40, generator=g) * torch.tensor([1, 1e-3, 30, 1e4, 0.1, 7.0])[:, None])
    x = x.to(torch.bfloat16)
    q, s = ops.per_token_quant_fp8(x)
    for r in range(x.shape[0]):
        row = [float(v) for v in x[r].float()]
        amax = max(max(abs(v) for v in row), _f32(1e-12))
        scale = _rn_f32(Fraction(amax) / 448)
        assert float(s[r, 0]) == scale
        for c, v in enumerate(row):
            y = _rn_f32(Fraction(v) / Fraction(scale))
            y = min(max(y, -448.0), 448.0)
            assert int(q[r, c].view(torch.uint8)) == int(e4m3.encode(np.array([y]))[0])


def test_per_token_quant_closed_form_properties():
    x, _, _ = inputs.config0(m=64)
    q, s = ops.per_token_quant_fp8(x)
    xf = x.float()
    # the largest |x| of each row maps to +-448 exactly
    idx = xf.abs().argmax(dim=-1)
    top = q.float()[torch.arange(64), idx].abs()
    assert (top == 448.0).all()
    # dequantised values are within half an e4m3 step (relative 1/16) of x
    deq = q.float() * s
    err = (deq - xf).abs()
    bound = xf.abs() / 16 + s * 2.0 ** -10 + 1e-30
    assert (err <= bound * 1.0001).all()
    # zero row: scale floor
    q0, s0 = ops.per_token_quant_fp8(torch.zeros(2, 8, dtype=torch.bfloat16))
    assert (s0 == torch.tensor(1e-12, dtype=torch.float32) / 448).all()
    assert (q0.view(torch.uint8) == 0).all()


def test_quantize_weight_is_per_row_quant():
    w = inputs.weight(64, 256, seed=3)
    qw, sw = ops.quantize_weight_fp8(w)
    qa, sa = ops.per_token_quant_fp8(w)
    assert torch.equal(sw, sa.reshape(-1))
    assert torch.equal(qw.view(torch.uint8), qa.view(torch.uint8))


def test_rmsnorm_exact_on_representable_rows():
    """Rows of +-1/+-2 have exact fp32 sums; the result is the textbook formula
    evaluated step by step in fp32 (numpy), incl. the bf16 rounding."""
    g = torch.Generator().manual_seed(1)
    x = (torch.randint(1, 3, (4, 64), generator=g) * (torch.randint(0, 2, (4, 64), generator=g) * 2 - 1)).float()
    w = torch.linspace(0.5, 1.5, 64)
    out = ops.rmsnorm(x.to(torch.bfloat16), w.to(torch.bfloat16), 1e-6)
    xn = x.numpy().astype(np.float32)
    wn = w.to(torch.bfloat16).float().numpy()
    for r in range(4):
        var = np.float32((xn[r] ** 2).sum() / np.float32(64))
        rstd = np.float32(1) / np.sqrt(np.float32(var + np.float32(1e-6)))
        y = (xn[r] * rstd).astype(np.float32) * wn
        ref = torch.from_numpy(y.astype(np.float32)).to(torch.bfloat16)
        assert torch.equal(out[r], ref)


def test_rmsnorm_float64_closed_form():
    x, g, eps = inputs.config0(m=32)
    out = ops.rmsnorm(x, g, eps).double()
    xd = x.double()
    ref = xd / torch.sqrt((xd * xd).mean(-1, keepdim=True) + eps) * g.double()
    rel = (out - ref).abs() / ref.abs().clamp(min=1e-6)
    assert rel.max() < 2.0 ** -8  # one bf16 rounding


def test_fused_add_rmsnorm_residual_is_bf16_sum():
    g = torch.Generator().manual_seed(2)
    x = torch.randn(3, 32, generator=g).to(torch.bfloat16)
    r = torch.randn(3, 32, generator=g).to(torch.bfloat16)
    _, res = ops.fused_add_rmsnorm(x, r, torch.ones(32), 1e-6)
    ref = (x.double() + r.double()).float().to(torch.bfloat16)  # exact sum, one rounding
    assert torch.equal(res, ref)


def test_silu_and_mul_float64():
    g = torch.Generator().manual_seed(3)
    x = (torch.randn(16, 64, generator=g) * 4).to(torch.bfloat16)
    out = ops.silu_and_mul(x).double()
    gt, up = x[:, :32].double(), x[:, 32:].double()
    ref = gt / (1 + torch.exp(-gt)) * up
    rel = (out - ref).abs() / ref.abs().clamp(min=1e-3)
    assert rel.max() < 2.0 ** -7  # two bf16 roundings
    assert ops.silu_and_mul(torch.zeros(1, 4, dtype=torch.bfloat16)).abs().max() == 0


def test_gemm_oracle_integer_exact_and_torch_scaled_mm():
    g = torch.Generator().manual_seed(4)
    a = torch.randint(-8, 9, (16, 64), generator=g).float()
    w = torch.randint(-8, 9, (24, 64), generator=g).float()
    qa, qw = a.to(torch.float8_e4m3fn), w.to(torch.float8_e4m3fn)
    out = ops.fp8_scaled_mm(qa, qw.t(), torch.ones(16, 1), torch.ones(24))
    assert torch.equal(out, (a.long() @ w.long().t()).float())
    # scales multiply rows / columns
    sa = torch.arange(1, 17, dtype=torch.float32).reshape(16, 1)
    sb = torch.full((24,), 0.5)
    out2 = ops.fp8_scaled_mm(qa, qw.t(), sa, sb)
    torch.testing.assert_close(out2, out * sa * 0.5)
    # agrees with the reference's literal CPU branch (bf16 double rounding)
    x = torch.randn(32, 256, generator=g).to(torch.bfloat16)
    wt = (0.02 * torch.randn(48, 256, generator=g)).to(torch.bfloat16)
    qa, sa = ops.per_token_quant_fp8(x)
    qw, sw = ops.quantize_weight_fp8(wt)
    lit = ops.fp8_scaled_mm_torch_cpu(qa, qw.t(), sa, sw, torch.bfloat16).float()
    ref = ops.fp8_scaled_mm(qa, qw.t(), sa, sw)
    assert ((lit - ref).abs().max() / ref.abs().max()) < 1e-2


def test_cos_sin_cache_float64():
    cache = ops.cos_sin_cache(128, 300, 1e6).double()
    inv = 1.0 / (1e6 ** (torch.arange(0, 128, 2, dtype=torch.float64) / 128))
    ang = torch.arange(300, dtype=torch.float64)[:, None] * inv[None]
    assert (cache[:, :64] - ang.cos()).abs().max() < 1e-4
    assert (cache[:, 64:] - ang.sin()).abs().max() < 1e-4
    assert torch.equal(cache[0, :64], torch.ones(64, dtype=torch.float64))


def test_rope_is_complex_rotation():
    """(x_i + i x_{i+D/2}) * exp(i * pos * inv_freq_i): an independent statement
    of rotate-half RoPE; a wrong sign or half pairing fails it."""
    g = torch.Generator().manual_seed(5)
    t, h, d = 6, 3, 128
    x = torch.randn(t, h, d, generator=g).to(torch.bfloat16)
    pos = torch.tensor([0, 1, 7, 100, 1000, 4095])
    cache = ops.cos_sin_cache(d, 4096, 1e6)
    out = ops.apply_rope(pos, x, cache).double()
    xd = x.double()
    z = torch.complex(xd[..., :64], xd[..., 64:])
    c = cache[pos].double()
    rot = torch.complex(c[:, :64], c[:, 64:])[:, None, :]
    zr = z * rot
    ref = torch.cat([zr.real, zr.imag], dim=-1)
    assert ((out - ref).abs() <= ref.abs() * 2.0 ** -8 + 1e-6).all()
    assert torch.equal(out[0], xd[0])  # position 0 is the identity


def test_qk_norm_rope_store_layout():
    t, hq, hk, d, slots = 5, 4, 2, 128, 16
    g = torch.Generator().manual_seed(6)
    q = torch.randn(t, hq, d, generator=g).to(torch.bfloat16)
    k = torch.randn(t, hk, d, generator=g).to(torch.bfloat16)
    v = torch.randn(t, hk, d, generator=g).to(torch.bfloat16)
    pos = torch.zeros(t, dtype=torch.int64)
    loc = torch.tensor([3, 9, 1, 15, 4])
    kc = torch.zeros(slots, hk, d, dtype=torch.float8_e4m3fn)
    vc = torch.zeros_like(kc)
    w = torch.ones(d, dtype=torch.bfloat16)
    qr = ops.qk_norm_rope_store_fp8(q, k, v, pos, loc, w, w, 1e-6, ops.cos_sin_cache(d, 8, 1e6),
                                    kc, vc)
    # position 0: rotation is the identity, so q is just the normalised q
    assert torch.equal(qr, ops.rmsnorm(q, w, 1e-6))
    for i, s in enumerate(loc.tolist()):
        assert torch.equal(vc[s].view(torch.uint8), v[i].to(torch.float8_e4m3fn).view(torch.uint8))
        assert torch.equal(kc[s].view(torch.uint8),
                           ops.rmsnorm(k[i], w, 1e-6).to(torch.float8_e4m3fn).view(torch.uint8))
    untouched = sorted(set(range(slots)) - set(loc.tolist()))
    assert (kc[untouched].view(torch.uint8) == 0).all()


def test_log_softmax_rows_normalised():
    g = torch.Generator().manual_seed(7)
    h = torch.randn(8, 64, generator=g).to(torch.bfloat16)
    w = (0.1 * torch.randn(100, 64, generator=g)).to(torch.bfloat16)
    lp = ops.restricted_logprobs_fp8(h, w).double()
    torch.testing.assert_close(lp.exp().sum(-1), torch.ones(8, dtype=torch.float64))


@pytest.mark.parametrize("cfg", [0, 3])
def test_inputs_are_seeded(cfg):
    if cfg == 0:
        a, b = inputs.config0(m=8), inputs.config0(m=8)
        assert torch.equal(a[0], b[0]) and torch.equal(a[1], b[1])
    else:
        a, b = inputs.config3(t=64, slots=1024), inputs.config3(t=64, slots=1024)
        assert all(torch.equal(x, y) for x, y in zip(a, b))
        loc = a[4]
        assert (loc > 0).all() and loc.unique().numel() == 64  # slot 0 never used, no collisions


def test_fp16_rows_round_to_fp16():
    """fp16 activations (accepted by the reference's fused ops, rms_fp8.py:86,
    silu_fp8.py:79-82): the oracle's intermediates are fp16 roundings of the
    float64 closed forms, and the residual is the fp16-rounded exact sum."""
    g = torch.Generator().manual_seed(11)
    x = torch.randn(8, 64, generator=g).to(torch.float16)
    w = (1 + 0.1 * torch.randn(64, generator=g)).to(torch.bfloat16)
    out = ops.rmsnorm(x, w, 1e-6)
    assert out.dtype == torch.float16
    xd = x.double()
    ref = xd / torch.sqrt((xd * xd).mean(-1, keepdim=True) + 1e-6) * w.double()
    assert ((out.double() - ref).abs() / ref.abs().clamp(min=1e-4)).max() < 2.0 ** -10
    r = torch.randn(8, 64, generator=g).to(torch.float16)
    _, res = ops.fused_add_rmsnorm(x, r, w, 1e-6)
    assert torch.equal(res, (x.double() + r.double()).to(torch.float16))
    s = (torch.randn(8, 64, generator=g) * 3).to(torch.float16)
    out = ops.silu_and_mul(s).double()
    gt, up = s[:, :32].double(), s[:, 32:].double()
    ref = gt / (1 + torch.exp(-gt)) * up
    assert ((out - ref).abs() / ref.abs().clamp(min=1e-3)).max() < 2.0 ** -9  # two fp16 roundings
