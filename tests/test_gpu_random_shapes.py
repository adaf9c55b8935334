"""Seeded random shapes through the main entry points, each at its own bar:

* the W8A8 GEMM against the fp32 dequantised oracle (max-abs-normalised
  1e-2 on sampled rows), its bf16 output equal to its fp32 output rounded
  once, the residual variant bit-exact with the GEMM then the add, the
  SiLU-and-mul variant bit-exact with the GEMM then ``silu_and_mul``; the
  same four through the prearranged-weight kernel, equal to the plain ones;
* paged attention against the oracle (1e-2 of each row's max) and the
  quantizing variant bit-exact with attention then the per-token quant, with
  and without the plan, on random head ratios, prefix lengths (0, partial and
  whole 32-key blocks) and own-slot counts;
* the row quantizers (quant, RMSNorm, add + RMSNorm, SiLU-and-mul) at the
  fp8 parity bar, bf16 and fp16, small, unit and large magnitudes.

The shapes are drawn from lists that cross every tile shape, edge tiles, K
tails (repacked by the wrapper) and the vector / generic row paths."""

import random

import pytest
import torch

from helpers import assert_fp8_parity, max_abs_rel
from oracle import ops

pytestmark = pytest.mark.gpu


@pytest.mark.parametrize("seed", range(24))
def test_random_gemm_variants(dev, seed):
    from flashrec_amd.kernel.sglops import (fp8_scaled_mm, fp8_scaled_mm_prearranged, fp8_scaled_mm_residual,
                                            fp8_scaled_mm_silu, interleave_gate_up, prearrange_fp8_weight,
                                            silu_and_mul)

    rnd = random.Random(seed)
    m = rnd.choice([1, 7, 33, 300, 512, 777, 1381, 2661, 4196])
    n = 16 * rnd.randint(1, 800)
    k = rnd.choice([16, 48, 64, 256, 1000, 1040, 2048, 2064])
    g = torch.Generator().manual_seed(1000 + seed)
    qa, sa = ops.per_token_quant_fp8(torch.randn(m, k, generator=g).to(torch.bfloat16))
    qw, sw = ops.quantize_weight_fp8((0.02 * torch.randn(n, k, generator=g)).to(torch.bfloat16))
    a, s_a, w, s_w = qa.to(dev), sa.to(dev), qw.to(dev), sw.to(dev)
    out32 = fp8_scaled_mm(a, w.t(), s_a, s_w, torch.float32)
    out16 = fp8_scaled_mm(a, w.t(), s_a, s_w, torch.bfloat16)
    rows = torch.randperm(m, generator=g)[:48]
    assert max_abs_rel(out32.cpu()[rows], ops.fp8_scaled_mm(qa[rows], qw.t(), sa[rows], sw)) < 1e-2
    assert torch.equal(out16.cpu(), out32.cpu().to(torch.bfloat16))
    res = (torch.randn(m, n, generator=g) * 2).to(torch.bfloat16).to(dev)
    want = (res + out16).cpu()
    got = fp8_scaled_mm_residual(a, w.t(), s_a, s_w, res)
    assert torch.equal(got.cpu().view(torch.int16), want.view(torch.int16))
    got = fp8_scaled_mm_silu(a, interleave_gate_up(w).t(), s_a, interleave_gate_up(s_w))
    assert torch.equal(got.cpu().view(torch.int16), silu_and_mul(out16).cpu().view(torch.int16))
    # prearranged weights: the same values (a zero K step may turn -0 into +0)
    print(f"random gemm seed {seed}: {m}x{n}x{k}", flush=True)
    pre = prearrange_fp8_weight(w.t())
    assert torch.equal(fp8_scaled_mm_prearranged(a, pre, s_a, s_w, torch.float32).cpu(), out32.cpu())
    assert torch.equal(fp8_scaled_mm_prearranged(a, pre, s_a, s_w, torch.bfloat16).cpu().float(),
                       out16.cpu().float())
    res2 = (torch.randn(m, n, generator=g) * 2).to(torch.bfloat16)
    got = fp8_scaled_mm_prearranged(a, pre, s_a, s_w, residual=res2.to(dev))
    assert torch.equal(got.cpu().float(), (res2 + out16.cpu()).float())
    got = fp8_scaled_mm_prearranged(a, prearrange_fp8_weight(interleave_gate_up(w).t()), s_a,
                                    interleave_gate_up(s_w), silu=True)
    assert torch.equal(got.cpu().float(), silu_and_mul(out16).cpu().float())


@pytest.mark.parametrize("seed", range(16))
def test_random_attention(dev, seed):
    from flashrec_amd.attention import attention_plan, paged_attention, paged_attention_quant_fp8
    from flashrec_amd.kernel.sglops import per_token_quant_fp8

    rnd = random.Random(seed)
    hk = rnd.choice([1, 2, 4, 8])
    hq = hk * rnd.choice([1, 2, 4])
    slots = rnd.choice([512, 4096, 20000])
    g = torch.Generator().manual_seed(2000 + seed)
    kc = (torch.randn(slots, hk, 128, generator=g) * rnd.choice([0.5, 1.0, 3.0])).to(torch.float8_e4m3fn)
    vc = torch.randn(slots, hk, 128, generator=g).to(torch.float8_e4m3fn)
    rows = []
    for _ in range(rnd.randint(1, 3)):
        plen = rnd.choice([0, 5, 31, 32, 33, 64, 100, 128])
        pre = torch.randint(1, slots, (plen,), generator=g, dtype=torch.int32)
        for _ in range(rnd.randint(1, 40)):
            own = rnd.randint(0 if plen else 1, 9)
            rows.append(torch.cat([pre, torch.randint(1, slots, (own,), generator=g, dtype=torch.int32)]))
    idx = torch.cat(rows)
    ln = torch.tensor([int(r.numel()) for r in rows], dtype=torch.int32)
    st = torch.zeros(len(rows), dtype=torch.int32)
    st[1:] = torch.cumsum(ln[:-1], 0)
    T = len(rows)
    q = (torch.randn(T, hq, 128, generator=g) * 2).to(torch.bfloat16)
    d = [t.to(dev) for t in (q, kc, vc, idx, st, ln)]
    scale = 128 ** -0.5
    for gp in (None, attention_plan(d[3], d[4], d[5], hq, hk)):
        att = paged_attention(*d, scale, group_prefix=gp)
        rq, rs = per_token_quant_fp8(att.reshape(T, -1))
        fq, fs = paged_attention_quant_fp8(*d, scale, group_prefix=gp)
        assert torch.equal(fq.view(torch.uint8).cpu(), rq.view(torch.uint8).cpu())
        assert torch.equal(fs.cpu(), rs.cpu())
    ref = ops.paged_attention(q, kc, vc, idx, st, ln, scale).float()
    err = ((att.cpu().float() - ref).abs().amax(-1) / ref.abs().amax(-1).clamp(min=1e-6)).max().item()
    assert err < 1e-2, err


@pytest.mark.parametrize("seed", range(24))
def test_random_row_quantizers(dev, seed):
    from flashrec_amd.kernel.rms_fp8 import fused_add_rmsnorm_per_token_quant_fp8, rmsnorm_per_token_quant_fp8
    from flashrec_amd.kernel.sglops import per_token_quant_fp8
    from flashrec_amd.kernel.silu_fp8 import silu_and_mul_per_token_quant_fp8

    rnd = random.Random(seed)
    m = rnd.choice([1, 3, 64, 300, 512, 1000, 4096])
    k = rnd.choice([8, 64, 100, 512, 1000, 2048, 6144])
    dt = rnd.choice([torch.bfloat16, torch.bfloat16, torch.float16])
    sc = rnd.choice([0.01, 1.0, 30.0])
    g = torch.Generator().manual_seed(3000 + seed)
    x = (torch.randn(m, k, generator=g) * sc).to(dt)
    w = (1 + 0.1 * torch.randn(k, generator=g)).to(dt)
    r = (torch.randn(m, k, generator=g) * sc).to(dt)
    kind = ("quant", "rms", "addrms", "silu")[seed % 4]
    if kind == "quant":
        q, s = per_token_quant_fp8(x.to(dev))
        q_ref, s_ref = ops.per_token_quant_fp8(x)
    elif kind == "rms":
        q, s = rmsnorm_per_token_quant_fp8(x.to(dev), w.to(dev), 1e-6)
        q_ref, s_ref = ops.rmsnorm_per_token_quant_fp8(x, w, 1e-6)
    elif kind == "addrms":
        q, s, res = fused_add_rmsnorm_per_token_quant_fp8(x.to(dev), r.to(dev), w.to(dev), 1e-6)
        q_ref, s_ref, res_ref = ops.fused_add_rmsnorm_per_token_quant_fp8(x, r.clone(), w, 1e-6)
        assert torch.equal(res.cpu().view(torch.int16), res_ref.view(torch.int16))
    else:
        xs = torch.cat([x, r], dim=1)
        q, s = silu_and_mul_per_token_quant_fp8(xs.to(dev))
        q_ref, s_ref = ops.silu_and_mul_per_token_quant_fp8(xs)
    assert_fp8_parity(q, s, q_ref, s_ref, label=f"{kind} {m}x{k} {dt} x{sc}")


@pytest.mark.parametrize("seed", range(8))
def test_random_log_softmax_topk(dev, seed):
    """row_topk with the log-softmax folded in, bit-identical to log_softmax_f32
    then row_topk, which is held to the oracle's top-k: random row counts,
    widths 4096 / 8192 (the folded kernel) and others (the two calls), k up
    to 1024, logit scales that make ties and underflowing exp."""
    from oracle import beam

    from flashrec_amd.kernel.beam_trie import row_topk
    from flashrec_amd.kernel.sglops import log_softmax_f32

    rnd = random.Random(seed)
    r = rnd.choice([1, 3, 64, 257, 1024])
    v = rnd.choice([4096, 8192, 8192, 1000])
    k = rnd.choice([1, 7, 256, 300, 512, 1000])
    sc = rnd.choice([0.5, 4.0, 60.0])
    g = torch.Generator().manual_seed(4000 + seed)
    x = torch.randn(r, v, generator=g) * sc
    if seed % 2:
        x = torch.round(x)  # ties
    cand = torch.randint(0, 10 ** 6, (v,), generator=g)
    xd, cd = x.to(dev), cand.to(dev)
    lp = log_softmax_f32(xd)
    fv, fi, ft = row_topk(xd, k, cd, log_softmax=True)
    rv, ri, rt = row_topk(lp, k, cd)
    assert torch.equal(fv.cpu().view(torch.int32), rv.cpu().view(torch.int32))
    assert torch.equal(fi.cpu(), ri.cpu()) and torch.equal(ft.cpu(), rt.cpu())
    ov, oi, _ = beam.row_topk(lp.cpu(), k, cand)
    assert torch.equal(rv.cpu().view(torch.int32), ov.view(torch.int32)) and torch.equal(ri.cpu(), oi)
