"""The W8A8 GEMM over prearranged weights (``fp8_scaled_mm_prearranged``).

It takes the same MFMA operands in the same K order as ``fp8_scaled_mm``, so
the two agree bit for bit (compared as values: a zero K step added after a
negative-zero sum may turn -0 into +0); each is also held to the fp32
dequantised-matmul oracle, and integer operands pin the accumulation exactly.
"""

import pytest
import torch

from helpers import max_abs_rel
from oracle import ops

pytestmark = pytest.mark.gpu

TOL = 1e-2


def _operands(m, n, k, seed):
    g = torch.Generator().manual_seed(seed)
    x = torch.randn(m, k, generator=g).to(torch.bfloat16)
    w = (0.02 * torch.randn(n, k, generator=g)).to(torch.bfloat16)
    qa, sa = ops.per_token_quant_fp8(x)
    qw, sw = ops.quantize_weight_fp8(w)
    return qa, sa, qw, sw


def _same_values(a, b):
    assert a.shape == b.shape and a.dtype == b.dtype
    af, bf = a.float().cpu(), b.float().cpu()
    same = (af == bf) | (torch.isnan(af) & torch.isnan(bf))
    assert bool(same.all()), f"{int((~same).sum())} of {same.numel()} outputs differ"


# config shapes (gate_up at 4096 and 512 rows, down, qkv, o, the SID head) and
# edge shapes: partial tiles, N not a multiple of 32, K tails of every kind
SHAPES = [(4096, 12288, 2048), (512, 12288, 2048), (4096, 2048, 6144), (4096, 4096, 2048), (4096, 2048, 2048),
          (300, 1000, 384), (33, 200, 320), (1, 256, 2048), (257, 264, 48), (64, 512, 1024)]


@pytest.mark.parametrize("m,n,k", SHAPES)
def test_prearranged_matches_plain_and_oracle(dev, m, n, k):
    from flashrec_amd.kernel.sglops import fp8_scaled_mm, fp8_scaled_mm_prearranged, prearrange_fp8_weight

    print(f"prearranged gemm {m}x{n}x{k}", flush=True)
    qa, sa, qw, sw = _operands(m, n, k, seed=m + 3 * n + 7 * k)
    a, b, sad, swd = qa.to(dev), qw.to(dev).t(), sa.to(dev), sw.to(dev)
    w = prearrange_fp8_weight(b)
    got = fp8_scaled_mm_prearranged(a, w, sad, swd, torch.bfloat16)
    want = fp8_scaled_mm(a, b, sad, swd, torch.bfloat16)
    torch.cuda.synchronize()
    _same_values(got, want)
    rows = torch.arange(0, m, max(1, m // 256))  # the oracle on a row sample (all rows up to 256)
    ref = ops.fp8_scaled_mm(qa[rows], qw.t(), sa[rows], sw)
    assert max_abs_rel(got[rows.to(dev)], ref) < TOL


def test_prearranged_layout_bytes(dev):
    """The documented layout: out[((n/32)*KT + k/64)*2048 + h*1024 + l*16 + b]
    = w[32*(n/32) + l%32][64*(k/64) + 32*(l/32) + 16*h + b], zeros past N, K."""
    from flashrec_amd.kernel.sglops import prearrange_fp8_weight

    n, k = 40, 200
    g = torch.Generator().manual_seed(2)
    codes = torch.randint(0, 126, (n, k), generator=g).to(torch.uint8)  # no NaN patterns
    w = prearrange_fp8_weight(codes.view(torch.float8_e4m3fn).to(dev).t())
    kt = 4  # ceil(200 / 64) = 4 steps, already a multiple of 4
    got = w.data.cpu().view(2, kt, 2, 64, 16)
    want = torch.zeros(2, kt, 2, 64, 16, dtype=torch.uint8)
    padded = torch.zeros(64, kt * 64, dtype=torch.uint8)
    padded[:n, :k] = codes
    for blk in range(2):
        for s in range(kt):
            for h in range(2):
                for lane in range(64):
                    r = 32 * blk + lane % 32
                    c = 64 * s + 32 * (lane // 32) + 16 * h
                    want[blk, s, h, lane] = padded[r, c:c + 16]
    assert torch.equal(got, want)


def test_prearranged_integer_exact(dev):
    from flashrec_amd.kernel.sglops import fp8_scaled_mm_prearranged, prearrange_fp8_weight

    g = torch.Generator().manual_seed(0)
    m, n, k = 512, 768, 1024
    a = torch.randint(-4, 5, (m, k), generator=g).float()
    wv = torch.randint(-4, 5, (n, k), generator=g).float()
    qa, qw = a.to(torch.float8_e4m3fn), wv.to(torch.float8_e4m3fn)
    w = prearrange_fp8_weight(qw.to(dev).t())
    out = fp8_scaled_mm_prearranged(qa.to(dev), w, torch.ones(m, 1, device=dev), torch.ones(n, device=dev),
                                    torch.float32)
    ref = (a.to(torch.int64) @ wv.to(torch.int64).t()).float()
    assert torch.equal(out.cpu(), ref)


@pytest.mark.parametrize("out_dtype", [torch.float16, torch.float32])
def test_prearranged_out_dtypes(dev, out_dtype):
    from flashrec_amd.kernel.sglops import fp8_scaled_mm, fp8_scaled_mm_prearranged, prearrange_fp8_weight

    qa, sa, qw, sw = _operands(1000, 8192, 2048, seed=5)
    a, b, sad, swd = qa.to(dev), qw.to(dev).t(), sa.to(dev), sw.to(dev)
    got = fp8_scaled_mm_prearranged(a, prearrange_fp8_weight(b), sad, swd, out_dtype)
    _same_values(got, fp8_scaled_mm(a, b, sad, swd, out_dtype))


@pytest.mark.parametrize("m,n,k", [(4096, 2048, 6144), (300, 1000, 384)])
def test_prearranged_residual_in_place(dev, m, n, k):
    from flashrec_amd.kernel.sglops import fp8_scaled_mm_prearranged, fp8_scaled_mm_residual, prearrange_fp8_weight

    qa, sa, qw, sw = _operands(m, n, k, seed=11)
    a, b, sad, swd = qa.to(dev), qw.to(dev).t(), sa.to(dev), sw.to(dev)
    r0 = torch.randn(m, n, generator=torch.Generator().manual_seed(1)).to(torch.bfloat16).to(dev)
    r1, r2 = r0.clone(), r0.clone()
    out = fp8_scaled_mm_prearranged(a, prearrange_fp8_weight(b), sad, swd, residual=r1)
    assert out.data_ptr() == r1.data_ptr()
    fp8_scaled_mm_residual(a, b, sad, swd, r2)
    _same_values(r1, r2)


@pytest.mark.parametrize("m,n,k", [(4096, 12288, 2048), (96, 512, 320)])
def test_prearranged_silu(dev, m, n, k):
    from flashrec_amd.kernel.sglops import (fp8_scaled_mm_prearranged, fp8_scaled_mm_silu, interleave_gate_up,
                                            prearrange_fp8_weight)

    qa, sa, qw, sw = _operands(m, n, k, seed=13)
    qwi, swi = interleave_gate_up(qw), interleave_gate_up(sw)
    a, b, sad, swd = qa.to(dev), qwi.to(dev).t(), sa.to(dev), swi.to(dev)
    got = fp8_scaled_mm_prearranged(a, prearrange_fp8_weight(b), sad, swd, silu=True)
    _same_values(got, fp8_scaled_mm_silu(a, b, sad, swd))


def test_prearranged_rejects_mismatched_k(dev):
    from flashrec_amd.kernel.sglops import fp8_scaled_mm_prearranged, prearrange_fp8_weight

    w = prearrange_fp8_weight(torch.zeros(256, 64, dtype=torch.float8_e4m3fn, device=dev))
    with pytest.raises(ValueError):
        fp8_scaled_mm_prearranged(torch.zeros(4, 128, dtype=torch.float8_e4m3fn, device=dev), w,
                                  torch.ones(4, 1, device=dev), torch.ones(64, device=dev))
