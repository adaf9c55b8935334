"""The W8A8 GEMM with the residual add in its epilogue
(``fp8_scaled_mm_residual`` -> ``fr_fp8_scaled_mm_residual``).

Bar: bit-exact against the two steps it replaces: ``fp8_scaled_mm`` (held to
the fp32 dequantised oracle in test_gpu_gemm.py) rounded to the residual's
dtype, then the residual add in that dtype (torch's bf16 / fp16 add, which
rounds the fp32 sum once: the reference's ``residual + x``,
sglops.py:53-55).  Covered: the decode step's o and down shapes (the
256 x 128 tile's fast epilogue), edge tiles and tails (the bounds-checked
path), the 256 x 256 tile (which routes the add through the bounds-checked
path), the 192 x 128 and 128 x 128 tiles and several tiles per workgroup
(M = 512, 1381 and 2661 rows), fp16, in place and into a separate buffer, a
strided residual."""

import pytest
import torch

from oracle import ops

pytestmark = pytest.mark.gpu


def _operands(m, n, k, seed, dtype=torch.bfloat16):
    g = torch.Generator().manual_seed(seed)
    x = torch.randn(m, k, generator=g).to(torch.bfloat16)
    w = (0.02 * torch.randn(n, k, generator=g)).to(torch.bfloat16)
    qa, sa = ops.per_token_quant_fp8(x)
    qw, sw = ops.quantize_weight_fp8(w)
    res = (torch.randn(m, n, generator=g) * 3).to(dtype)
    return qa, sa, qw, sw, res


def _two_steps(dev, qa, sa, qw, sw, res):
    from flashrec_amd.kernel.sglops import fp8_scaled_mm

    prod = fp8_scaled_mm(qa.to(dev), qw.to(dev).t(), sa.to(dev), sw.to(dev), res.dtype)
    return res.to(dev) + prod


def _bits(t):
    return t.contiguous().view(torch.int16).cpu()


def _assert_same(got, ref, label=""):
    g, r = _bits(got), _bits(ref)
    bad = (g != r).nonzero()
    if bad.numel():
        idx = [tuple(int(v) for v in bad[i]) for i in range(min(5, bad.shape[0]))]
        gf, rf = got.float().cpu(), ref.float().cpu()
        ex = [(i, float(gf[i]), float(rf[i])) for i in idx]
        raise AssertionError(f"{label}: {bad.shape[0]} of {g.numel()} differ, e.g. {ex}")


@pytest.mark.parametrize("m,n,k", [(4096, 2048, 2048), (4096, 2048, 6144), (300, 520, 384), (33, 100, 256),
                                   (4096 + 100, 2048 + 64, 2048), (512, 2048, 1040), (1, 256, 2048),
                                   (512, 12288, 2048), (1381, 12352, 2048), (2661, 6144, 2048)])
def test_residual_in_place_matches_two_steps(dev, m, n, k):
    from flashrec_amd.kernel.sglops import fp8_scaled_mm_residual

    qa, sa, qw, sw, res = _operands(m, n, k, seed=m + n + k)
    ref = _two_steps(dev, qa, sa, qw, sw, res)
    stream = res.to(dev)
    got = fp8_scaled_mm_residual(qa.to(dev), qw.to(dev).t(), sa.to(dev), sw.to(dev), stream)
    assert got.data_ptr() == stream.data_ptr()
    _assert_same(got, ref)


def test_residual_256x256_tile_and_fp16(dev):
    """4096 x 12288 takes the 256 x 256 tile, whose residual add runs in the
    bounds-checked epilogue; fp16 residual stream."""
    from flashrec_amd.kernel.sglops import fp8_scaled_mm_residual

    qa, sa, qw, sw, res = _operands(4096, 12288, 2048, seed=5, dtype=torch.float16)
    ref = _two_steps(dev, qa, sa, qw, sw, res)
    got = fp8_scaled_mm_residual(qa.to(dev), qw.to(dev).t(), sa.to(dev), sw.to(dev), res.to(dev))
    _assert_same(got, ref)


def test_residual_into_separate_strided_buffers(dev):
    """Residual a column slice of a wider buffer; out another one; the
    residual itself is left unchanged."""
    from flashrec_amd.kernel.sglops import fp8_scaled_mm_residual

    m, n, k = 4096, 2048, 2048
    qa, sa, qw, sw, res = _operands(m, n, k, seed=7)
    ref = _two_steps(dev, qa, sa, qw, sw, res)
    wide = torch.zeros(m, n + 256, dtype=torch.bfloat16, device=dev)
    wide[:, 128:128 + n] = res.to(dev)
    rv = wide[:, 128:128 + n]
    out = torch.empty(m, n + 64, dtype=torch.bfloat16, device=dev)[:, :n]
    got = fp8_scaled_mm_residual(qa.to(dev), qw.to(dev).t(), sa.to(dev), sw.to(dev), rv, out=out)
    assert got.data_ptr() == out.data_ptr()
    _assert_same(got, ref)
    assert torch.equal(_bits(rv), _bits(res))


def test_residual_boundary_checks(dev):
    from flashrec_amd import _lib
    from flashrec_amd.kernel.sglops import fp8_scaled_mm_residual

    qa, sa, qw, sw, res = _operands(64, 256, 128, seed=9)
    a, b, s_a, s_b = qa.to(dev), qw.to(dev).t(), sa.to(dev), sw.to(dev)
    with pytest.raises(TypeError):
        fp8_scaled_mm_residual(a, b, s_a, s_b, res.float().to(dev))
    with pytest.raises(ValueError):
        fp8_scaled_mm_residual(a, b, s_a, s_b, res[:, :128].contiguous().to(dev))
    r = res.to(dev)
    st = torch.cuda.current_stream().cuda_stream
    lib = _lib.load()
    # fp32 outputs are not taken; a short residual stride is refused
    assert lib.fr_fp8_scaled_mm_residual(a.data_ptr(), 128, b.data_ptr(), 128, s_a.data_ptr(), 64, s_b.data_ptr(),
                                         256, r.data_ptr(), 256, r.data_ptr(), 256, 64, 256, 128,
                                         _lib.DTYPE_CODE[torch.float32], st) == _lib.FR_EUNSUPPORTED
    assert lib.fr_fp8_scaled_mm_residual(a.data_ptr(), 128, b.data_ptr(), 128, s_a.data_ptr(), 64, s_b.data_ptr(),
                                         256, r.data_ptr(), 200, r.data_ptr(), 256, 64, 256, 128,
                                         _lib.DTYPE_CODE[torch.bfloat16], st) == _lib.FR_EINVAL


def test_residual_at_addresses_with_bit31_set(dev):
    """Regression: the residual's per-wave base address is split into two
    32-bit words; a low word with bit 31 set once sign-extended into the high
    word.  Place the residual (and the output) where every row's address has
    bit 31 of its low word set."""
    from flashrec_amd.kernel.sglops import fp8_scaled_mm_residual

    m, n, k = 4096, 2048, 2048
    qa, sa, qw, sw, res = _operands(m, n, k, seed=13)
    ref = _two_steps(dev, qa, sa, qw, sw, res)
    need = m * n * 2
    pool = torch.empty((1 << 31) + 2 * need, dtype=torch.uint8, device=dev)
    base = pool.data_ptr()
    off = 0
    while not ((base + off) & 0x80000000 and (base + off + need - 1) & 0x80000000):
        off += 1 << 24
    assert off + need <= pool.numel()
    stream = pool[off: off + need].view(torch.bfloat16).view(m, n)
    stream.copy_(res.to(dev))
    got = fp8_scaled_mm_residual(qa.to(dev), qw.to(dev).t(), sa.to(dev), sw.to(dev), stream)
    _assert_same(got, ref)
    del pool, stream
    torch.cuda.empty_cache()
