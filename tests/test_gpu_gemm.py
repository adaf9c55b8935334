"""Parity of the W8A8 fp8 GEMM with the fp32 dequantised-matmul oracle.

Acceptance: bf16 outputs within 1e-2 of the oracle, relative to the
output's max |value| (max-abs normalised).  Integer-valued operands with
unit scales make the product exact, which pins the accumulation itself.
"""

import pytest
import torch

from helpers import max_abs_rel
from oracle import inputs, ops

pytestmark = pytest.mark.gpu

TOL = 1e-2


def _operands(m, n, k, seed):
    g = torch.Generator().manual_seed(seed)
    x = torch.randn(m, k, generator=g).to(torch.bfloat16)
    w = (0.02 * torch.randn(n, k, generator=g)).to(torch.bfloat16)
    qa, sa = ops.per_token_quant_fp8(x)
    qw, sw = ops.quantize_weight_fp8(w)
    return qa, sa, qw, sw


def _run(dev, qa, sa, qw, sw, out_dtype=torch.bfloat16, bias=None):
    from flashrec_amd.kernel.sglops import fp8_scaled_mm

    b = qw.to(dev).t()  # [K, N] column-major view, as Linear keeps it
    return fp8_scaled_mm(qa.to(dev), b, sa.to(dev), sw.to(dev), out_dtype,
                         None if bias is None else bias.to(dev))


@pytest.mark.parametrize("m,n,k", [(4, 128, 64), (1, 256, 2048), (33, 100, 256), (300, 520, 384),
                                   (128, 128, 128), (512, 4096, 2048), (256, 2048, 6144),
                                   (64, 8192, 2048), (17, 48, 48)])
def test_gemm_vs_dequant_oracle(dev, m, n, k):
    qa, sa, qw, sw = _operands(m, n, k, seed=m + n + k)
    out = _run(dev, qa, sa, qw, sw)
    assert out.dtype == torch.bfloat16 and out.shape == (m, n)
    ref = ops.fp8_scaled_mm(qa, qw.t(), sa, sw)
    assert max_abs_rel(out, ref) < TOL


def test_gemm_integer_exact(dev):
    """Small-integer e4m3 operands, unit scales, fp32 out: the product is exact."""
    g = torch.Generator().manual_seed(0)
    m, n, k = 256, 512, 1024
    a = torch.randint(-4, 5, (m, k), generator=g).float()
    w = torch.randint(-4, 5, (n, k), generator=g).float()
    qa, qw = a.to(torch.float8_e4m3fn), w.to(torch.float8_e4m3fn)
    one_m = torch.ones(m, 1)
    one_n = torch.ones(n)
    out = _run(dev, qa, one_m, qw, one_n, out_dtype=torch.float32)
    ref = (a.to(torch.int64) @ w.to(torch.int64).t()).float()
    assert torch.equal(out.cpu(), ref)


def test_gemm_onehot_columns(dev):
    """One-hot K rows pick single products: catches transposed / shifted operands."""
    m, n, k = 64, 256, 256
    a = torch.zeros(m, k)
    a[torch.arange(m), (torch.arange(m) * 7) % k] = 1.0
    w = torch.arange(n * k, dtype=torch.float32).reshape(n, k) % 13 - 6
    qa, qw = a.to(torch.float8_e4m3fn), w.to(torch.float8_e4m3fn)
    sa = torch.full((m, 1), 0.5)
    sw = torch.linspace(1, 2, n)
    out = _run(dev, qa, sa, qw, sw, out_dtype=torch.float32)
    ref = ops.fp8_scaled_mm(qa, qw.t(), sa, sw)
    assert torch.equal(out.cpu(), ref)


@pytest.mark.parametrize("out_dtype", [torch.float16, torch.float32])
def test_gemm_out_dtypes_and_bias(dev, out_dtype):
    qa, sa, qw, sw = _operands(96, 640, 512, seed=4)
    bias = torch.randn(640).to(out_dtype)
    out = _run(dev, qa, sa, qw, sw, out_dtype=out_dtype, bias=bias)
    assert out.dtype == out_dtype
    ref = ops.fp8_scaled_mm(qa, qw.t(), sa, sw, bias=bias.float())
    assert max_abs_rel(out, ref) < TOL


def test_gemm_per_tensor_scales(dev):
    qa, _, qw, _ = _operands(40, 200, 256, seed=6)
    sa = torch.tensor([0.25])
    sw = torch.tensor([3.0])
    out = _run(dev, qa, sa, qw, sw)
    ref = ops.fp8_scaled_mm(qa, qw.t(), sa, sw)
    assert max_abs_rel(out, ref) < TOL


@pytest.mark.parametrize("m,n,k", [(9, 70, 40), (300, 520, 1000), (64, 256, 2056)])
def test_gemm_odd_k_is_padded_for_mfma(dev, m, n, k):
    """K not a multiple of 16: the wrapper zero-pads K and runs the MFMA kernel."""
    qa, sa, qw, sw = _operands(m, n, k, seed=8 + k)
    out = _run(dev, qa, sa, qw, sw, out_dtype=torch.float32)
    ref = ops.fp8_scaled_mm(qa, qw.t(), sa, sw)
    # fp32 outputs: only the order of the scaling against the sum differs
    assert max_abs_rel(out, ref) < 1e-4


def test_gemm_unaligned_views_are_repacked(dev):
    """Operand views at odd byte offsets / row strides reach the MFMA kernel as aligned copies."""
    from flashrec_amd.kernel.sglops import fp8_scaled_mm

    qa, sa, qw, sw = _operands(33, 96, 256, seed=12)
    wide = torch.zeros(33, 256 + 3, dtype=torch.uint8, device=dev)
    wide[:, 3:] = qa.view(torch.uint8).to(dev)
    a_view = wide[:, 3:].view(torch.float8_e4m3fn)  # row stride 259, data at +3 bytes
    out = fp8_scaled_mm(a_view, qw.to(dev).t(), sa.to(dev), sw.to(dev), torch.float32)
    ref = ops.fp8_scaled_mm(qa, qw.t(), sa, sw)
    assert max_abs_rel(out, ref) < 1e-4


def test_gemm_scalar_kernel_through_the_c_abi(dev):
    """A C caller passing K % 16 != 0 gets the library's scalar kernel (the
    Python wrapper never sends it there); same result."""
    from flashrec_amd import _lib

    m, n, k = 9, 70, 40
    qa, sa, qw, sw = _operands(m, n, k, seed=8)
    a, w, s_a, s_w = qa.to(dev), qw.to(dev), sa.to(dev).reshape(-1), sw.to(dev)
    out = torch.empty(m, n, dtype=torch.float32, device=dev)
    rc = _lib.load().fr_fp8_scaled_mm(a.data_ptr(), k, w.data_ptr(), k, s_a.data_ptr(), m, s_w.data_ptr(), n,
                                      None, 0, out.data_ptr(), n, m, n, k, 2,
                                      torch.cuda.current_stream(dev).cuda_stream)
    assert rc == _lib.FR_OK
    ref = ops.fp8_scaled_mm(qa, qw.t(), sa, sw)
    assert max_abs_rel(out, ref) < 1e-5


def test_gemm_row_major_b_is_copied(dev):
    from flashrec_amd.kernel.sglops import fp8_scaled_mm

    qa, sa, qw, sw = _operands(16, 64, 128, seed=2)
    b_rowmajor = qw.t().contiguous().to(dev)  # [K, N] row-major
    out = fp8_scaled_mm(qa.to(dev), b_rowmajor, sa.to(dev), sw.to(dev), torch.bfloat16)
    ref = ops.fp8_scaled_mm(qa, qw.t(), sa, sw)
    assert max_abs_rel(out, ref) < TOL


def _all_rows_rel(out, qa, sa, qw, sw, chunk=1024):
    """max |out - oracle| / max |oracle| over every row, the oracle evaluated
    in row chunks (fp32 dequantised matmul)."""
    out = out.cpu().float()
    b = qw.float() * sw.reshape(-1, 1).float()  # [N, K]
    err, peak = 0.0, 0.0
    for r0 in range(0, out.shape[0], chunk):
        a = qa[r0:r0 + chunk].float() * sa[r0:r0 + chunk].reshape(-1, 1).float()
        ref = a @ b.t()
        err = max(err, (out[r0:r0 + chunk] - ref).abs().max().item())
        peak = max(peak, ref.abs().max().item())
    return err / peak


def test_gemm_config1_full_size_rows(dev):
    """Config 1 at M=4096 (gate_up, K=2048, N=12288, the headline shape):
    every row against the oracle, plus agreement of a row sample with the
    reference's literal torch._scaled_mm CPU branch."""
    x, gamma, eps = inputs.config0(m=4096)
    qa, sa = ops.rmsnorm_per_token_quant_fp8(x, gamma, eps)
    qw, sw = ops.quantize_weight_fp8(inputs.config1_weight())
    out = _run(dev, qa, sa, qw, sw)
    assert torch.isfinite(out).all()
    rel = _all_rows_rel(out, qa, sa, qw, sw)
    print(f"config1 M=4096 all rows: max-abs-normalised error {rel:.2e}")
    assert rel < TOL
    rows = torch.randperm(4096, generator=torch.Generator().manual_seed(1))[:64]
    lit = ops.fp8_scaled_mm_torch_cpu(qa[rows], qw.t(), sa[rows], sw, torch.bfloat16)
    assert max_abs_rel(out.cpu()[rows], lit.float()) < TOL


def test_gemm_config1_m512_all_rows(dev):
    """Config 1 at its primary size, M=512 (the 192x128 one-round tiles)."""
    x, gamma, eps = inputs.config0(m=512)
    qa, sa = ops.rmsnorm_per_token_quant_fp8(x, gamma, eps)
    qw, sw = ops.quantize_weight_fp8(inputs.config1_weight())
    out = _run(dev, qa, sa, qw, sw)
    rel = _all_rows_rel(out, qa, sa, qw, sw)
    print(f"config1 M=512 all rows: {rel:.2e}")
    assert rel < TOL


def test_gemm_config2_down_all_rows(dev):
    """Config 2: SiLU->fp8 of the seeded [4096, 12288] input, then the down
    GEMM (K=6144, N=2048) at exactly that shape, every row."""
    x, w = inputs.config2()
    qa, sa = ops.silu_and_mul_per_token_quant_fp8(x)
    qw, sw = ops.quantize_weight_fp8(w)
    out = _run(dev, qa, sa, qw, sw)
    rel = _all_rows_rel(out, qa, sa, qw, sw)
    print(f"config2 down 4096x2048x6144 all rows: {rel:.2e}")
    assert rel < TOL


@pytest.mark.parametrize("name,n,k", [("qkv", 4096, 2048), ("o", 2048, 2048)])
def test_gemm_config4_shapes_all_rows(dev, name, n, k):
    """The config-4 decode-step projections at their exact 4096-row shapes."""
    qa, sa, qw, sw = _operands(4096, n, k, seed=n + 3 * k)
    out = _run(dev, qa, sa, qw, sw)
    rel = _all_rows_rel(out, qa, sa, qw, sw)
    print(f"config4 {name} 4096x{n}x{k} all rows: {rel:.2e}")
    assert rel < TOL


@pytest.mark.parametrize("out_dtype", [torch.bfloat16, torch.float32, torch.float16])
@pytest.mark.parametrize("m,n,k", [(4096 + 100, 12288, 2048), (2661, 6144, 2048), (1381, 12352, 2048),
                                   (3685, 2176, 2048)])
def test_gemm_multi_tile_edges(dev, m, n, k, out_dtype):
    """Several tiles per workgroup with edge tiles among them, on each tile
    shape (the tile choice gives these 256x256 in 4 rounds, 256x128 in 2,
    192x128 in 3 with a partial last column tile, 128x128 in 2): after a
    partial tile's epilogue the next tile's first waits must not assume the
    full tile's store count (and after a full one they may).  Seeded rows,
    including every row of the last (partial) m-tile, against the oracle."""
    qa, sa, qw, sw = _operands(m, n, k, seed=m + n)
    out = _run(dev, qa, sa, qw, sw, out_dtype=out_dtype).cpu()
    g = torch.Generator().manual_seed(5)
    rows = torch.cat([torch.randperm(m, generator=g)[:48], torch.arange(m - 40, m)])
    ref = ops.fp8_scaled_mm(qa[rows], qw.t(), sa[rows], sw)
    got = out[rows].float()
    assert max_abs_rel(got, ref) < TOL
    assert torch.isfinite(out).all()


@pytest.mark.parametrize("m,n,k", [(1637, 12288, 2064), (2624, 6144, 1088), (1344, 12288, 2112),
                                   (3648, 2112, 1040), (4096, 2048, 1088), (512, 12288, 2112)])
def test_gemm_k_tail_multi_tile(dev, m, n, k):
    """K not a multiple of the 128-byte ring rows (K % 128 = 16, 64, 64, 16)
    on shapes that give workgroups several tiles of each shape (256x256 in 2
    rounds, 256x128 in 2, 192x128 in 3, 128x128 in 2) and on two one-round
    shapes: the zero-filled tail of each tile's last slot must not leak into
    the next tile's first slots."""
    qa, sa, qw, sw = _operands(m, n, k, seed=k)
    out = _run(dev, qa, sa, qw, sw).cpu()
    g = torch.Generator().manual_seed(6)
    rows = torch.cat([torch.randperm(m, generator=g)[:48], torch.arange(m - 16, m)])
    ref = ops.fp8_scaled_mm(qa[rows], qw.t(), sa[rows], sw)
    assert max_abs_rel(out[rows].float(), ref) < TOL
    assert torch.isfinite(out).all()


@pytest.mark.parametrize("out_dtype", [torch.bfloat16, torch.float32])
@pytest.mark.parametrize("m,n,k", [(512, 12288, 2048), (512, 12200, 2048), (500, 12288, 1040)])
def test_gemm_192_column_tiles(dev, m, n, k, out_dtype):
    """The 192 x 128 tile (taken when it gives every CU one tile, e.g. 512
    rows x 12288): full tiles, a partial last column tile, a partial last row
    tile and a K tail."""
    qa, sa, qw, sw = _operands(m, n, k, seed=n + k)
    out = _run(dev, qa, sa, qw, sw, out_dtype=out_dtype).cpu()
    g = torch.Generator().manual_seed(7)
    rows = torch.cat([torch.randperm(m, generator=g)[:32], torch.arange(m - 16, m)])
    ref = ops.fp8_scaled_mm(qa[rows], qw.t(), sa[rows], sw)
    assert max_abs_rel(out[rows].float(), ref) < TOL
    assert torch.isfinite(out).all()


@pytest.mark.parametrize("m,n,k,out_dtype", [
    (4100, 136, 2064, torch.bfloat16),   # narrow N, K tail, ragged M
    (1023, 2048, 1040, torch.float16),
    (500, 12200, 256, torch.bfloat16),   # 192-column tiles, ragged N
    (2048, 1000, 6144, torch.float32),
    (64, 4096, 2048, torch.bfloat16),
    (7, 48, 16, torch.float32),
])
def test_gemm_integer_exact_pow2_scales(dev, m, n, k, out_dtype):
    """Small-integer operands with power-of-two row/column scales: every product,
    sum and scaling step is exact in fp32, so the output must equal the exact
    result rounded once to the output type, for every tile shape and dtype."""
    g = torch.Generator().manual_seed(m * 7 + n + k)
    a = torch.randint(-3, 4, (m, k), generator=g).double()
    w = torch.randint(-3, 4, (n, k), generator=g).double()
    sa = torch.exp2(torch.randint(-6, 2, (m, 1), generator=g).double())
    sw = torch.exp2(torch.randint(-6, 2, (n,), generator=g).double())
    if out_dtype == torch.float16:
        sa = sa * 2.0 ** -6  # keep |out| inside fp16's range
    qa, qw = a.float().to(torch.float8_e4m3fn), w.float().to(torch.float8_e4m3fn)
    out = _run(dev, qa, sa.float(), qw, sw.float(), out_dtype=out_dtype)
    ref = ((a @ w.t()) * sa * sw[None, :]).to(out_dtype)
    assert torch.equal(out.cpu(), ref)


@pytest.mark.parametrize("m,n,k", [(4096, 12288, 2048), (4096, 2048, 2048), (512, 12288, 2048), (300, 520, 384)])
def test_gemm_16bit_outputs_round_the_fp32_product(dev, m, n, k):
    """bf16 / fp16 outputs are the fp32 output rounded once more (torch's
    ``(out.float() * sa * sb).to(dtype)``, sglops.py:111-139): bit-exact on
    the 256x256, 256x128 and 192x128 tiles and on edge tiles.  (The compiler
    once folded the last fp32 multiply into the fp16 conversion, one rounding
    instead of two, which differed at fp16 halfway points.)"""
    qa, sa, qw, sw = _operands(m, n, k, seed=m + k)
    f32 = _run(dev, qa, sa, qw, sw, torch.float32)
    for dt in (torch.bfloat16, torch.float16):
        got = _run(dev, qa, sa, qw, sw, dt)
        assert torch.equal(got.view(torch.int16).cpu(), f32.to(dt).view(torch.int16).cpu()), dt
