"""Host-side logic of the Python mirror that runs without a GPU."""

import pytest
import torch

from flashrec_amd.layers.linear import Linear, as_channel_scale


def test_channel_scale_expands_per_tensor():
    s = as_channel_scale(torch.tensor(2.0), 6)
    assert s.shape == (6,) and torch.equal(s, torch.full((6,), 2.0))
    s = as_channel_scale(torch.arange(4.0), 4)
    assert torch.equal(s, torch.arange(4.0))


def test_channel_scale_rejects_blockwise():
    """Reference tests/test_mlp.py:69-71."""
    with pytest.raises(ValueError, match="block-wise"):
        as_channel_scale(torch.ones(3), 4096)


def test_prequantized_load_keeps_column_major_view():
    lin = Linear(2048, 4096)
    lin.load(torch.empty(4096, 2048, dtype=torch.float8_e4m3fn), weight_scale=torch.tensor(0.5))
    assert lin._use_fp8
    assert tuple(lin._fp8_weight.shape) == (2048, 4096)
    assert lin._fp8_weight.stride() == (1, 2048)
    assert tuple(lin._fp8_scale.shape) == (4096,)


def test_nvfp4_load_rejected():
    """Reference tests/test_mlp.py:99-104."""
    lin = Linear(4, 4)
    with pytest.raises(NotImplementedError):
        lin.load(torch.zeros(4, 2, dtype=torch.uint8), weight_scale=torch.ones(4))


def test_unquantized_linear_is_plain_linear():
    lin = Linear(8, 4)
    w = torch.randn(4, 8)
    lin.load(w)
    x = torch.randn(3, 8)
    torch.testing.assert_close(lin(x), x @ w.t())


def test_kv_pool_slot_zero_is_dummy():
    """Reference tests/test_kv_pool.py:78-98: slot 0 is never allocated."""
    from flashrec_amd.kvcache.pool import TokenToKVPool

    pool = TokenToKVPool(1, 8, 1, 16, torch.float8_e4m3fn, torch.device("cpu"))
    assert pool.available_size() == 7
    got = pool.alloc(7)
    assert 0 not in got.tolist() and sorted(got.tolist()) == list(range(1, 8))
    assert pool.alloc(1) is None
    pool.free(torch.tensor([0, 3]))
    assert pool.available_size() == 1 and pool.alloc(1).tolist() == [3]


def test_restricted_head_validates_range():
    from flashrec_amd.logits import RestrictedLMHead

    head = RestrictedLMHead([5, 6, 7])
    with pytest.raises(ValueError):
        head.bind(torch.zeros(6, 4))
    with pytest.raises(RuntimeError):
        RestrictedLMHead([1, 2]).compute_into(torch.zeros(1, 4), torch.zeros(4, 4), torch.zeros(1, 2))


def test_bench_refuses_multi_gpu():
    import subprocess
    import sys
    from pathlib import Path

    root = Path(__file__).resolve().parents[1]
    res = subprocess.run([sys.executable, str(root / "bench.py"), "--gpus", "2"],
                         capture_output=True, text=True, timeout=120)
    assert res.returncode == 2 and "one GPU" in res.stderr


def test_scaled_mm_rejects_short_bias():
    """The GEMM epilogue reads bias[0..N): a shorter bias is refused before any launch."""
    from flashrec_amd.kernel.sglops import fp8_scaled_mm

    a = torch.zeros(4, 32, dtype=torch.float8_e4m3fn)
    b = torch.zeros(8, 32, dtype=torch.float8_e4m3fn).t()
    with pytest.raises(ValueError, match="bias"):
        fp8_scaled_mm(a, b, torch.ones(4, 1), torch.ones(8), torch.bfloat16, bias=torch.zeros(7))


def test_scaled_mm_abi_rejects_bias_length():
    """fr_fp8_scaled_mm returns FR_EINVAL for a bias length other than N (no launch)."""
    from flashrec_amd import _lib

    lib = _lib.load()
    # non-null (never dereferenced) pointers: the length check comes first
    p = 4096
    rc = lib.fr_fp8_scaled_mm(p, 32, p, 32, p, 1, p, 1, p, 7, p, 8, 4, 8, 32, 0, None)
    assert rc == _lib.FR_EINVAL


def test_silu_gemm_abi_rejects_bad_shapes():
    """fr_fp8_scaled_mm_silu: N not a multiple of 16 is FR_EINVAL, K not a
    multiple of 16 FR_EUNSUPPORTED (no scalar SiLU kernel), both before any launch."""
    from flashrec_amd import _lib

    lib = _lib.load()
    p = 4096
    assert lib.fr_fp8_scaled_mm_silu(p, 256, p, 256, p, 64, p, 248, p, 128, 64, 248, 256, None) == _lib.FR_EINVAL
    assert lib.fr_fp8_scaled_mm_silu(p, 256, p, 256, p, 64, p, 256, p, 128, 64, 256, 250, None) == \
        _lib.FR_EUNSUPPORTED


def test_log_softmax_topk_abi_checks():
    """fr_log_softmax_row_topk: bad sizes are FR_EINVAL, widths other than
    4096 / 8192 and unaligned rows FR_EUNSUPPORTED (the caller runs the two
    calls), all before any launch."""
    from flashrec_amd import _lib

    lib = _lib.load()
    p = 4096
    assert lib.fr_log_softmax_row_topk(p, 8192, 4, 0, 8, p, p, p, p, None) == _lib.FR_EINVAL
    assert lib.fr_log_softmax_row_topk(p, 100, 4, 8192, 8, p, p, p, p, None) == _lib.FR_EINVAL
    assert lib.fr_log_softmax_row_topk(p, 2000, 4, 2000, 8, p, p, p, p, None) == _lib.FR_EUNSUPPORTED
    assert lib.fr_log_softmax_row_topk(p + 4, 8192, 4, 8192, 8, p, p, p, p, None) == _lib.FR_EUNSUPPORTED
    assert lib.fr_log_softmax_row_topk(p, 8193, 4, 8192, 8, p, p, p, p, None) == _lib.FR_EUNSUPPORTED
    assert lib.fr_log_softmax_row_topk(p, 8192, 4, 8192, 2048, p, p, p, p, None) == _lib.FR_EUNSUPPORTED
    assert lib.fr_log_softmax_row_topk(p, 8192, 0, 8192, 8, p, p, p, p, None) == _lib.FR_OK


def test_silu_gemm_wrapper_checks_before_the_device():
    """fp8_scaled_mm_silu refuses wrong dtypes, mismatched K and N not a multiple of 16 before any launch."""
    from flashrec_amd.kernel.sglops import fp8_scaled_mm_silu

    a = torch.zeros(4, 32, dtype=torch.float8_e4m3fn)
    b = torch.zeros(40, 32, dtype=torch.float8_e4m3fn).t()
    with pytest.raises(ValueError, match="multiple of 16"):
        fp8_scaled_mm_silu(a, b, torch.ones(4, 1), torch.ones(40))
    with pytest.raises(TypeError):
        fp8_scaled_mm_silu(a.float(), b, torch.ones(4, 1), torch.ones(40))
    with pytest.raises(ValueError, match="shape mismatch"):
        fp8_scaled_mm_silu(a, torch.zeros(48, 16, dtype=torch.float8_e4m3fn), torch.ones(4, 1), torch.ones(16))


def test_interleave_gate_up_order():
    """Chunks of 16: 8 gate rows, then the 8 up rows of the same columns."""
    from flashrec_amd.kernel.sglops import interleave_gate_up

    n = 24
    w = torch.arange(2 * n * 3).reshape(2 * n, 3)
    got = interleave_gate_up(w)
    want = [r for c in range(n // 8) for r in list(range(8 * c, 8 * c + 8)) + list(range(n + 8 * c, n + 8 * c + 8))]
    assert torch.equal(got, w[want])
    assert torch.equal(interleave_gate_up(torch.arange(2 * n)), torch.arange(2 * n)[want])
    assert torch.equal(interleave_gate_up(w.t().contiguous(), dim=1), w[want].t())
    with pytest.raises(ValueError):
        interleave_gate_up(torch.zeros(40, 2))


def test_log_softmax_rejects_mismatched_out():
    from flashrec_amd.kernel.sglops import log_softmax_f32

    logits = torch.zeros(4, 16)
    for bad in (torch.zeros(4, 8), torch.zeros(4, 16, dtype=torch.float16), torch.zeros(16, 4).t()):
        with pytest.raises(ValueError):
            log_softmax_f32(logits, out=bad)


def test_linear_rejects_wrong_bias_and_rows():
    lin = Linear(8, 4)
    with pytest.raises(ValueError):
        lin.load(torch.randn(4, 8), bias=torch.zeros(3))
    with pytest.raises(ValueError):
        lin.load(torch.randn(5, 8))


def test_linear_codes_move_with_module():
    lin = Linear(16, 8)
    lin.load(torch.zeros(8, 16, dtype=torch.float8_e4m3fn), weight_scale=torch.arange(8.0))
    assert set(dict(lin.named_buffers())) == {"w_codes", "w_scale"}
    lin = lin.to(torch.bfloat16)  # a float cast keeps the codes and scales as they are
    assert lin._fp8_weight.dtype == torch.float8_e4m3fn and lin._fp8_scale.dtype == torch.float32
    assert torch.equal(lin._fp8_scale, torch.arange(8.0))


def test_kv_pool_free_and_realloc_order():
    """LIFO reuse: the last freed ids come back first, in the order freed."""
    from flashrec_amd.kvcache.pool import TokenToKVPool

    pool = TokenToKVPool(1, 10, 1, 8, torch.bfloat16, torch.device("cpu"))
    a = pool.alloc(4)
    assert a.tolist() == [6, 7, 8, 9] and pool.last_alloc_cpu == [6, 7, 8, 9]
    pool.free([7, 0, -1, 9])
    assert pool.available_size() == 7
    assert pool.alloc(2).tolist() == [7, 9]
    assert pool.alloc(0).numel() == 0 and pool.last_alloc_cpu == []
    assert pool.alloc(100) is None
    with pytest.raises(TypeError):
        TokenToKVPool(1, 4, 1, 8, torch.float16, torch.device("cpu"))


def test_pinned_upload_ring_reuses_regions():
    """The upload ring wraps and retires the copies whose regions it reuses (CPU-side logic)."""
    from flashrec_amd.kvcache.pool import _PinnedUpload

    class _Ev:
        def __init__(self):
            self.waited = False

        def synchronize(self):
            self.waited = True

    up = _PinnedUpload(torch.device("cpu"), capacity=16)
    up._host = torch.empty(16, dtype=torch.int64)
    evs = []
    for n in (6, 6, 3):
        start = up._reserve(n)
        ev = _Ev()
        evs.append(ev)
        up._inflight.append((start, start + n, ev))
    assert [r[:2] for r in up._inflight] == [(0, 6), (6, 12), (12, 15)]
    start = up._reserve(5)  # does not fit at 15: wraps to 0 and retires (0, 6) only
    assert start == 0 and evs[0].waited and not evs[1].waited and not evs[2].waited
    start = up._reserve(4)  # [5, 9) meets (6, 12)
    assert start == 5 and evs[1].waited and not evs[2].waited


def test_req_to_token_pool_contract():
    """ReqToTokenPool (python/flashrec/kvcache/pool.py:148-182): an int32
    [max_reqs, max_seq_len] table, row 0 never handed out, rows taken from
    the top of the free list and returned in order."""
    from flashrec_amd.kvcache import ReqToTokenPool

    pool = ReqToTokenPool(6, 32, torch.device("cpu"))
    assert pool.req_to_token.shape == (6, 32) and pool.req_to_token.dtype == torch.int32
    assert not pool.req_to_token.any()
    assert pool.available_size() == 5
    got = pool.alloc(2)
    assert got.dtype == torch.int64 and got.tolist() == [4, 5] and pool.last_alloc_cpu == [4, 5]
    assert pool.alloc(4) is None and pool.last_alloc_cpu == []
    assert pool.alloc(0).numel() == 0
    pool.free(torch.tensor([0, 5, -1]))
    assert pool.available_size() == 4
    assert pool.alloc(1).tolist() == [5]
    assert sorted(pool.alloc(3).tolist()) == [1, 2, 3] and pool.available_size() == 0


def test_kvcache_module_exports_both_pools():
    import flashrec_amd.kvcache as kv
    from flashrec_amd.kvcache import pool

    assert kv.ReqToTokenPool is pool.ReqToTokenPool and kv.TokenToKVPool is pool.TokenToKVPool


def test_row_kernels_refuse_other_dtypes_before_launch():
    """bf16, fp16 and fp32 activations are taken (fp32 without intermediate
    rounding, as the reference's CPU composition); other dtypes raise
    TypeError before any device work, and host tensors of a taken dtype raise
    the no-CPU-path error (there is no fallback)."""
    from flashrec_amd.kernel.rms_fp8 import (fused_add_rmsnorm_per_token_quant_fp8,
                                             rmsnorm_per_token_quant_fp8)
    from flashrec_amd.kernel.silu_fp8 import silu_and_mul_per_token_quant_fp8

    w = torch.ones(8, dtype=torch.bfloat16)
    x64 = torch.ones(2, 8, dtype=torch.float64)
    with pytest.raises(TypeError):
        rmsnorm_per_token_quant_fp8(x64, w, 1e-6)
    with pytest.raises(TypeError):
        fused_add_rmsnorm_per_token_quant_fp8(torch.ones(2, 8), torch.ones(2, 8, dtype=torch.bfloat16), w, 1e-6)
    with pytest.raises(TypeError):
        silu_and_mul_per_token_quant_fp8(x64)
    for dt in (torch.bfloat16, torch.float16, torch.float32):
        with pytest.raises(RuntimeError, match="no CPU path"):
            rmsnorm_per_token_quant_fp8(torch.ones(2, 8, dtype=dt), w, 1e-6)
        with pytest.raises(RuntimeError, match="no CPU path"):
            silu_and_mul_per_token_quant_fp8(torch.ones(2, 8, dtype=dt))


def test_rotary_embedding_refuses_odd_head():
    from flashrec_amd.kernel.sglops import rope_inplace_any

    with pytest.raises((ValueError, RuntimeError)):
        rope_inplace_any(torch.zeros(2, dtype=torch.int64), torch.zeros(2, 6), torch.zeros(2, 6), 3,
                         torch.zeros(4, 3))
