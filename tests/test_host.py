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
