"""Pins for oracle.paged_attention that do not restate its formula: closed
forms of softmax attention, the grouped-query head mapping, and torch's own
scaled_dot_product_attention (an independent implementation), both in fp32 and
in the reference's bf16 call sequence (flashinfer.py:380-431)."""

import pytest
import torch
import torch.nn.functional as F

from oracle import ops

E4M3 = torch.float8_e4m3fn


def _pool(slots, hk, d, seed):
    g = torch.Generator().manual_seed(seed)
    k = (torch.randn(slots, hk, d, generator=g)).to(E4M3)
    v = (torch.randn(slots, hk, d, generator=g)).to(E4M3)
    return k, v


def _decode_plan(lens, slots, seed):
    g = torch.Generator().manual_seed(seed)
    idx = [torch.randint(1, slots, (n,), generator=g, dtype=torch.int32) for n in lens]
    kv_indices = torch.cat(idx) if idx else torch.empty(0, dtype=torch.int32)
    indptr = torch.zeros(len(lens) + 1, dtype=torch.int32)
    indptr[1:] = torch.cumsum(torch.tensor(lens, dtype=torch.int32), 0)
    return kv_indices, indptr


def test_single_key_returns_its_value():
    k, v = _pool(8, 2, 128, 0)
    q = torch.randn(3, 4, 128, generator=torch.Generator().manual_seed(12)).to(torch.bfloat16)
    idx = torch.tensor([5, 2, 7], dtype=torch.int32)
    start = torch.tensor([0, 1, 2], dtype=torch.int32)
    ln = torch.ones(3, dtype=torch.int32)
    out = ops.paged_attention(q, k, v, idx, start, ln, 128 ** -0.5)
    for t, slot in enumerate([5, 2, 7]):
        for h in range(4):
            assert torch.equal(out[t, h], v[slot, h // 2].float().to(torch.bfloat16))


def test_identical_keys_give_the_mean_value():
    """All keys equal -> uniform weights -> mean of V (any q)."""
    k, v = _pool(16, 1, 128, 1)
    k[:] = k[3]
    q = torch.randn(1, 2, 128, generator=torch.Generator().manual_seed(13)).to(torch.bfloat16) * 5
    idx = torch.arange(1, 11, dtype=torch.int32)
    out = ops.paged_attention(q, k, v, idx, torch.tensor([0], dtype=torch.int32),
                              torch.tensor([10], dtype=torch.int32), 0.3)
    mean = v[1:11, 0].double().mean(0)
    for h in range(2):
        assert torch.allclose(out[0, h].double(), mean, rtol=2 ** -8, atol=1e-6)


def test_zero_query_is_uniform():
    k, v = _pool(32, 2, 128, 2)
    q = torch.zeros(1, 2, 128, dtype=torch.bfloat16)
    idx = torch.tensor([4, 9, 4, 17, 30], dtype=torch.int32)  # a repeated slot counts twice
    out = ops.paged_attention(q, k, v, idx, torch.tensor([0], dtype=torch.int32),
                              torch.tensor([5], dtype=torch.int32), 1.0)
    for h in range(2):
        mean = v[idx.long(), h].double().mean(0)
        assert torch.allclose(out[0, h].double(), mean, rtol=2 ** -8, atol=1e-6)


def test_dominant_key_wins():
    """A key aligned with q at a huge score takes all the weight."""
    k, v = _pool(8, 1, 128, 3)
    q = torch.zeros(1, 1, 128)
    q[0, 0, 0] = 1.0
    k = k.float()
    k[:, :, 0] = 0.0
    k[6, 0, 0] = 448.0
    k = k.to(E4M3)
    out = ops.paged_attention(q.to(torch.bfloat16), k, v, torch.arange(8, dtype=torch.int32),
                              torch.tensor([0], dtype=torch.int32), torch.tensor([8], dtype=torch.int32), 1.0)
    assert torch.equal(out[0, 0], v[6, 0].float().to(torch.bfloat16))


def test_grouped_query_heads_use_their_kv_head():
    """Query head h reads kv head h // (Hq/Hk): with one key, each output equals
    that kv head's value row (kv heads made distinct)."""
    hq, hk = 8, 2
    k, v = _pool(4, hk, 128, 4)
    v[:, 1] = (-v[:, 0].float()).to(E4M3)
    q = torch.randn(1, hq, 128, generator=torch.Generator().manual_seed(14)).to(torch.bfloat16)
    out = ops.paged_attention(q, k, v, torch.tensor([3], dtype=torch.int32),
                              torch.tensor([0], dtype=torch.int32), torch.tensor([1], dtype=torch.int32), 0.1)
    for h in range(hq):
        assert torch.equal(out[0, h], v[3, h // 4].float().to(torch.bfloat16))


@pytest.mark.parametrize("hq,hk", [(16, 8), (4, 4), (8, 1)])
def test_matches_torch_sdpa_fp32(hq, hk):
    """torch's SDPA (math, fp32) over the same gathered rows, rounded to bf16 once."""
    lens = [1, 5, 64, 130]
    k, v = _pool(512, hk, 128, 5)
    idx, indptr = _decode_plan(lens, 512, 6)
    q = torch.randn(len(lens), hq, 128, generator=torch.Generator().manual_seed(hq * 10 + hk)).to(torch.bfloat16)
    out = ops.paged_attention(q, k, v, idx, indptr[:-1].contiguous(), torch.tensor(lens, dtype=torch.int32),
                              128 ** -0.5)
    for i, n in enumerate(lens):
        sl = idx[indptr[i]:indptr[i + 1]].long()
        kk = k[sl].float().permute(1, 0, 2).repeat_interleave(hq // hk, 0)  # [Hq, n, D]
        vv = v[sl].float().permute(1, 0, 2).repeat_interleave(hq // hk, 0)
        ref = F.scaled_dot_product_attention(q[i].float()[:, None, :], kk, vv, scale=128 ** -0.5)[:, 0]
        got = out[i].float()
        exp = ref.to(torch.bfloat16).float()
        # equal except one-ulp bf16 rounding flips (fp32 summation order) on a
        # few elements
        flips = got != exp
        assert ((got - exp).abs() <= 2.0 ** -7 * exp.abs() + 1e-30).all()
        assert flips.float().mean().item() < 0.02


def test_matches_reference_bf16_call_sequence():
    """The reference's decode fallback (bf16 gather + SDPA) agrees to bf16
    rounding of its intermediate probabilities (max-abs normalised 1e-2)."""
    lens = [3, 17, 129]
    k, v = _pool(256, 8, 128, 7)
    idx, indptr = _decode_plan(lens, 256, 8)
    q = torch.randn(len(lens), 16, 128, generator=torch.Generator().manual_seed(11)).to(torch.bfloat16)
    ours = ops.paged_attention(q, k, v, idx, indptr[:-1].contiguous(), torch.tensor(lens, dtype=torch.int32),
                               128 ** -0.5).float()
    ref = ops.sdpa_reference_style(q, k, v, idx, indptr).float()
    assert ((ours - ref).abs().max() / ref.abs().max()).item() < 1e-2


def test_empty_row_is_zero():
    k, v = _pool(4, 1, 128, 9)
    out = ops.paged_attention(torch.ones(1, 1, 128, dtype=torch.bfloat16), k, v,
                              torch.empty(0, dtype=torch.int32), torch.zeros(1, dtype=torch.int32),
                              torch.zeros(1, dtype=torch.int32), 1.0)
    assert torch.count_nonzero(out) == 0
