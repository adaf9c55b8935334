"""Parity of the fused QK-norm + RoPE + fp8 KV write and of the KV store."""

import pytest
import torch

from helpers import assert_rope_parity, code_flip_stats, codes
from oracle import inputs, ops

pytestmark = pytest.mark.gpu


def _assert_k_pages(kc, kc_ref, k, kw, eps, loc):
    """K pages: e4m3 of the rotated bf16 K.  Bytes equal except downstream of
    a norm flip: then the decoded value may move by the rotation bound plus
    one e4m3 step of either side."""
    frac, _ = code_flip_stats(kc, kc_ref)
    assert frac < 1e-3
    got = kc.cpu().float()[loc]
    ref = kc_ref.float()[loc]
    n = ops.rmsnorm(k, kw, eps).float()
    half = n.shape[-1] // 2
    bound = 2.0 ** -7 * (n.abs() + torch.cat([n[..., half:], n[..., :half]], -1).abs())
    bound = bound + 2.0 ** -3 * torch.maximum(got.abs(), ref.abs()) + 2.0 ** -9
    assert ((got - ref).abs() <= bound).all()


def _check(dev, q, k, v, pos, loc, qw, kw, eps, cache, slots, hk, d):
    from flashrec_amd.kernel.qk_rope_kv import fused_qk_norm_rope_store_fp8

    kc_ref = torch.zeros(slots, hk, d, dtype=torch.float8_e4m3fn)
    vc_ref = torch.zeros_like(kc_ref)
    q_ref = ops.qk_norm_rope_store_fp8(q, k, v, pos, loc, qw, kw, eps, cache, kc_ref, vc_ref)

    qd, kd, vd = q.to(dev), k.to(dev), v.to(dev)
    kc = torch.zeros(slots, hk, d, dtype=torch.float8_e4m3fn, device=dev)
    vc = torch.zeros_like(kc)
    ok = fused_qk_norm_rope_store_fp8(qd, kd, vd, pos.to(dev), loc.to(dev), qw.to(dev), kw.to(dev),
                                      eps, cache.to(dev), kc, vc)
    assert ok
    torch.cuda.synchronize()
    assert_rope_parity(qd, q_ref, ops.rmsnorm(q, qw, eps))
    # V: pure conversion + scatter, bit-exact including untouched slots
    assert torch.equal(codes(vc), codes(vc_ref))
    _assert_k_pages(kc, kc_ref, k, kw, eps, loc)
    # k and v inputs are not modified
    assert torch.equal(kd.cpu().view(torch.int16), k.view(torch.int16))
    return qd, kc, vc


def test_reference_case(dev):
    """The shapes of the reference's tests/test_qk_rope_kv.py:10-63."""
    torch.manual_seed(4)
    t, hq, hk, d = 7, 16, 8, 128
    cache = ops.cos_sin_cache(d, 2048, 1_000_000)
    q = torch.randn(t, hq, d, dtype=torch.bfloat16)
    k = torch.randn(t, hk, d, dtype=torch.bfloat16)
    v = torch.randn(t, hk, d, dtype=torch.bfloat16)
    pos = torch.arange(t, dtype=torch.int64) + 3
    loc = torch.arange(1, t + 1, dtype=torch.int64)
    ones = torch.ones(d, dtype=torch.bfloat16)
    _check(dev, q, k, v, pos, loc, ones, ones, 1e-6, cache, t + 4, hk, d)


def test_config3_full(dev):
    q, k, v, pos, loc = inputs.config3()
    cache = ops.cos_sin_cache(128, 4096, 1e6)
    g = torch.Generator().manual_seed(13)
    qw = (1 + 0.1 * torch.randn(128, generator=g)).to(torch.bfloat16)
    kw = (1 + 0.1 * torch.randn(128, generator=g)).to(torch.bfloat16)
    _, kc, vc = _check(dev, q, k, v, pos, loc, qw, kw, 1e-6, cache, 65536, 8, 128)
    # slot layout: written slots are exactly loc, everything else untouched (zero)
    written = torch.zeros(65536, dtype=torch.bool)
    written[loc] = True
    vbytes = codes(vc).reshape(65536, -1)
    assert (vbytes[~written] == 0).all()
    assert (vbytes[written] != 0).any(dim=1).all()


def test_strided_views_of_fused_qkv(dev):
    """q/k/v as views into one [T, Hq+2Hk, D] buffer (how Qwen3Attention calls it)."""
    t, hq, hk, d = 33, 16, 8, 128
    g = torch.Generator().manual_seed(21)
    qkv = torch.randn(t, hq + 2 * hk, d, generator=g).to(torch.bfloat16)
    cache = ops.cos_sin_cache(d, 512, 1e6)
    pos = torch.randint(0, 512, (t,), generator=g)
    loc = torch.randperm(200, generator=g)[:t] + 1
    w = torch.ones(d, dtype=torch.bfloat16)
    q, k, v = qkv[:, :hq], qkv[:, hq:hq + hk], qkv[:, hq + hk:]
    kc_ref = torch.zeros(201, hk, d, dtype=torch.float8_e4m3fn)
    vc_ref = torch.zeros_like(kc_ref)
    q_ref = ops.qk_norm_rope_store_fp8(q, k, v, pos, loc, w, w, 1e-6, cache, kc_ref, vc_ref)

    from flashrec_amd.kernel.qk_rope_kv import fused_qk_norm_rope_store_fp8

    qkv_d = qkv.to(dev)
    kc = torch.zeros(201, hk, d, dtype=torch.float8_e4m3fn, device=dev)
    vc = torch.zeros_like(kc)
    assert fused_qk_norm_rope_store_fp8(qkv_d[:, :hq], qkv_d[:, hq:hq + hk], qkv_d[:, hq + hk:],
                                        pos.to(dev), loc.to(dev), w.to(dev), w.to(dev), 1e-6,
                                        cache.to(dev), kc, vc)
    assert_rope_parity(qkv_d[:, :hq], q_ref, ops.rmsnorm(q, w, 1e-6))
    assert torch.equal(codes(vc), codes(vc_ref))
    _assert_k_pages(kc, kc_ref, k, w, 1e-6, loc)


@pytest.mark.parametrize("hq,hk,d", [(6, 2, 64), (4, 4, 128), (3, 1, 100)])
def test_generic_head_shapes(dev, hq, hk, d):
    t = 9
    g = torch.Generator().manual_seed(hq * 100 + d)
    q = torch.randn(t, hq, d, generator=g).to(torch.bfloat16)
    k = torch.randn(t, hk, d, generator=g).to(torch.bfloat16)
    v = torch.randn(t, hk, d, generator=g).to(torch.bfloat16)
    cache = ops.cos_sin_cache(d, 64, 1e4)
    pos = torch.randint(0, 64, (t,), generator=g)
    loc = torch.randperm(30, generator=g)[:t] + 1
    w = (1 + 0.1 * torch.randn(d, generator=g)).to(torch.bfloat16)
    _check(dev, q, k, v, pos, loc, w, w, 1e-6, cache, 31, hk, d)


def test_unsupported_head_dim_returns_false(dev):
    from flashrec_amd.kernel.qk_rope_kv import fused_qk_norm_rope_store_fp8

    t, d = 2, 256
    q = torch.zeros(t, 2, d, dtype=torch.bfloat16, device=dev)
    kc = torch.zeros(4, 1, d, dtype=torch.float8_e4m3fn, device=dev)
    cache = torch.zeros(8, d, device=dev)
    pos = torch.zeros(t, dtype=torch.int64, device=dev)
    assert not fused_qk_norm_rope_store_fp8(q, q[:, :1], q[:, :1], pos, pos, q[0, 0], q[0, 0],
                                            1e-6, cache, kc, kc)


def test_rope_inplace_matches_oracle(dev):
    from flashrec_amd.kernel.sglops import apply_rope_inplace

    t, hq, hk, d = 50, 16, 8, 128
    g = torch.Generator().manual_seed(31)
    q = torch.randn(t, hq * d, generator=g).to(torch.bfloat16)
    k = torch.randn(t, hk * d, generator=g).to(torch.bfloat16)
    cache = ops.cos_sin_cache(d, 1024, 1e6)
    pos = torch.randint(0, 1024, (t,), generator=g)
    qd, kd = q.to(dev), k.to(dev)
    assert apply_rope_inplace(pos.to(dev), qd, kd, d, cache.to(dev))
    q_ref = ops.apply_rope(pos, q.view(t, hq, d), cache).reshape(t, -1)
    k_ref = ops.apply_rope(pos, k.view(t, hk, d), cache).reshape(t, -1)
    assert torch.equal(qd.cpu().view(torch.int16), q_ref.view(torch.int16))
    assert torch.equal(kd.cpu().view(torch.int16), k_ref.view(torch.int16))


def test_store_kv_cache_bf16_and_fp8(dev):
    from flashrec_amd.kernel.sglops import store_kv_cache

    n, row = 100, 8 * 128
    g = torch.Generator().manual_seed(41)
    k = torch.randn(n, row, generator=g).to(torch.bfloat16)
    v = torch.randn(n, row, generator=g).to(torch.bfloat16)
    loc = torch.randperm(500, generator=g)[:n] + 1
    kc = torch.zeros(501, row, dtype=torch.float8_e4m3fn, device=dev)
    vc = torch.zeros_like(kc)
    store_kv_cache(kc, vc, loc.to(dev), k.to(dev), v.to(dev))
    kc_ref = torch.zeros(501, 8, 128, dtype=torch.float8_e4m3fn)
    vc_ref = torch.zeros_like(kc_ref)
    ops.store_kv(kc_ref, vc_ref, loc, k, v)
    assert torch.equal(codes(kc), codes(kc_ref).reshape(501, row))
    assert torch.equal(codes(vc), codes(vc_ref).reshape(501, row))
    # fp8 rows are copied byte for byte
    kc2 = torch.zeros_like(kc)
    vc2 = torch.zeros_like(vc)
    store_kv_cache(kc2, vc2, loc.to(dev), kc[loc.to(dev)], vc[loc.to(dev)])
    assert torch.equal(codes(kc2), codes(kc))
    assert torch.equal(codes(vc2), codes(vc))


def test_out_of_range_slots_are_skipped(dev):
    from flashrec_amd.kernel.sglops import store_kv_cache

    k = torch.ones(3, 16, dtype=torch.bfloat16, device=dev)
    loc = torch.tensor([1, -1, 99], device=dev)
    kc = torch.zeros(4, 16, dtype=torch.float8_e4m3fn, device=dev)
    vc = torch.zeros_like(kc)
    store_kv_cache(kc, vc, loc, k, k)
    c = codes(kc)
    assert (c[1] == 0x38).all()  # e4m3(1.0)
    assert (c[[0, 2, 3]] == 0).all()


@pytest.mark.parametrize("hq,hk,d", [(16, 8, 128), (6, 2, 64)])
def test_rope_and_store_kv_bf16_pool(dev, hq, hk, d):
    """Matching-dtype fused path (reference sglops.py:154-204): q and k rotated
    in place, the rotated k and the untouched v written to a bf16 pool; the
    oracle is RoPE then the pool store (qwen3.py:108-128's unfused order).
    (16, 8, 128) takes the vector kernel, (6, 2, 64) the generic one."""
    from flashrec_amd.kernel.sglops import apply_rope_and_store_kv

    t, slots = 37, 300
    g = torch.Generator().manual_seed(53)
    qkv = torch.randn(t, (hq + 2 * hk) * d, generator=g).to(torch.bfloat16)
    q, k, v = qkv.split([hq * d, hk * d, hk * d], dim=-1)  # strided views, as in the model
    cache = ops.cos_sin_cache(d, 512, 1e6)
    pos = torch.randint(0, 512, (t,), generator=g)
    loc = torch.randperm(slots - 1, generator=g)[:t] + 1
    loc[5] = slots + 7  # out of range slot: skipped
    qkv_d = qkv.to(dev)
    qd, kd, vd = qkv_d.split([hq * d, hk * d, hk * d], dim=-1)
    kc = torch.zeros(slots, hk, d, dtype=torch.bfloat16, device=dev)
    vc = torch.zeros_like(kc)
    assert apply_rope_and_store_kv(pos.to(dev), qd, kd, vd, loc.to(dev), kc, vc, d, cache.to(dev))
    torch.cuda.synchronize()

    q_ref = ops.apply_rope(pos, q.reshape(t, hq, d), cache)
    k_ref = ops.apply_rope(pos, k.reshape(t, hk, d), cache)
    bits = lambda x: x.cpu().contiguous().view(torch.int16)  # noqa: E731
    assert torch.equal(bits(qd).view(t, hq, d), bits(q_ref))
    assert torch.equal(bits(kd).view(t, hk, d), bits(k_ref))
    assert torch.equal(bits(vd), bits(v))  # v is not modified
    kc_ref = torch.zeros(slots, hk, d, dtype=torch.bfloat16)
    vc_ref = torch.zeros_like(kc_ref)
    keep = loc < slots
    ops.store_kv(kc_ref, vc_ref, loc[keep], k_ref[keep], v.reshape(t, hk, d)[keep])
    assert torch.equal(bits(kc), bits(kc_ref))
    assert torch.equal(bits(vc), bits(vc_ref))


def test_rope_and_store_kv_declines_fp8_pool(dev):
    """An fp8 pool with bf16 activations is not this path (the reference returns False too)."""
    from flashrec_amd.kernel.sglops import apply_rope_and_store_kv

    q = torch.zeros(2, 128, dtype=torch.bfloat16, device=dev)
    kc = torch.zeros(4, 1, 128, dtype=torch.float8_e4m3fn, device=dev)
    assert not apply_rope_and_store_kv(torch.zeros(2, dtype=torch.int64, device=dev), q, q.clone(),
                                       q.clone(), torch.ones(2, dtype=torch.int64, device=dev), kc,
                                       kc.clone(), 128, torch.zeros(8, 128, device=dev))


def test_store_kv_cache_bf16_pool(dev):
    from flashrec_amd.kernel.sglops import store_kv_cache

    n, row, slots = 64, 4 * 96, 200
    g = torch.Generator().manual_seed(59)
    k = torch.randn(n, row, generator=g).to(torch.bfloat16)
    v = torch.randn(n, row, generator=g).to(torch.bfloat16)
    loc = torch.randperm(slots - 1, generator=g)[:n] + 1
    kc = torch.zeros(slots, row, dtype=torch.bfloat16, device=dev)
    vc = torch.zeros_like(kc)
    store_kv_cache(kc, vc, loc.to(dev), k.to(dev), v.to(dev))
    kc_ref = torch.zeros(slots, 4, 96, dtype=torch.bfloat16)
    vc_ref = torch.zeros_like(kc_ref)
    ops.store_kv(kc_ref, vc_ref, loc, k, v)
    assert torch.equal(kc.cpu().view(torch.int16), kc_ref.view(slots, row).view(torch.int16))
    assert torch.equal(vc.cpu().view(torch.int16), vc_ref.view(slots, row).view(torch.int16))
    # odd row width: the element-wise form
    k3 = k[:, :37].contiguous()
    kc3 = torch.zeros(slots, 37, dtype=torch.bfloat16, device=dev)
    vc3 = torch.zeros_like(kc3)
    store_kv_cache(kc3, vc3, loc.to(dev), k3.to(dev), k3.to(dev))
    ref3 = torch.zeros(slots, 37, dtype=torch.bfloat16)
    ref3[loc] = k3
    assert torch.equal(kc3.cpu(), ref3) and torch.equal(vc3.cpu(), ref3)


@pytest.mark.parametrize("dtype,d,strided", [(torch.float16, 128, False), (torch.float32, 128, False),
                                             (torch.bfloat16, 256, False), (torch.bfloat16, 64, True),
                                             (torch.float32, 192, True)])
def test_rotary_embedding_other_layouts(dev, dtype, d, strided):
    """RotaryEmbedding.forward answers for the layouts the bf16 kernel declines
    (the reference falls through to FlashInfer or torch there,
    python/flashrec/layers/rotary.py:43-71): fp16 / fp32 heads, D > 128 and
    heads whose elements are not contiguous, bit-exact with the oracle."""
    from flashrec_amd.layers.rotary import RotaryEmbedding

    t, hq, hk = 37, 4, 2
    g = torch.Generator().manual_seed(d + (7 if strided else 0))
    q = torch.randn(t, hq * d, generator=g).to(dtype)
    k = torch.randn(t, hk * d, generator=g).to(dtype)
    rope = RotaryEmbedding(d, 512, 1e6, device=dev)
    pos = torch.randint(0, 512, (t,), generator=g)
    if strided:  # every other element of a wider buffer
        qb = torch.zeros(t, 2 * hq * d, dtype=dtype, device=dev)
        kb = torch.zeros(t, 2 * hk * d, dtype=dtype, device=dev)
        qd, kd = qb[:, ::2], kb[:, ::2]
        qd.copy_(q.to(dev))
        kd.copy_(k.to(dev))
    else:
        qd, kd = q.to(dev), k.to(dev)
    qo, ko = rope(pos.to(dev), qd, kd)
    assert qo.data_ptr() == qd.data_ptr() and ko.data_ptr() == kd.data_ptr()
    cache = ops.cos_sin_cache(d, 512, 1e6)
    q_ref = ops.apply_rope(pos, q.view(t, hq, d), cache).reshape(t, -1)
    k_ref = ops.apply_rope(pos, k.view(t, hk, d), cache).reshape(t, -1)
    assert torch.equal(qd.cpu(), q_ref) and torch.equal(kd.cpu(), k_ref)
    if strided:  # the interleaved elements are untouched
        assert not qb[:, 1::2].any() and not kb[:, 1::2].any()


def test_out_of_range_position_writes_no_kv(dev):
    """A token whose position has no cos/sin row leaves its slot as it was:
    neither K nor V is written (fp8 pool through the fused op, bf16 pool
    through apply_rope_and_store_kv)."""
    from flashrec_amd.kernel.qk_rope_kv import fused_qk_norm_rope_store_fp8
    from flashrec_amd.kernel.sglops import apply_rope_and_store_kv

    t, hq, hk, d, slots, rows = 16, 16, 8, 128, 64, 256
    g = torch.Generator().manual_seed(5)
    q = torch.randn(t, hq, d, generator=g).to(torch.bfloat16).to(dev)
    k = torch.randn(t, hk, d, generator=g).to(torch.bfloat16).to(dev)
    v = torch.randn(t, hk, d, generator=g).to(torch.bfloat16).to(dev)
    pos = torch.randint(0, rows, (t,), generator=g)
    pos[3] = rows + 5
    pos[9] = -1
    loc = (torch.randperm(slots - 1, generator=g)[:t] + 1).to(dev)
    cache = ops.cos_sin_cache(d, rows, 1e6).to(dev)
    w = torch.ones(d, dtype=torch.bfloat16, device=dev)
    kc = torch.zeros(slots, hk, d, dtype=torch.float8_e4m3fn, device=dev)
    vc = torch.zeros_like(kc)
    assert fused_qk_norm_rope_store_fp8(q.clone(), k, v, pos.to(dev), loc, w, w, 1e-6, cache, kc, vc)
    for cache_k, cache_v in ((kc, vc),):
        for bad in (3, 9):
            s = int(loc[bad])
            assert not codes(cache_k[s]).any() and not codes(cache_v[s]).any()
        good = [i for i in range(t) if i not in (3, 9)]
        assert codes(cache_v[loc[good]]).any()
    kb = torch.zeros(slots, hk * d, dtype=torch.bfloat16, device=dev)
    vb = torch.zeros_like(kb)
    assert apply_rope_and_store_kv(pos.to(dev), q.clone().view(t, -1), k.clone().view(t, -1),
                                   v.view(t, -1), loc, kb, vb, d, cache)
    for bad in (3, 9):
        s = int(loc[bad])
        assert not kb[s].any() and not vb[s].any()
    good = [i for i in range(t) if i not in (3, 9)]
    assert torch.equal(vb[loc[good]], v[good].reshape(len(good), -1))
