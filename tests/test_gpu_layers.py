"""Layer-level behaviour on the GPU: Linear, RMSNorm.quant_fp8, the KV pool,
the fp8 restricted lm_head, and HIP-graph capture of the path."""

import pytest
import torch
import torch.nn.functional as F

from helpers import assert_fp8_parity, codes, max_abs_rel
from oracle import ops

pytestmark = pytest.mark.gpu


def test_linear_quantize_and_forward(dev):
    from flashrec_amd.layers.linear import Linear

    g = torch.Generator().manual_seed(2)
    w = torch.randn(384, 256, generator=g).to(torch.bfloat16)
    x = torch.randn(3, 5, 256, generator=g).to(torch.bfloat16)
    lin = Linear(256, 384)
    lin.load(w.to(dev), quantize_fp8=True)
    assert lin._fp8_weight.shape == (256, 384) and lin._fp8_weight.stride() == (1, 256)
    out = lin(x.to(dev))
    assert out.shape == (3, 5, 384) and out.dtype == torch.bfloat16
    qa, sa = ops.per_token_quant_fp8(x)
    qw, sw = ops.quantize_weight_fp8(w)
    ref = ops.fp8_scaled_mm(qa, qw.t(), sa, sw).reshape(3, 5, 384)
    assert max_abs_rel(out, ref) < 1e-2
    # the quantised model stays close to the bf16 product
    assert max_abs_rel(out, F.linear(x.float(), w.float())) < 5e-2


def test_shared_quant_matches_separate_linears(dev):
    """Reference tests/test_rms_fp8.py:44-64: one per-token quant feeding two
    Linear.forward_fp8 calls equals each Linear's own forward."""
    from flashrec_amd.kernel.sglops import per_token_quant_fp8
    from flashrec_amd.layers.linear import Linear

    torch.manual_seed(2)
    x = torch.randn(4, 64, dtype=torch.bfloat16).to(dev)
    q_lin, k_lin = Linear(64, 128), Linear(64, 32)
    q_lin.load(torch.randn(128, 64, dtype=torch.bfloat16).to(dev), quantize_fp8=True)
    k_lin.load(torch.randn(32, 64, dtype=torch.bfloat16).to(dev), quantize_fp8=True)
    q_fp8, scale = per_token_quant_fp8(x)
    torch.testing.assert_close(q_lin.forward_fp8(q_fp8, scale, x.shape, x.dtype), q_lin(x),
                               atol=2e-2, rtol=2e-2)
    torch.testing.assert_close(k_lin.forward_fp8(q_fp8, scale, x.shape, x.dtype), k_lin(x),
                               atol=2e-2, rtol=2e-2)


def test_prequantized_checkpoint_load(dev):
    from flashrec_amd.layers.linear import Linear

    g = torch.Generator().manual_seed(3)
    w = torch.randn(64, 128, generator=g)
    q = w.to(torch.float8_e4m3fn)
    x = torch.randn(8, 128, generator=g).to(torch.bfloat16)
    lin = Linear(128, 64)
    lin.load(q.to(dev), weight_scale=torch.tensor(0.5))
    out = lin(x.to(dev))
    qa, sa = ops.per_token_quant_fp8(x)
    ref = ops.fp8_scaled_mm(qa, q.t(), sa, torch.full((64,), 0.5))
    assert max_abs_rel(out, ref) < 1e-2


def test_rmsnorm_module_quant(dev):
    from flashrec_amd.layers.norm import RMSNorm

    norm = RMSNorm(2048).to(dev)
    g = torch.Generator().manual_seed(5)
    x = torch.randn(32, 2048, generator=g).to(torch.bfloat16)
    r = torch.randn(32, 2048, generator=g).to(torch.bfloat16)
    q, s = norm.quant_fp8(x.to(dev))
    q_ref, s_ref = ops.rmsnorm_per_token_quant_fp8(x, torch.ones(2048), 1e-6)
    assert_fp8_parity(q, s, q_ref, s_ref)
    q, s, res = norm.quant_fp8(x.to(dev), r.to(dev))
    q_ref, s_ref, res_ref = ops.fused_add_rmsnorm_per_token_quant_fp8(x, r, torch.ones(2048), 1e-6)
    assert_fp8_parity(q, s, q_ref, s_ref)
    assert torch.equal(res.cpu().view(torch.int16), res_ref.view(torch.int16))


def test_kv_pool_store(dev):
    from flashrec_amd.kvcache.pool import TokenToKVPool

    pool = TokenToKVPool(2, 64, 8, 128, torch.float8_e4m3fn, dev)
    loc = pool.alloc(10)
    assert 0 not in loc.cpu().tolist()
    g = torch.Generator().manual_seed(6)
    k = torch.randn(10, 8, 128, generator=g).to(torch.bfloat16)
    v = torch.randn(10, 8, 128, generator=g).to(torch.bfloat16)
    pool.store(1, k.to(dev), v.to(dev), loc)
    kc_ref = torch.zeros(64, 8, 128, dtype=torch.float8_e4m3fn)
    vc_ref = torch.zeros_like(kc_ref)
    ops.store_kv(kc_ref, vc_ref, loc.cpu(), k, v)
    assert torch.equal(codes(pool.k[1]), codes(kc_ref))
    assert torch.equal(codes(pool.v[1]), codes(vc_ref))
    assert (codes(pool.k[0]) == 0).all()


def test_restricted_lm_head_fp8(dev):
    from flashrec_amd.logits import RestrictedLMHead

    g = torch.Generator().manual_seed(7)
    vocab, hidden, lo, n = 12000, 256, 1000, 8192
    w = (0.02 * torch.randn(vocab, hidden, generator=g)).to(torch.bfloat16)
    h = torch.randn(64, hidden, generator=g).to(torch.bfloat16)
    head = RestrictedLMHead(list(range(lo, lo + n)), fp8=True)
    head.bind(w.to(dev))
    lp, ids = head.compute(h.to(dev), w.to(dev))
    assert lp.shape == (64, n) and lp.dtype == torch.float32
    assert ids.cpu().tolist() == list(range(lo, lo + n))
    ref = ops.restricted_logprobs_fp8(h, w[lo:lo + n])
    assert (lp.cpu() - ref).abs().max().item() < 2e-3
    torch.testing.assert_close(lp.exp().sum(-1).cpu(), torch.ones(64), atol=1e-4, rtol=0)
    # per-codebook levels are slices of the same quantised weight
    head.bind_codebook([4096, 2048, 2048])
    lp1, ids1 = head.compute_level(h.to(dev), 1)
    ref1 = ops.restricted_logprobs_fp8(h, w[lo + 4096:lo + 6144])
    assert ids1.cpu().tolist() == list(range(lo + 4096, lo + 6144))
    assert (lp1.cpu() - ref1).abs().max().item() < 2e-3
    # logits without the log-softmax, from bf16 rows or from rows quantised
    # by the fused RMSNorm -> e4m3: the same bits as the norm then the head
    from flashrec_amd.kernel.sglops import log_softmax_f32, rmsnorm
    from flashrec_amd.layers.norm import RMSNorm

    lg, ids2 = head.compute_logits(h.to(dev), w.to(dev))
    assert torch.equal(ids2.cpu(), ids.cpu())
    assert torch.equal(log_softmax_f32(lg).cpu(), lp.cpu())
    norm = RMSNorm(hidden)
    norm.weight = torch.nn.Parameter((1 + 0.1 * torch.randn(hidden, generator=g)).to(torch.bfloat16).to(dev),
                                     requires_grad=False)
    x = (3 * torch.randn(64, hidden, generator=g)).to(torch.bfloat16).to(dev)
    want, _ = head.compute_logits(rmsnorm(x, norm.weight, norm.eps), w.to(dev))
    got, _ = head.compute_logits_fp8(*norm.quant_fp8(x), w.to(dev))
    assert torch.equal(got.cpu().view(torch.int32), want.cpu().view(torch.int32))


def test_graph_capture_replays(dev):
    """The quant + GEMM + log_softmax chain is graph-capturable; every replay
    matches eager execution (with eager work in between replays)."""
    from flashrec_amd.logits import RestrictedLMHead

    g = torch.Generator().manual_seed(8)
    w = (0.02 * torch.randn(4096, 512, generator=g)).to(torch.bfloat16).to(dev)
    h = torch.randn(128, 512, generator=g).to(torch.bfloat16).to(dev)
    head = RestrictedLMHead(list(range(100, 2148)), fp8=True)
    head.bind(w)
    out = torch.empty(128, 2048, dtype=torch.float32, device=dev)
    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(s):
        for _ in range(2):
            head.compute_into(h, w, out)
    torch.cuda.current_stream().wait_stream(s)
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        head.compute_into(h, w, out)
    for i in range(3):
        h.copy_(torch.randn(128, 512, generator=g).to(torch.bfloat16).to(dev))
        eager, _ = head.compute(h, w)
        torch.cuda.synchronize()
        graph.replay()
        torch.cuda.synchronize()
        assert torch.equal(out, eager), f"replay {i} differs"


def test_kv_pool_alloc_uploads_without_blocking(dev):
    """alloc() stages ids in pinned memory and copies them asynchronously;
    many allocations wrap the staging ring and every result stays intact."""
    from flashrec_amd.kvcache.pool import TokenToKVPool

    pool = TokenToKVPool(1, 1 << 17, 1, 8, torch.bfloat16, dev)
    pool._upload.capacity = 1024  # small ring: forces wrap-around
    got, want = [], []
    for i in range(200):
        n = 1 + (i * 37) % 300
        ids = pool.alloc(n)
        assert ids.device.type == "cuda" and ids.dtype == torch.int64
        got.append(ids)
        want.append(list(pool.last_alloc_cpu))
    torch.cuda.synchronize()
    for ids, w in zip(got, want):
        assert ids.cpu().tolist() == w
    flat = [x for w in want for x in w]
    assert len(set(flat)) == len(flat) and 0 not in flat
    pool.free(torch.cat(got))
    assert pool.available_size() == (1 << 17) - 1


def test_kv_pool_bf16_store(dev):
    from flashrec_amd.kvcache.pool import TokenToKVPool

    pool = TokenToKVPool(1, 32, 2, 64, torch.bfloat16, dev)
    loc = pool.alloc(5)
    k = torch.randn(5, 2, 64, dtype=torch.bfloat16, device=dev)
    v = torch.randn(5, 2, 64, dtype=torch.bfloat16, device=dev)
    pool.store(0, k, v, loc)
    torch.cuda.synchronize()
    assert torch.equal(pool.k[0][loc], k) and torch.equal(pool.v[0][loc], v)
    assert (pool.k[0][0] == 0).all()
