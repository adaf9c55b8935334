"""Per-row candidate top-k (fr_row_topk) against oracle/beam.row_topk and
torch.topk, bit-exact, and the composed beam step (row top-k -> fused trie
mask/top-K/expand/advance) against the oracle's composition."""

import pytest
import torch

from oracle import beam

pytestmark = pytest.mark.gpu


def _check(dev, x, k, cand=None):
    from flashrec_amd.kernel.beam_trie import row_topk

    print(f"row_topk shape={tuple(x.shape)} k={k}", flush=True)
    vals, idx, tok = row_topk(x.to(dev), k, None if cand is None else cand.to(dev))
    rv, ri, rt = beam.row_topk(x, k, cand)
    assert torch.equal(idx.cpu(), ri)
    assert torch.equal(vals.cpu().view(torch.int32), rv.view(torch.int32))  # bits, NaN and -0 included
    assert torch.equal(tok.cpu(), rt)
    return vals, idx, tok


def test_config4_shape_against_torch_topk(dev):
    """8 requests x 512 beams over the 8192-token SID head, C = 2 x 512."""
    g = torch.Generator().manual_seed(0)
    x = torch.log_softmax(torch.randn(8, 512, 8192, generator=g) * 2, dim=-1)
    cand = torch.arange(140000, 148192)
    vals, idx, _ = _check(dev, x, 1024, cand)
    # the same selection as torch.topk wherever the scores are tie-free
    tv, ti = torch.topk(x, 1024, dim=-1, largest=True, sorted=True)
    assert torch.equal(vals.cpu(), tv)
    distinct = torch.tensor([row.unique().numel() == row.numel() for row in x.reshape(-1, 8192)[:64]])
    rows = torch.nonzero(distinct).reshape(-1)
    assert torch.equal(idx.cpu().reshape(-1, 1024)[rows], ti.reshape(-1, 1024)[rows])


@pytest.mark.parametrize("r,v,k", [(3, 1, 1), (5, 5, 3), (7, 100, 100), (4, 1000, 37), (9, 1024, 1024),
                                   (6, 1030, 513), (3, 4096, 256), (2, 16384, 1000), (300, 256, 256),
                                   (2, 9000, 1)])
def test_shapes(dev, r, v, k):
    g = torch.Generator().manual_seed(r * 1000 + v + k)
    _check(dev, torch.randn(r, v, generator=g), k, torch.randint(0, 10 ** 6, (v,), generator=g))


def test_ties_specials_and_strides(dev):
    g = torch.Generator().manual_seed(5)
    x = torch.round(torch.randn(16, 2000, generator=g) * 2) / 2  # heavy ties at every boundary
    x[0, ::7] = -0.0
    x[1, 5] = float("nan")
    x[1, 900] = float("nan")
    x[2, :] = float("-inf")
    x[3, 10:20] = float("inf")
    for k in (1, 100, 333, 1024):
        _check(dev, x, k)
    # a strided view whose rows are not 16-byte aligned (scalar loads)
    from flashrec_amd.kernel.beam_trie import row_topk

    big = torch.randn(10, 1027, generator=g)
    xv = big[:, 3:1003]
    vals, idx, _ = row_topk(big.to(dev)[:, 3:1003], 64)
    rv, ri, _ = beam.row_topk(xv, 64)
    assert torch.equal(idx.cpu(), ri) and torch.equal(vals.cpu(), rv)


def test_rejects_unsupported(dev):
    from flashrec_amd._lib import FlashRecKernelError
    from flashrec_amd.kernel.beam_trie import row_topk

    with pytest.raises(FlashRecKernelError):
        row_topk(torch.randn(2, 4096, device=dev), 2048)
    with pytest.raises(FlashRecKernelError):
        row_topk(torch.randn(2, 100, device=dev), 101)


def test_graph_replay(dev):
    from flashrec_amd.kernel.beam_trie import row_topk

    x = torch.randn(64, 8192, device=dev)
    vals = torch.empty(64, 512, device=dev)
    idx = torch.empty(64, 512, dtype=torch.int64, device=dev)
    tok = torch.empty(64, 512, dtype=torch.int64, device=dev)
    row_topk(x, 512, out=(vals, idx), out_tokens=tok)
    torch.cuda.synchronize()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        row_topk(x, 512, out=(vals, idx), out_tokens=tok)
    for i in range(3):
        x.copy_(torch.randn(64, 8192, device=dev))
        ev, ei, _ = row_topk(x, 512)
        g.replay()
        torch.cuda.synchronize()
        assert torch.equal(vals, ev) and torch.equal(idx, ei)


def _trie(g, levels, codes, items):
    """Dense tables of a random trie of `items` SIDs, `levels` tokens each,
    level l's codes at token_base + l*codes + c (the reference's dense
    allow/next tables, python/flashrec/search/trie.py:208-251: next_node int32,
    leaves -> -1 (unconstrained), missing children -> invalid)."""
    sids = torch.randint(0, codes, (items, levels), generator=g)
    prefixes = {(): 0}
    for s in sids.tolist():
        for d in range(1, levels):
            prefixes.setdefault(tuple(s[:d]), len(prefixes))
    n_nodes = len(prefixes)
    invalid = n_nodes
    vsz = levels * codes
    allow = torch.zeros(n_nodes + 1, vsz, dtype=torch.bool)
    nxt = torch.full((n_nodes + 1, vsz), invalid, dtype=torch.int32)
    for s in sids.tolist():
        for d in range(levels):
            node = prefixes[tuple(s[:d])]
            rel = d * codes + s[d]
            allow[node, rel] = True
            nxt[node, rel] = prefixes.get(tuple(s[: d + 1]), -1) if d + 1 < levels else -1
    return allow, nxt, invalid


def test_beam_step_composition(dev):
    """logprobs -> row top-C -> trie mask/top-K/expand/advance, level 1 of a
    3-level x 64-code trie, 3 requests x 64 beams, C = 128, K = 64."""
    from flashrec_amd.kernel.beam_trie import genrec_mask_topk_expand, row_topk

    g = torch.Generator().manual_seed(9)
    levels, codes, n, bw, c = 3, 64, 3, 64, 128
    allow, nxt, invalid = _trie(g, levels, codes, 3000)
    base = 50000
    vocab = 512  # head columns: the trie's 192 codes and others
    cand = base + torch.arange(vocab)
    logp = torch.log_softmax(torch.randn(n, bw, vocab, generator=g) * 3, dim=-1)
    cum = torch.sort(torch.randn(n, bw, generator=g), dim=-1, descending=True).values
    # level-1 nodes of each beam: walk its level-0 token
    l0 = torch.randint(0, codes, (n, bw), generator=g)
    nodes = nxt[0, l0].long()
    ti = torch.randint(0, 9, (n, bw, levels), generator=g)
    ti[:, :, 0] = base + l0
    col = torch.full((n,), 1, dtype=torch.int32)

    v, _, t = row_topk(logp.to(dev), c, cand.to(dev))
    got = genrec_mask_topk_expand(cum.to(dev), v, t, select_k=bw, node_ids=nodes.to(dev),
                                  allow_table=allow.to(dev), token_base=base, token_ids=ti.to(dev),
                                  col=col.to(dev), next_node=nxt.to(dev), invalid_node=invalid)
    rv, _, rt = beam.row_topk(logp, c, cand)
    ref = beam.genrec_mask_topk_expand(cum, rv, rt, bw, nodes, allow, base, ti, col, nxt.long(), invalid)
    for a, b in zip((got.vals, got.parents, got.tokens, got.indices, got.token_ids, got.node_ids), ref):
        assert torch.equal(a.cpu(), b)
    # every pick is a valid trie edge, and the advanced nodes are level-2 nodes or invalid
    picked = got.tokens.cpu()
    par = got.parents.cpu()
    ok = allow[nodes.gather(1, par), picked - base]
    assert ok[got.vals.cpu() > float("-inf")].all()


def test_without_indices(dev):
    from flashrec_amd.kernel.beam_trie import row_topk

    x = torch.randn(33, 3000, device=dev)
    v0, i0, t0 = row_topk(x, 200, torch.arange(3000, device=dev) * 3)
    v1, i1, t1 = row_topk(x, 200, torch.arange(3000, device=dev) * 3, need_idx=False)
    assert i1 is None
    assert torch.equal(v0, v1) and torch.equal(t0, t1) and torch.equal(t0, i0 * 3)


@pytest.mark.parametrize("v", [4096, 8192, 2000])
def test_log_softmax_folded(dev, v):
    """row_topk(logits, log_softmax=True) (fr_log_softmax_row_topk for V = 4096
    and 8192; the two calls otherwise) is bit-identical to log_softmax_f32
    then row_topk, which is held to the oracle here as well; rows with heavy
    ties, -inf entries, a -inf row and a NaN included."""
    from flashrec_amd.kernel.beam_trie import row_topk
    from flashrec_amd.kernel.sglops import log_softmax_f32

    g = torch.Generator().manual_seed(v)
    x = torch.randn(40, v, generator=g) * 3
    x[0] = torch.round(x[0])  # heavy ties
    x[1, ::3] = float("-inf")
    x[2] = float("-inf")
    x[3, 17] = float("nan")
    x[4, :] = 0.0
    cand = torch.randint(0, 10 ** 6, (v,), generator=g)
    xd, cd = x.to(dev), cand.to(dev)
    lp = log_softmax_f32(xd)
    for k in (1, 200, 512, 1024):
        print(f"log_softmax folded top-k V={v} k={k}", flush=True)
        rv, ri, rt = row_topk(lp, k, cd)
        fv, fi, ft = row_topk(xd, k, cd, log_softmax=True)
        assert torch.equal(fv.cpu().view(torch.int32), rv.cpu().view(torch.int32))
        assert torch.equal(fi.cpu(), ri.cpu()) and torch.equal(ft.cpu(), rt.cpu())
        ov, oi, ot = beam.row_topk(lp.cpu(), k, cand)
        assert torch.equal(rv.cpu().view(torch.int32), ov.view(torch.int32)) and torch.equal(ri.cpu(), oi)
    # a strided view (rows not 16-byte aligned) takes the two calls
    wide = torch.randn(8, v + 1, generator=g).to(dev)[:, 1:]
    fv, fi, _ = row_topk(wide, 64, log_softmax=True)
    rv, ri, _ = row_topk(log_softmax_f32(wide.contiguous()), 64)
    assert torch.equal(fv.cpu().view(torch.int32), rv.cpu().view(torch.int32)) and torch.equal(fi.cpu(), ri.cpu())
