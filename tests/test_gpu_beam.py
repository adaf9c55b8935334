"""The fused beam step (through the C ABI) against oracle/beam.py, bit-exact:
picked scores, parents, tokens and flat indices, the expanded token rows and
the advanced trie nodes."""

import pytest
import torch

from oracle import beam

pytestmark = pytest.mark.gpu


def _case(n, bw, c, vocab, n_nodes, density, seed, tie=False, unconstrained=0.1, nan=False):
    g = torch.Generator().manual_seed(seed)
    cum = torch.randn(n, bw, generator=g) * 3
    lp = torch.randn(n, bw, c, generator=g)
    if tie:  # coarse values: many exact ties
        cum = torch.round(cum)
        lp = torch.round(lp * 2) / 2
    lp = torch.sort(lp, dim=-1, descending=True).values
    if nan:
        lp[0, 1, 3] = float("nan")
        lp[0, 2, 0] = float("-inf")
    base = 1000
    tok = base + torch.randint(-2, vocab + 2, (n, bw, c), generator=g)  # a few outside the table
    nodes = torch.randint(0, n_nodes, (n, bw), generator=g)
    nodes[torch.rand(n, bw, generator=g) < unconstrained] = -1
    allow = torch.rand(n_nodes, vocab, generator=g) < density
    nxt = torch.randint(0, n_nodes, (n_nodes, vocab), generator=g)
    ti = torch.randint(0, 50000, (n, bw, 4), generator=g)
    col = torch.randint(0, 4, (n,), generator=g).to(torch.int32)
    return cum, lp, tok, nodes, allow, nxt, ti, col, base


def _compare(dev, args, k, do_expand=None, **flags):
    from flashrec_amd.kernel.beam_trie import genrec_mask_topk_expand

    cum, lp, tok, nodes, allow, nxt, ti, col, base = args
    got = genrec_mask_topk_expand(
        cum.to(dev), lp.to(dev), tok.to(dev), select_k=k, node_ids=nodes.to(dev), allow_table=allow.to(dev),
        token_base=base, token_ids=ti.to(dev), col=col.to(dev), next_node=nxt.to(dev), invalid_node=-9,
        do_expand=None if do_expand is None else do_expand.to(dev), **flags)
    ref = beam.genrec_mask_topk_expand(cum, lp, tok, k, nodes, allow, base, ti, col, nxt, -9, do_expand,
                                       **flags)
    assert torch.equal(got.vals.cpu(), ref[0])
    assert torch.equal(got.parents.cpu(), ref[1])
    assert torch.equal(got.tokens.cpu(), ref[2])
    assert torch.equal(got.indices.cpu(), ref[3])
    rows = torch.ones(cum.shape[0], dtype=torch.bool) if do_expand is None else do_expand.bool()
    if ref[4] is not None:
        assert got.token_ids is not None
        assert torch.equal(got.token_ids.cpu()[rows], ref[4][rows])
    else:
        assert got.token_ids is None
    if ref[5] is not None:
        assert got.node_ids is not None
        assert torch.equal(got.node_ids.cpu()[rows], ref[5][rows])
    else:
        assert got.node_ids is None
    return got


def test_config4_shape(dev):
    """8 requests x 512 beams x 256 candidates, K = 512, dense random trie."""
    _compare(dev, _case(8, 512, 256, 256, 300, 0.9, 1), 512)


@pytest.mark.parametrize("n,bw,c,k", [(3, 50, 100, 50), (2, 37, 65, 20), (1, 16, 64, 1000), (4, 200, 7, 130),
                                      (2, 512, 1024, 1024), (1, 2048, 16, 32), (2, 1100, 8, 8)])
def test_shapes(dev, n, bw, c, k):
    _compare(dev, _case(n, bw, c, 300, 40, 0.5, n * 7 + bw), k)


def test_ties_nan_and_sparse_trie(dev):
    """Many exact ties; a NaN and a -inf score; a trie sparse enough that
    some requests have fewer than K valid candidates."""
    _compare(dev, _case(3, 64, 40, 300, 20, 0.02, 3, tie=True, unconstrained=0.0, nan=True), 64)
    _compare(dev, _case(3, 64, 40, 300, 20, 0.3, 4, tie=True, nan=True), 64)


def test_flags_and_do_expand(dev):
    args = _case(4, 96, 33, 200, 30, 0.6, 5)
    _compare(dev, args, 96, apply_mask=False)
    _compare(dev, args, 96, apply_expand=False)
    _compare(dev, args, 96, apply_advance=False)
    _compare(dev, args, 96, do_expand=torch.tensor([1, 0, 1, 0], dtype=torch.uint8))


def test_workspace_ping_pong(dev):
    """Feeding a step's token / node planes back in reads one ping-pong plane
    and writes the other (no copy of the plane, never in place)."""
    from flashrec_amd.kernel.beam_trie import GenrecFusedWorkspace, genrec_mask_topk_expand

    cum, lp, tok, nodes, allow, nxt, ti, col, base = _case(2, 64, 32, 200, 30, 0.7, 6)
    ws = GenrecFusedWorkspace()
    d = dict(select_k=64, allow_table=allow.to(dev), token_base=base, next_node=nxt.to(dev), invalid_node=-9,
             workspace=ws)
    r1 = genrec_mask_topk_expand(cum.to(dev), lp.to(dev), tok.to(dev), node_ids=nodes.to(dev),
                                 token_ids=ti.to(dev), col=1, **d)
    t1, n1 = r1.token_ids.clone(), r1.node_ids.clone()
    r2 = genrec_mask_topk_expand(cum.to(dev), lp.to(dev), tok.to(dev), node_ids=r1.node_ids,
                                 token_ids=r1.token_ids, col=2, **d)
    assert r2.token_ids.data_ptr() != r1.token_ids.data_ptr() or r2.token_ids is not r1.token_ids
    ref = beam.genrec_mask_topk_expand(cum, lp, tok, 64, n1.cpu(), allow, base, t1.cpu(), 2, nxt, -9)
    assert torch.equal(r2.token_ids.cpu(), ref[4])
    assert torch.equal(r2.node_ids.cpu(), ref[5])
