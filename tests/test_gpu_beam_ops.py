"""The unfused trie steps and the graph-capture entry of the beam module
(reference python/flashrec/kernel/beam_trie.py:82-229, :633-684) against
oracle/beam.py, bit-exact."""

import pytest
import torch

from oracle import beam

pytestmark = pytest.mark.gpu


def _table(g, n_nodes, vsz, density=0.4):
    return torch.rand(n_nodes, vsz, generator=g) < density


@pytest.mark.parametrize("rows,cols,n_nodes,vsz", [(512, 1024, 3000, 256), (7, 33, 5, 10), (16, 8, 0, 0)])
def test_trie_mask_candidates(dev, rows, cols, n_nodes, vsz):
    from flashrec_amd.kernel.beam_trie import trie_mask_candidates

    g = torch.Generator().manual_seed(rows + cols)
    base = 1000
    scores = torch.randn(rows, cols, generator=g)
    scores[0, :3] = torch.tensor([float("nan"), float("inf"), float("-inf")])
    toks = base + torch.randint(-3, max(vsz, 1) + 3, (rows, cols), generator=g)
    nodes = torch.randint(-1, n_nodes + 2, (rows,), generator=g)
    allow = _table(g, n_nodes, vsz)
    got = trie_mask_candidates(scores.to(dev), toks.to(dev), nodes.to(dev), allow.to(dev), base)
    ref = beam.trie_mask_candidates(scores, toks, nodes, allow, base)
    assert torch.equal(got.cpu().view(torch.int32), ref.view(torch.int32))  # NaN payloads too
    # in place, custom fill value
    sd = scores.to(dev)
    out = trie_mask_candidates(sd, toks.to(dev), nodes.to(dev), allow.to(dev), base, out=sd, neg_inf=-1e30)
    assert out.data_ptr() == sd.data_ptr()
    assert torch.equal(out.cpu().view(torch.int32),
                       beam.trie_mask_candidates(scores, toks, nodes, allow, base, -1e30).view(torch.int32))


@pytest.mark.parametrize("next_dtype", [torch.int32, torch.int64])
def test_trie_advance_nodes(dev, next_dtype):
    from flashrec_amd.kernel.beam_trie import trie_advance_nodes, trie_advance_nodes_batched

    g = torch.Generator().manual_seed(5)
    bw, picks, n_nodes, vsz, base, invalid = 512, 512, 20000, 256, 7, 20000
    nodes = torch.randint(-1, n_nodes, (bw,), generator=g)
    parents = torch.randint(-1, bw + 1, (picks,), generator=g)
    toks = base + torch.randint(-2, vsz + 2, (picks,), generator=g)
    nxt = torch.randint(0, n_nodes + 1, (n_nodes, vsz), generator=g).to(next_dtype)
    got = trie_advance_nodes(nodes.to(dev), parents.to(dev), toks.to(dev), nxt.to(dev), base, invalid)
    assert torch.equal(got.cpu(), beam.trie_advance_nodes(nodes, parents, toks, nxt, base, invalid))
    n = 8
    nodes2 = torch.randint(-1, n_nodes, (n, bw), generator=g)
    par2 = torch.randint(0, bw, (n, bw), generator=g)
    tok2 = base + torch.randint(0, vsz, (n, bw), generator=g)
    got2 = trie_advance_nodes_batched(nodes2.to(dev), par2.to(dev), tok2.to(dev), nxt.to(dev), base, invalid)
    assert torch.equal(got2.cpu(), beam.trie_advance_nodes_batched(nodes2, par2, tok2, nxt, base, invalid))


@pytest.mark.parametrize("col", [0, 3, 5])
def test_beam_expand_token_ids(dev, col):
    from flashrec_amd.kernel.beam_trie import beam_expand_token_ids

    g = torch.Generator().manual_seed(col)
    ti = torch.randint(0, 1 << 40, (512, 5), generator=g)
    parents = torch.randint(-1, 514, (512,), generator=g)
    new = torch.randint(0, 1 << 40, (512,), generator=g)
    got = beam_expand_token_ids(ti.to(dev), parents.to(dev), new.to(dev), col)
    assert torch.equal(got.cpu(), beam.beam_expand_token_ids(ti, parents, new, col))
    with pytest.raises(IndexError):
        beam_expand_token_ids(ti.to(dev), parents.to(dev), new.to(dev), 7)


@pytest.mark.parametrize("reference_scratch", [True, False])
def test_call_genrec_cuda_into_caller_buffers(dev, reference_scratch):
    """graph.py's call into its own buffers: with the reference's [N, BW*C]
    fp32 scratch (large enough: used) or none (the library's static scratch),
    the same results as genrec_mask_topk_expand."""
    from flashrec_amd.kernel.beam_trie import call_genrec_cuda, genrec_mask_topk_expand

    g = torch.Generator().manual_seed(9)
    n, bw, c, vsz, n_nodes, base = 4, 64, 128, 256, 300, 500
    cum = torch.randn(n, bw, generator=g)
    lp = torch.sort(torch.randn(n, bw, c, generator=g), dim=-1, descending=True).values
    tok = base + torch.randint(0, vsz, (n, bw, c), generator=g)
    nodes = torch.randint(0, n_nodes, (n, bw), generator=g)
    allow = (torch.rand(n_nodes, vsz, generator=g) < 0.5).to(torch.uint8)
    nxt = torch.randint(0, n_nodes, (n_nodes, vsz), generator=g).to(torch.int32)
    ti = torch.randint(0, 9999, (n, bw, 3), generator=g)
    col = torch.full((n,), 1, dtype=torch.int32)
    d = {k: v.to(dev) for k, v in dict(cum=cum, lp=lp, tok=tok, nodes=nodes, allow=allow, nxt=nxt, ti=ti,
                                         col=col).items()}
    want = genrec_mask_topk_expand(d["cum"], d["lp"], d["tok"], select_k=bw, node_ids=d["nodes"],
                                   allow_table=d["allow"], token_base=base, token_ids=d["ti"], col=d["col"],
                                   next_node=d["nxt"], invalid_node=n_nodes)
    outs = [torch.empty(n, bw, device=dev), *(torch.empty(n, bw, dtype=torch.int64, device=dev) for _ in range(3))]
    tok_out = torch.empty_like(d["ti"])
    node_out = torch.empty_like(d["nodes"])
    scratch = torch.empty(n, bw * c, dtype=torch.float32, device=dev) if reference_scratch else None
    ok = call_genrec_cuda(*outs, scratch, d["cum"], d["lp"], d["tok"], d["nodes"], d["allow"], d["ti"], tok_out,
                          d["nxt"], node_out, torch.ones(n, dtype=torch.uint8, device=dev), base, n_nodes, d["col"])
    assert ok
    torch.cuda.synchronize()
    for a, b in zip((*outs, tok_out, node_out), want):
        assert torch.equal(a, b)
