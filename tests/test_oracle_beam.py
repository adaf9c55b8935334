"""Pins for oracle/beam.py that do not restate it: torch.topk (an independent
selection) on tie-free inputs, and small cases whose answers are written out
by hand."""

import torch

from oracle import beam

NEG = float("-inf")


def _sorted_rows(t):
    return torch.sort(t, dim=-1, descending=True).values


def test_matches_torch_topk_without_ties():
    """The reference's PyTorch branch is a flat torch.topk over the masked
    scores: with distinct scores and at least K valid candidates the
    selections agree exactly."""
    g = torch.Generator().manual_seed(0)
    n, bw, c, k = 3, 24, 10, 24
    cum = torch.randn(n, bw, generator=g)
    lp = _sorted_rows(torch.randn(n, bw, c, generator=g))
    tok = torch.randint(100, 140, (n, bw, c), generator=g)
    nodes = torch.randint(-1, 6, (n, bw), generator=g)
    allow = torch.rand(6, 40, generator=g) > 0.3
    vals, parents, tokens, idx, _, _ = beam.genrec_mask_topk_expand(cum, lp, tok, k, nodes, allow, 100)
    scores = (cum[:, :, None] + lp).reshape(n, -1)
    node = nodes[:, :, None].expand(n, bw, c).reshape(n, -1)
    rel = tok.reshape(n, -1) - 100
    ok = allow[node.clamp(min=0), rel] | (node < 0)
    masked = scores.masked_fill(~ok, NEG)
    assert ((masked > NEG).sum(1) >= k).all()
    tv, ti = torch.topk(masked, k, dim=-1, largest=True, sorted=True)
    assert torch.equal(vals, tv)
    assert torch.equal(idx, ti)
    assert torch.equal(parents, ti // c)
    assert torch.equal(tokens, tok.reshape(n, -1).gather(1, ti))


def test_ties_rank_by_flat_index():
    cum = torch.tensor([[0.0, 0.0, 1.0]])
    lp = torch.tensor([[[2.0, 1.0], [2.0, 0.5], [1.0, 1.0]]])  # scores 2,1 | 2,0.5 | 2,2
    tok = torch.arange(6).view(1, 3, 2)
    vals, parents, tokens, idx, _, _ = beam.genrec_mask_topk_expand(cum, lp, tok, 5)
    assert idx.tolist() == [[0, 2, 4, 5, 1]]
    assert vals.tolist() == [[2.0, 2.0, 2.0, 2.0, 1.0]]
    assert parents.tolist() == [[0, 1, 2, 2, 0]]


def test_masked_and_missing_picks():
    """Node 0 allows only token 11; beam 1 is unconstrained (node -1); the
    -inf score and the NaN are never picked; 4 picks of 2 valid pad with
    (-inf, parent 0, index 0, token top_tokens[0, 0, 0])."""
    cum = torch.tensor([[0.0, 0.0]])
    lp = torch.tensor([[[3.0, 2.0, 1.0], [float("nan"), 0.5, NEG]]])
    tok = torch.tensor([[[10, 11, 12], [10, 12, 13]]])
    nodes = torch.tensor([[0, -1]])
    allow = torch.zeros(1, 8, dtype=torch.bool)
    allow[0, 1] = True  # token 11 (base 10)
    vals, parents, tokens, idx, _, _ = beam.genrec_mask_topk_expand(cum, lp, tok, 4, nodes, allow, 10)
    assert vals.tolist() == [[2.0, 0.5, NEG, NEG]]
    assert idx.tolist() == [[1, 4, 0, 0]]
    assert parents.tolist() == [[0, 1, 0, 0]]
    assert tokens.tolist() == [[11, 12, 10, 10]]


def test_expand_and_advance_by_hand():
    cum = torch.tensor([[0.0, -1.0, -5.0]])
    lp = torch.tensor([[[0.0, -2.0], [0.0, -3.0], [0.0, -4.0]]])  # 0,-2 | -1,-4 | -5,-9
    tok = torch.tensor([[[20, 21], [22, 23], [24, 25]]])
    nodes = torch.tensor([[1, 2, -1]])
    allow = torch.ones(3, 8, dtype=torch.bool)
    nxt = torch.arange(24).view(3, 8)
    ti = torch.tensor([[[7, 7, 7], [8, 8, 8], [9, 9, 9]]])
    vals, parents, tokens, idx, tout, nout = beam.genrec_mask_topk_expand(
        cum, lp, tok, 2, nodes, allow, 20, ti, 1, nxt, -3)
    assert vals.tolist() == [[0.0, -1.0]]
    assert parents.tolist() == [[0, 1]]
    assert tokens.tolist() == [[20, 22]]
    # rows 0, 1 rebuilt from their parents with column 1 = the new token; row 2 (>= K) copied
    assert tout.tolist() == [[[7, 20, 7], [8, 22, 8], [9, 9, 9]]]
    # node of parent 0 is 1 -> next[1][20 - 20] = 8; parent 1 node 2 -> next[2][2] = 18; row 2 copied
    assert nout.tolist() == [[8, 18, -1]]


def test_trie_rules():
    allow = torch.tensor([[True, False]])
    nxt = torch.tensor([[5, 6]])
    assert beam.cand_ok(-1, 999, allow, 10)           # unconstrained
    assert beam.cand_ok(0, 10, allow, 10)
    assert not beam.cand_ok(0, 11, allow, 10)
    assert not beam.cand_ok(0, 12, allow, 10)         # outside the table
    assert not beam.cand_ok(0, 9, allow, 10)
    assert beam.transition(-4, 10, nxt, 10, -1) == -4  # unconstrained stays
    assert beam.transition(0, 11, nxt, 10, -1) == 6
    assert beam.transition(0, 12, nxt, 10, -1) == -1   # outside -> invalid
    assert beam.transition(7, 10, nxt, 10, -1) == 5    # node clamped to the table


def test_row_topk_matches_torch_topk_without_ties():
    g = torch.Generator().manual_seed(2)
    x = torch.randn(6, 300, generator=g)
    assert x.unique().numel() == x.numel()
    cand = torch.arange(1000, 1300)
    for k in (1, 17, 300):
        vals, idx, tok = beam.row_topk(x, k, cand)
        tv, ti = torch.topk(x, k, dim=-1, largest=True, sorted=True)
        assert torch.equal(vals, tv) and torch.equal(idx, ti)
        assert torch.equal(tok, ti + 1000)


def test_row_topk_ties_nan_and_signed_zero_by_hand():
    nan, inf = float("nan"), float("inf")
    x = torch.tensor([[0.0, -0.0, 1.0, nan, -inf, 1.0, inf, nan, -0.0]])
    vals, idx, tok = beam.row_topk(x, 9)
    # NaN first (by index), then +inf, the 1.0 tie by index, the three zeros
    # (signed zero equal) by index, then -inf
    assert idx.tolist() == [[3, 7, 6, 2, 5, 0, 1, 8, 4]]
    assert torch.equal(tok, idx)
    assert torch.isnan(vals[0, :2]).all()
    assert vals[0, 2:].tolist() == [inf, 1.0, 1.0, 0.0, -0.0, -0.0, -inf]
    _, idx3, _ = beam.row_topk(x, 3)
    assert idx3.tolist() == [[3, 7, 6]]


def test_unfused_mask_matches_scalar_rule_and_hand_case():
    """trie_mask_candidates against cand_ok() element by element (random
    tables with out-of-table tokens, unconstrained nodes, NaN scores), and a
    hand-worked case."""
    g = torch.Generator().manual_seed(21)
    rows, cols, n_nodes, vsz, base = 12, 9, 7, 10, 100
    scores = torch.randn(rows, cols, generator=g)
    scores[0, 0] = float("nan")
    toks = base + torch.randint(-2, vsz + 2, (rows, cols), generator=g)
    nodes = torch.randint(-1, n_nodes + 2, (rows,), generator=g)  # -1 and past the table
    allow = torch.rand(n_nodes, vsz, generator=g) < 0.5
    got = beam.trie_mask_candidates(scores, toks, nodes, allow, base)
    for r in range(rows):
        for c in range(cols):
            ok = beam.cand_ok(int(nodes[r]), int(toks[r, c]), allow, base)
            want = scores[r, c] if ok else torch.tensor(float("-inf"))
            assert torch.equal(got[r, c], want) or (torch.isnan(want) and torch.isnan(got[r, c]))
    # hand case: node 1 allows relative tokens 0 and 2 only
    allow2 = torch.tensor([[1, 1, 1], [1, 0, 1]], dtype=torch.bool)
    out = beam.trie_mask_candidates(torch.ones(1, 4), torch.tensor([[5, 6, 7, 9]]), torch.tensor([1]), allow2, 5)
    assert out.tolist() == [[1.0, float("-inf"), 1.0, float("-inf")]]


def test_unfused_advance_and_expand_match_scalar_rules():
    g = torch.Generator().manual_seed(22)
    bw, picks, n_nodes, vsz, base, invalid = 6, 10, 5, 8, 50, 99
    nodes = torch.randint(-1, n_nodes, (bw,), generator=g)
    parents = torch.randint(-2, bw + 2, (picks,), generator=g)  # clamped
    toks = base + torch.randint(-1, vsz + 1, (picks,), generator=g)
    nxt = torch.randint(0, n_nodes, (n_nodes, vsz), generator=g)
    got = beam.trie_advance_nodes(nodes, parents, toks, nxt, base, invalid)
    for i in range(picks):
        p = min(max(int(parents[i]), 0), bw - 1)
        assert int(got[i]) == beam.transition(int(nodes[p]), int(toks[i]), nxt, base, invalid)
    batched = beam.trie_advance_nodes_batched(nodes.view(2, 3), parents.view(2, 5).clamp(0, 2), toks.view(2, 5),
                                              nxt, base, invalid)
    for r in range(2):
        assert torch.equal(batched[r], beam.trie_advance_nodes(nodes.view(2, 3)[r], parents.view(2, 5)[r].clamp(0, 2),
                                                               toks.view(2, 5)[r], nxt, base, invalid))
    ti = torch.arange(12).view(3, 4)
    out = beam.beam_expand_token_ids(ti, torch.tensor([2, 0, 5]), torch.tensor([70, 71, 72]), 1)
    assert out.tolist() == [[8, 70, 10, 11], [0, 71, 2, 3], [8, 72, 10, 11]]
    out = beam.beam_expand_token_ids(ti, torch.tensor([1]), torch.tensor([9]), 4)  # appends a column
    assert out.tolist() == [[4, 5, 6, 7, 9]]
