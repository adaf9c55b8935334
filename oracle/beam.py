"""Torch-CPU restatement of the beam step: the per-row candidate top-k, then
the fused trie mask -> top-K -> expand -> advance.  TEST INFRASTRUCTURE ONLY (see ``oracle/__init__.py``).

python/flashrec/kernel/beam_trie.py:585-633 (the PyTorch branch, the source
of correctness) fixes the arithmetic: scores = cum + top_logprobs, masked to
-inf by the trie rule of :87-112, flat top-K over BW*C per request, parents =
index // C, tokens gathered, token rows expanded (:437-451), nodes advanced
(:155-181).  What the branch leaves to torch.topk's internals is taken from
the reference's CUDA kernel (csrc/beam_trie.cuh:548-757): ties rank by flat
index ascending; with masking on, masked candidates are never picked and
missing picks are (-inf, index 0, parent 0, token top_tokens[n, 0, 0]); rows
b >= K of the token and node planes are copied; nothing is expanded or
advanced for a request whose do_expand is 0.  NaN scores count as masked.
"""

from __future__ import annotations

from typing import Optional, Union

import torch

NEG_INF = float("-inf")


def cand_ok(node: int, tok: int, allow: torch.Tensor, token_base: int) -> bool:
    """beam_trie.cuh:37-49 (and beam_trie.py:104-112)."""
    if node < 0:
        return True
    n_nodes, vsz = allow.shape
    rel = tok - token_base
    if rel < 0 or rel >= vsz or n_nodes <= 0:
        return False
    return bool(allow[min(max(node, 0), n_nodes - 1), rel])


def transition(old: int, tok: int, next_node: torch.Tensor, token_base: int, invalid: int) -> int:
    """beam_trie.cuh:51-64 (and beam_trie.py:172-181)."""
    if old < 0:
        return old
    n_nodes, vsz = next_node.shape
    rel = tok - token_base
    if rel < 0 or rel >= vsz or n_nodes <= 0:
        return invalid
    return int(next_node[min(old, n_nodes - 1), rel])


def genrec_mask_topk_expand(cum, top_logprobs, top_tokens, select_k, node_ids=None, allow_table=None,
                            token_base=0, token_ids=None, col: Union[int, torch.Tensor] = 0,
                            next_node=None, invalid_node=0, do_expand: Optional[torch.Tensor] = None,
                            apply_mask=True, apply_expand=True, apply_advance=True):
    n, bw = cum.shape
    c = top_logprobs.shape[2]
    k = int(select_k)
    mask = bool(apply_mask and node_ids is not None and allow_table is not None)
    expand = bool(apply_expand and token_ids is not None)
    advance = bool(apply_advance and mask and expand and next_node is not None)
    scores = (cum.float()[:, :, None] + top_logprobs.float()).reshape(n, bw * c)
    toks = top_tokens.long().reshape(n, bw * c)
    valid = ~torch.isnan(scores)
    if mask:
        allow = allow_table.bool()
        n_nodes, vsz = allow.shape
        node = node_ids.long()[:, :, None].expand(n, bw, c).reshape(n, bw * c)
        rel = toks - int(token_base)
        in_range = (rel >= 0) & (rel < vsz) & (n_nodes > 0)
        ok = allow[node.clamp(0, max(n_nodes - 1, 0)), rel.clamp(0, max(vsz - 1, 0))] & in_range
        ok = ok | (node < 0)
        valid &= ok & (scores != NEG_INF)
    vals = torch.full((n, k), NEG_INF, dtype=torch.float32)
    indices = torch.zeros(n, k, dtype=torch.int64)
    for r in range(n):
        idx = torch.nonzero(valid[r]).reshape(-1)
        # score descending, ties by flat index ascending (stable sort of the
        # index-ordered candidates)
        order = torch.sort(scores[r, idx], descending=True, stable=True).indices
        take = idx[order][:k]
        vals[r, : take.numel()] = scores[r, take]
        indices[r, : take.numel()] = take
    got = valid.sum(1).clamp(max=k)
    parents = torch.where(torch.arange(k)[None, :] < got[:, None], indices // c, torch.zeros_like(indices))
    tokens = toks.gather(1, indices)
    tok_out = token_ids.clone().long() if expand else None
    node_out = node_ids.clone().long() if advance else None
    if expand:
        cols = col.reshape(-1).long() if isinstance(col, torch.Tensor) else torch.full((n,), int(col))
        if cols.numel() == 1:
            cols = cols.expand(n)
        width = token_ids.shape[2]
        kk = min(k, bw)
        for r in range(n):
            if do_expand is not None and int(do_expand.reshape(-1)[r]) == 0:
                continue
            par = parents[r, :kk].clamp(0, bw - 1)
            rows = token_ids[r, par].clone().long()
            colr = max(int(cols[r]), 0)
            if colr < width:
                rows[:, colr] = tokens[r, :kk]
            tok_out[r, :kk] = rows
            if advance:
                for b in range(kk):
                    node_out[r, b] = transition(int(node_ids[r, int(par[b])]), int(tokens[r, b]),
                                                next_node.long(), token_base, invalid_node)
    return vals, parents, tokens, indices, tok_out, node_out


def row_topk(x: torch.Tensor, k: int, cand_ids: Optional[torch.Tensor] = None):
    """Sorted per-row top-k with the candidate-id gather (scheduler.py:1476-1481,
    graph.py:33-43): the stable descending sort's first k, i.e. equal scores
    by ascending index, NaN first (torch's ordering).  Returns (vals, idx,
    tokens) where tokens = cand_ids[idx] (idx when cand_ids is None)."""
    x2 = x.float().reshape(-1, x.shape[-1])
    vals, idx = torch.sort(x2, dim=-1, descending=True, stable=True)
    vals, idx = vals[:, :k], idx[:, :k]
    tokens = cand_ids.long()[idx] if cand_ids is not None else idx.clone()
    shape = tuple(x.shape[:-1]) + (k,)
    return vals.reshape(shape), idx.reshape(shape), tokens.reshape(shape)


# ---------------------------------------------------------------- unfused steps
def trie_mask_candidates(scores, cand_tokens, node_ids, allow_table, token_base, neg_inf=NEG_INF):
    """python/flashrec/kernel/beam_trie.py:105-117 (PyTorch branch): scores
    [rows, cols] kept where cand_ok(node_ids[row], token), else neg_inf."""
    allow = allow_table.bool()
    n_nodes, vsz = allow.shape
    rel = cand_tokens.long() - int(token_base)
    in_range = (rel >= 0) & (rel < vsz)
    node = node_ids.long().reshape(-1, 1).expand_as(rel)
    if n_nodes > 0 and vsz > 0:
        ok = allow[node.clamp(0, n_nodes - 1), rel.clamp(0, vsz - 1)] & in_range
    else:
        ok = torch.zeros_like(in_range)
    ok = ok | (node < 0)
    return scores.float().masked_fill(~ok, neg_inf)


def trie_advance_nodes(node_ids, parents, tokens, next_node, token_base, invalid_node):
    """python/flashrec/kernel/beam_trie.py:145-162 (PyTorch branch), one
    plane: new node of each pick = transition(node_ids[clamp(parent)], token)."""
    n_nodes, vsz = next_node.shape
    par = parents.long().reshape(-1).clamp(0, max(int(node_ids.numel()) - 1, 0))
    old = node_ids.long().reshape(-1)[par]
    rel = tokens.long().reshape(-1) - int(token_base)
    in_range = (rel >= 0) & (rel < vsz) & (n_nodes > 0)
    if n_nodes > 0 and vsz > 0:
        nxt = next_node.long()[old.clamp(0, n_nodes - 1), rel.clamp(0, vsz - 1)]
    else:
        nxt = torch.zeros_like(old)
    nxt = torch.where(in_range, nxt, torch.full_like(nxt, int(invalid_node)))
    return torch.where(old < 0, old, nxt)


def trie_advance_nodes_batched(node_ids, parents, tokens, next_node, token_base, invalid_node):
    """python/flashrec/kernel/beam_trie.py:165-192: one plane per request."""
    return torch.stack([trie_advance_nodes(node_ids[r], parents[r], tokens[r], next_node, token_base, invalid_node)
                        for r in range(int(node_ids.shape[0]))])


def beam_expand_token_ids(token_ids, parents, new_tokens, col):
    """python/flashrec/kernel/beam_trie.py:218-228 (PyTorch branch)."""
    par = parents.long().reshape(-1).clamp(0, max(int(token_ids.shape[0]) - 1, 0))
    rows = token_ids[par].clone()
    if col >= rows.shape[1]:
        rows = torch.nn.functional.pad(rows, (0, 1))
    rows[:, col] = new_tokens.reshape(-1).to(rows.dtype)
    return rows
