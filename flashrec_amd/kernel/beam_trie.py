"""Fused trie mask + top-K + beam expand, interface of ``flashrec.kernel.beam_trie``.

Reference: python/flashrec/kernel/beam_trie.py:229-290 (result tuple,
workspace), :536-633 (``genrec_mask_topk_expand``).  Backed by the gfx950
kernels ``fr_genrec_mask_topk_expand`` (flashrec_amd/csrc/beam_trie.hip).
As in the reference's CUDA path, each beam's candidate row must be sorted
descending (it comes from a sorted per-row top-k), the expanded token plane
is written to a workspace ping-pong buffer (never the one it gathers from),
and ``inplace`` is not honoured (the reference honours it only in its
PyTorch branch).
"""

from __future__ import annotations

import warnings
from typing import Dict, NamedTuple, Optional, Tuple, Union

import torch

from flashrec_amd._lib import Unsupported, call, load, require_device, stream_of


class GenrecFusedResult(NamedTuple):
    vals: torch.Tensor
    parents: torch.Tensor
    tokens: torch.Tensor
    indices: torch.Tensor
    token_ids: Optional[torch.Tensor]
    node_ids: Optional[torch.Tensor]


class GenrecFusedWorkspace:
    """Named device buffers reused across steps, grown on demand
    (beam_trie.py:243-290): ``get`` returns a view of the first ``shape[0]``
    rows of a buffer whose trailing shape matches."""

    def __init__(self) -> None:
        self._bufs: Dict[str, torch.Tensor] = {}

    def get(self, name: str, shape: tuple, dtype: torch.dtype, device) -> torch.Tensor:
        shape = tuple(int(x) for x in shape)
        device = torch.device(device)
        if device.type == "cuda" and device.index is None:
            device = torch.device("cuda", torch.cuda.current_device())
        t = self._bufs.get(name)
        fits = (t is not None and t.dtype == dtype and t.device == device and t.ndim == len(shape)
                and tuple(t.shape[1:]) == shape[1:] and t.shape[0] >= shape[0])
        if not fits:
            rows = shape[0]
            if t is not None and t.dtype == dtype and t.device == device and tuple(t.shape[1:]) == shape[1:]:
                rows = max(rows, int(t.shape[0]))
            t = torch.empty((rows,) + shape[1:], dtype=dtype, device=device)
            self._bufs[name] = t
        return t[: shape[0]]

    def get_filled(self, name: str, shape: tuple, dtype: torch.dtype, device, value) -> torch.Tensor:
        before = self._bufs.get(name)
        view = self.get(name, shape, dtype, device)
        if before is None or before.data_ptr() != self._bufs[name].data_ptr():
            self._bufs[name].fill_(value)
        return view

    def pair(self, name: str, shape: tuple, dtype: torch.dtype, device) -> Tuple[torch.Tensor, torch.Tensor]:
        return self.get(f"{name}_a", shape, dtype, device), self.get(f"{name}_b", shape, dtype, device)


def _same(a: torch.Tensor, b: torch.Tensor) -> bool:
    return (a.dtype == b.dtype and a.device == b.device and a.shape == b.shape
            and a.data_ptr() == b.data_ptr() and a.stride() == b.stride())


def _pingpong(ws: GenrecFusedWorkspace, name: str, user: torch.Tensor, dtype) -> Tuple[torch.Tensor, torch.Tensor]:
    """(read, write) planes: the kernel never gathers from the plane it writes
    (beam_trie.py:371-386)."""
    a, b = ws.pair(name, tuple(user.shape), dtype, user.device)
    if _same(user, a):
        return a, b
    if _same(user, b):
        return b, a
    return user, (b if user.data_ptr() == a.data_ptr() else a)


def _i64(t: torch.Tensor) -> torch.Tensor:
    t = t if t.dtype == torch.int64 else t.to(torch.int64)
    return t if t.is_contiguous() else t.contiguous()


def genrec_mask_topk_expand(
    cum: torch.Tensor,
    top_logprobs: torch.Tensor,
    top_tokens: torch.Tensor,
    *,
    select_k: int,
    node_ids: Optional[torch.Tensor] = None,
    allow_table: Optional[torch.Tensor] = None,
    token_base: int = 0,
    token_ids: Optional[torch.Tensor] = None,
    col: Union[int, torch.Tensor] = 0,
    next_node: Optional[torch.Tensor] = None,
    invalid_node: int = 0,
    do_expand: Optional[torch.Tensor] = None,
    apply_mask: bool = True,
    apply_expand: bool = True,
    apply_advance: bool = True,
    inplace: bool = False,
    workspace: Optional[GenrecFusedWorkspace] = None,
) -> GenrecFusedResult:
    """Mask + top-K + expand/advance (beam_trie.py:536-633).

    cum [N, BW] fp32, top_logprobs [N, BW, C] fp32 (rows sorted descending),
    top_tokens [N, BW, C]; node_ids [N, BW]; allow_table [nodes, vsz]
    bool/uint8; token_ids [N, BW, L]; next_node [nodes, vsz]; col int or [N].
    """
    del inplace
    require_device(cum, top_logprobs, top_tokens)
    n, bw = int(cum.shape[0]), int(cum.shape[1])
    c = int(top_logprobs.shape[2])
    k = int(select_k)
    dev = cum.device
    mask_i = int(bool(apply_mask and node_ids is not None and allow_table is not None))
    expand_i = int(bool(apply_expand and token_ids is not None))
    advance_i = int(bool(apply_advance and mask_i and expand_i and next_node is not None))
    ws = workspace if workspace is not None else GenrecFusedWorkspace()
    vals = ws.get("vals", (n, k), torch.float32, dev)
    parents = ws.get("parents", (n, k), torch.int64, dev)
    tokens = ws.get("sel_tokens", (n, k), torch.int64, dev)
    indices = ws.get("indices", (n, k), torch.int64, dev)
    if n == 0:
        return GenrecFusedResult(vals, parents, tokens, indices, None, None)
    nbytes = int(load().fr_genrec_scratch_bytes(n, bw, k))
    if nbytes < 0:
        raise ValueError(f"select_k={k} outside 1..1024")
    scratch = ws.get("scratch", (max(nbytes, 8),), torch.uint8, dev)
    cum_c = cum.to(torch.float32).contiguous()
    lp_c = top_logprobs.to(torch.float32).contiguous()
    tok_c = _i64(top_tokens)
    node_in = allow = None
    n_nodes = vsz = 0
    if mask_i:
        node_in = _i64(node_ids)
        allow = allow_table.view(torch.uint8) if allow_table.dtype == torch.bool else allow_table
        if allow.dtype != torch.uint8:
            raise TypeError(f"allow_table dtype must be bool/uint8, got {allow_table.dtype}")
        allow = allow.contiguous()
        n_nodes, vsz = int(allow.shape[0]), int(allow.shape[1])
    tok_in = tok_out = None
    width = 0
    if expand_i:
        tok_in, tok_out = _pingpong(ws, "tok", _i64(token_ids), torch.int64)
        width = int(tok_in.shape[-1])
    if (isinstance(col, torch.Tensor) and col.device == dev and col.dtype == torch.int32
            and col.is_contiguous() and col.numel() == n):
        col_t = col  # read only (const int32_t* col): no staging copy
    else:
        col_t = ws.get("col", (n,), torch.int32, dev)
        if isinstance(col, torch.Tensor):
            src = col.to(device=dev, dtype=torch.int32).reshape(-1)
            col_t.copy_(src.expand(n) if src.numel() == 1 else src[:n])
        else:
            col_t.fill_(int(col))
    do_exp = None
    if do_expand is not None:
        do_exp = do_expand.to(device=dev, dtype=torch.uint8).reshape(-1).contiguous()
    nxt = node_out = None
    next_i32 = 0
    if advance_i:
        # the trie keeps next_node as int32 (trie.py:220): read it as is
        # rather than widening the whole table every step
        if next_node.dtype == torch.int32:
            nxt, next_i32 = next_node.contiguous(), 1
        else:
            nxt = _i64(next_node)
        node_in, node_out = _pingpong(ws, "node", node_in, torch.int64)
        if int(nxt.shape[1]) != vsz or int(nxt.shape[0]) != n_nodes:
            raise ValueError("next_node and allow_table shapes differ")

    def p(t):
        return 0 if t is None else t.data_ptr()

    call("fr_genrec_mask_topk_expand",
         vals.data_ptr(), parents.data_ptr(), tokens.data_ptr(), indices.data_ptr(),
         scratch.data_ptr(), int(scratch.numel()),
         cum_c.data_ptr(), lp_c.data_ptr(), tok_c.data_ptr(), p(node_in), p(allow),
         p(tok_in), p(tok_out), p(nxt), p(node_out), p(do_exp), col_t.data_ptr(),
         int(token_base), n_nodes, vsz, int(invalid_node), n, bw, c, k, width,
         mask_i, expand_i, advance_i, next_i32, stream_of(cum))
    return GenrecFusedResult(vals, parents, tokens, indices,
                             tok_out if expand_i else None, node_out if advance_i else None)


def row_topk(
    scores: torch.Tensor,
    k: int,
    cand_ids: Optional[torch.Tensor] = None,
    *,
    out: Optional[Tuple[torch.Tensor, Optional[torch.Tensor]]] = None,
    out_tokens: Optional[torch.Tensor] = None,
    need_idx: bool = True,
    log_softmax: bool = False,
) -> Tuple[torch.Tensor, Optional[torch.Tensor], torch.Tensor]:
    """Sorted top-``k`` over the last dim of fp32 ``scores`` [..., V] and the
    candidate-id gather: (vals, idx, tokens) with tokens = cand_ids[idx] (idx
    when cand_ids is None).  Stands for ``torch.topk(..., sorted=True)`` +
    ``fill_topk_tokens`` (scheduler.py:1476-1481, graph.py:33-43, :186-193);
    equal scores come out by ascending index, NaN first.  ``out`` / ``out_tokens``
    are caller-owned buffers (graph-capture safe), as in graph.py:186-193.
    With ``need_idx=False`` the column indices are not written and idx is
    None (the beam step consumes only scores and tokens).
    With ``log_softmax=True`` ``scores`` are logits and the top-``k`` is taken
    over ``log_softmax(scores, -1)`` (logits.py:118-120 then the top-k),
    bit-identical to ``log_softmax_f32`` then ``row_topk``; for V = 4096 and
    8192 the log-probs are formed in registers and never written
    (``fr_log_softmax_row_topk``), other widths run the two calls.
    k <= min(V, 1024), V <= 16384."""
    require_device(scores)
    if scores.dtype != torch.float32:
        raise TypeError(f"row_topk takes fp32 scores, got {scores.dtype}")
    v = int(scores.shape[-1])
    x = scores.reshape(-1, v)
    if x.stride(-1) != 1:
        x = x.contiguous()
    r = int(x.shape[0])
    shape = tuple(scores.shape[:-1]) + (int(k),)
    if out is not None:
        vals, idx = out
    else:
        vals = torch.empty(shape, dtype=torch.float32, device=scores.device)
        idx = torch.empty(shape, dtype=torch.int64, device=scores.device) if need_idx else None
    if not need_idx:
        idx = None
    tokens = out_tokens if out_tokens is not None else torch.empty(shape, dtype=torch.int64,
                                                                   device=scores.device)
    for t, dt in ((vals, torch.float32), (idx, torch.int64), (tokens, torch.int64)):
        if t is not None and (t.dtype != dt or not t.is_contiguous() or t.numel() != r * int(k)):
            raise ValueError("row_topk output buffers must be contiguous [..., k] fp32/int64")
    cid = None
    if cand_ids is not None:
        cid = _i64(cand_ids.reshape(-1))
        if int(cid.numel()) < v:
            raise ValueError(f"cand_ids has {cid.numel()} entries for {v} columns")
    ldx = x.stride(0) if r > 1 else v
    outs = (0 if cid is None else cid.data_ptr(), vals.data_ptr(), 0 if idx is None else idx.data_ptr(),
            tokens.data_ptr(), stream_of(scores))
    if log_softmax:
        try:
            call("fr_log_softmax_row_topk", x.data_ptr(), ldx, r, v, int(k), *outs)
            return vals, idx, tokens
        except Unsupported:
            from flashrec_amd.kernel.sglops import log_softmax_f32

            x = log_softmax_f32(x)
            ldx = x.stride(0) if r > 1 else v
    call("fr_row_topk", x.data_ptr(), ldx, r, v, int(k), *outs)
    return vals, idx, tokens


# ---------------------------------------------------------------------------
# The rest of the reference module's interface (beam_trie.py:82-229, 302-353,
# 633-690): the unfused trie steps that search/trie.py and search/state.py
# call, the aliasing helpers the scheduler uses for its ping-pong stacks, and
# the graph-capture entry into caller-owned buffers.

tensors_alias = _same  # same storage, dtype, device, shape and strides (beam_trie.py:302-310)


def row_aliases_stack(row: Optional[torch.Tensor], stacked_row: torch.Tensor) -> bool:
    return row is not None and tensors_alias(row, stacked_row)


def rows_alias_stack(rows, stacked: torch.Tensor) -> bool:
    """Whether ``rows[i]`` is exactly ``stacked[i]`` for every row (beam_trie.py:319-325)."""
    return len(rows) == int(stacked.shape[0]) and all(
        row_aliases_stack(r, stacked[i]) for i, r in enumerate(rows))


def pick_pingpong_stack(ws: GenrecFusedWorkspace, name: str, rows, shape: tuple, dtype: torch.dtype,
                        device) -> torch.Tensor:
    """The workspace plane already holding ``rows`` (no copy), else plane ``a``
    with the rows copied in (beam_trie.py:328-352)."""
    planes = ws.pair(name, shape, dtype, device)
    for plane in planes:
        if rows_alias_stack(rows, plane):
            return plane
    a = planes[0]
    for i in range(int(shape[0])):
        if rows[i] is None:
            raise ValueError(f"{name}: missing row {i}")
        a[i].copy_(rows[i])
    return a


def try_load_beam_trie() -> bool:
    """True when the HIP kernels can run here (a GPU and the library)."""
    if not torch.cuda.is_available():
        return False
    try:
        load()
    except Exception:
        return False
    return True


def _u8_table(table: torch.Tensor) -> torch.Tensor:
    t = table.view(torch.uint8) if table.dtype == torch.bool else table
    if t.dtype != torch.uint8:
        raise TypeError(f"allow_table must be bool or uint8, got {table.dtype}")
    return t.contiguous()


def trie_mask_candidates(scores: torch.Tensor, cand_tokens: torch.Tensor, node_ids: torch.Tensor,
                         allow_table: torch.Tensor, token_base: int, out: Optional[torch.Tensor] = None,
                         neg_inf: float = float("-inf")) -> torch.Tensor:
    """``scores[r, c]`` where token ``cand_tokens[r, c]`` is allowed under trie
    node ``node_ids[r]``, ``neg_inf`` elsewhere (beam_trie.py:82-117)."""
    require_device(scores, cand_tokens, node_ids, allow_table)
    if scores.dim() != 2 or tuple(cand_tokens.shape) != tuple(scores.shape):
        raise ValueError("scores and cand_tokens must be [rows, cols] of one shape")
    rows, cols = int(scores.shape[0]), int(scores.shape[1])
    if int(node_ids.numel()) != rows:
        raise ValueError(f"node_ids has {node_ids.numel()} entries for {rows} rows")
    sc = scores.to(torch.float32).contiguous()
    out = torch.empty_like(sc) if out is None else out
    if out.dtype != torch.float32 or tuple(out.shape) != (rows, cols) or not out.is_contiguous():
        raise ValueError("out must be a contiguous fp32 tensor of the scores' shape")
    allow = _u8_table(allow_table)
    call("fr_trie_mask_candidates", out.data_ptr(), sc.data_ptr(), _i64(cand_tokens).data_ptr(),
         _i64(node_ids.reshape(-1)).data_ptr(), allow.data_ptr(), rows, cols, int(allow.shape[0]),
         int(allow.shape[1]), int(token_base), float(neg_inf), stream_of(sc))
    return out


def _advance(node_ids, parents, tokens, next_node, token_base, invalid_node, out, batch, rows, picks):
    require_device(node_ids, parents, tokens, next_node)
    if next_node.dtype not in (torch.int32, torch.int64):
        raise TypeError(f"next_node must be int32 or int64, got {next_node.dtype}")
    nxt = next_node.contiguous()
    par = _i64(parents.to(device=node_ids.device).reshape(batch, picks))
    tok = _i64(tokens.to(device=node_ids.device).reshape(batch, picks))
    if out is None:
        out = torch.empty((batch, picks), dtype=torch.int64, device=node_ids.device)
    if out.dtype != torch.int64 or out.numel() != batch * picks or not out.is_contiguous():
        raise ValueError("out must be a contiguous int64 tensor with one entry per pick")
    call("fr_trie_advance_nodes", out.data_ptr(), _i64(node_ids).data_ptr(), par.data_ptr(), tok.data_ptr(),
         nxt.data_ptr(), int(nxt.dtype == torch.int32), batch, rows, picks, int(nxt.shape[0]),
         int(nxt.shape[1]), int(token_base), int(invalid_node), stream_of(node_ids))
    return out


def trie_advance_nodes(node_ids: torch.Tensor, parents: torch.Tensor, tokens: torch.Tensor,
                       next_node: torch.Tensor, token_base: int, invalid_node: int,
                       out: Optional[torch.Tensor] = None) -> torch.Tensor:
    """Each pick's new trie node: its parent beam's node stepped on its token
    (beam_trie.py:120-162); ``node_ids`` [rows], ``parents`` / ``tokens`` [picks]."""
    picks = int(parents.numel())
    res = _advance(node_ids, parents, tokens, next_node, token_base, invalid_node,
                   None if out is None else out.view(1, -1), 1, int(node_ids.numel()), picks)
    return res.view(picks) if out is None else out


def trie_advance_nodes_batched(node_ids: torch.Tensor, parents: torch.Tensor, tokens: torch.Tensor,
                               next_node: torch.Tensor, token_base: int, invalid_node: int,
                               out: Optional[torch.Tensor] = None) -> torch.Tensor:
    """Per request: ``node_ids`` [n, bw], ``parents`` / ``tokens`` [n, k]
    (beam_trie.py:165-192); a 1-D ``node_ids`` is the unbatched form."""
    if node_ids.dim() == 1:
        return trie_advance_nodes(node_ids, parents, tokens, next_node, token_base, invalid_node, out)
    n, bw = int(node_ids.shape[0]), int(node_ids.shape[1])
    picks = int(parents.numel()) // max(n, 1)
    res = _advance(node_ids, parents, tokens, next_node, token_base, invalid_node, out, n, bw, picks)
    return res.view(n, picks)


def beam_expand_token_ids(token_ids: torch.Tensor, parents: torch.Tensor, new_tokens: torch.Tensor, col: int,
                          out: Optional[torch.Tensor] = None) -> torch.Tensor:
    """Token rows of the picks: row ``parents[p]`` of ``token_ids`` [rows,
    width] with column ``col`` set to ``new_tokens[p]`` (beam_trie.py:195-228;
    ``col == width`` appends the column, as the reference's PyTorch branch
    does).  int64 tokens."""
    require_device(token_ids, parents, new_tokens)
    if token_ids.dim() != 2:
        raise ValueError("token_ids must be [rows, width]")
    rows, width = int(token_ids.shape[0]), int(token_ids.shape[1])
    col = int(col)
    if col < 0 or col > width:
        raise IndexError(f"col {col} outside 0..{width}")
    par = _i64(parents.to(device=token_ids.device).reshape(-1))
    picks = int(par.numel())
    toks = _i64(new_tokens.to(device=token_ids.device).reshape(-1))
    if int(toks.numel()) != picks:
        raise ValueError("one new token per parent")
    src = _i64(token_ids)
    shape = (picks, max(width, col + 1))
    if out is None:
        out = torch.empty(shape, dtype=torch.int64, device=token_ids.device)
    if out.dtype != torch.int64 or tuple(out.shape) != shape or not out.is_contiguous():
        raise ValueError(f"out must be a contiguous int64 tensor of shape {shape}")
    if picks and rows == 0:
        raise IndexError("no token rows to gather from")
    call("fr_beam_expand_token_ids", out.data_ptr(), src.data_ptr(), par.data_ptr(), toks.data_ptr(), rows, width,
         picks, col, stream_of(src))
    return out if token_ids.dtype == torch.int64 else out.to(token_ids.dtype)


def call_genrec_cuda(out_vals, out_parents, out_tokens, out_indices, scratch, cum, top_logprobs, top_tokens,
                     node_in, allow_u8, tok_in, tok_out, next_node, node_out, do_exp, token_base: int,
                     invalid_node: int, col_t, apply_mask: int = 1, apply_expand: int = 1,
                     apply_advance: int = 1) -> bool:
    """The fused step into caller-owned buffers, graph-capture safe
    (beam_trie.py:633-684): K is ``out_vals.shape[1]``.  The caller's
    ``scratch`` (the reference sizes it [N, BW * C] fp32) is used when it is
    large enough; otherwise the library's static per-device scratch
    (``fr_genrec_mask_topk_expand_noalloc``).  Returns False when neither fits."""
    lib = load()
    n, bw = int(cum.shape[0]), int(cum.shape[1])
    c = int(top_logprobs.shape[2])
    k = int(out_vals.shape[1])
    width = int(tok_in.shape[-1]) if tok_in is not None else 0
    allow = _u8_table(allow_u8) if allow_u8 is not None else None
    next_i32 = int(next_node is not None and next_node.dtype == torch.int32)

    def p(t):
        return 0 if t is None else t.data_ptr()

    args = (p(cum), p(top_logprobs), p(top_tokens), p(node_in), p(allow), p(tok_in), p(tok_out), p(next_node),
            p(node_out), p(do_exp), p(col_t), int(token_base), 0 if allow is None else int(allow.shape[0]),
            0 if allow is None else int(allow.shape[1]), int(invalid_node), n, bw, c, k, width,
            int(apply_mask), int(apply_expand), int(apply_advance), next_i32, stream_of(cum))
    head = (p(out_vals), p(out_parents), p(out_tokens), p(out_indices))
    need = int(lib.fr_genrec_scratch_bytes(n, bw, k))
    if need < 0:
        return False
    have = 0 if scratch is None else int(scratch.numel()) * scratch.element_size()
    if have >= need:
        rc = lib.fr_genrec_mask_topk_expand(*head, scratch.data_ptr(), have, *args)
    else:
        global _warned_static_scratch
        if not _warned_static_scratch:
            # the static array is one per GPU: beam steps running on two
            # streams at once would overwrite each other's slice lists
            warnings.warn(f"genrec scratch of {have} bytes is below the {need} needed; using the library's "
                          "static per-GPU scratch, which concurrent beam steps on one GPU must not share",
                          RuntimeWarning, stacklevel=2)
            _warned_static_scratch = True
        rc = lib.fr_genrec_mask_topk_expand_noalloc(*head, *args)
    return rc == 0


_warned_static_scratch = False
