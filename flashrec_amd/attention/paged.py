"""Paged fp8 attention backend, interface of ``flashrec.attention.flashinfer``.

Reference: python/flashrec/attention/flashinfer.py:73-431 (``AttentionBackend``).
The reference plans FlashInfer wrappers per batch and runs them per layer; the
result it defines is that of its ``_sdpa`` fallback (:380-431).  Here the plan
is two int32 arrays per query token — where its slot list starts in
``kv_indices`` and how many slots it sees — and every layer runs the gfx950
kernel ``fr_paged_attention_fp8`` over the e4m3 pool.  The plan is built in
``prepare`` (outside graph capture, as the reference's is); under graph decode
it is written into persistent per-batch-size buffers, so ``forward`` allocates
only its output and can be captured.
"""

from __future__ import annotations

from typing import Dict, List, Optional, Tuple

import torch

from flashrec_amd._lib import Unsupported, call, load, require_device, stream_of


class AttentionBackend:
    """Drop-in for the reference backend (flashinfer.py:73-141): same
    constructor, ``prepare`` / ``forward`` and graph-decode hooks."""

    def __init__(
        self,
        kv_pool,
        num_qo_heads: int,
        num_kv_heads: int,
        head_dim: int,
        backend: str = "hip",
        fi_backend: str = "fa2",
    ):
        if num_qo_heads % num_kv_heads != 0:
            raise ValueError("num_qo_heads must be a multiple of num_kv_heads")
        if head_dim != 128:
            raise ValueError("the paged attention kernel takes head_dim 128")
        self.kv_pool = kv_pool
        self.num_qo_heads = int(num_qo_heads)
        self.num_kv_heads = int(num_kv_heads)
        self.head_dim = int(head_dim)
        self.n_rep = self.num_qo_heads // self.num_kv_heads
        self.device = kv_pool.device
        self.backend = backend
        self.fi_backend = fi_backend
        self.q_dtype = torch.bfloat16
        # the reference shares one workspace between prefill and decode when it
        # cannot allocate two; this backend has no workspace to overlap
        self.prefill_overlap_ok = True
        self.scale = self.head_dim ** -0.5
        self._plan: Optional[Dict[str, torch.Tensor]] = None
        self._graph_bufs: Dict[int, Dict[str, torch.Tensor]] = {}
        self._graph_bs: Optional[int] = None

    # ---------------------------------------------------------- graph decode
    def init_graph_wrappers(self, capture_bs: List[int], max_seq_len: int) -> None:
        """Persistent plan buffers per captured batch size (flashinfer.py:143-185)."""
        max_seq_len = max(int(max_seq_len), 1)
        for bs in capture_bs:
            bs = int(bs)
            if bs <= 0 or bs in self._graph_bufs:
                continue
            dev = self.device
            self._graph_bufs[bs] = {
                "indptr": torch.zeros(bs + 1, dtype=torch.int32, device=dev),
                "indices": torch.zeros(bs * max_seq_len, dtype=torch.int32, device=dev),
                "last": torch.ones(bs, dtype=torch.int32, device=dev),
                "kv_len": torch.zeros(bs, dtype=torch.int32, device=dev),
                "group_prefix": torch.zeros(max(plan_size(bs, self.num_qo_heads, self.num_kv_heads), 1),
                                            dtype=torch.int32, device=dev),
            }

    def graph_bufs(self, bs: int) -> Optional[dict]:
        return self._graph_bufs.get(int(bs))

    def begin_graph_decode(self, bs: int) -> None:
        if int(bs) not in self._graph_bufs:
            raise RuntimeError(f"no graph plan buffers for bs={bs}")
        self._graph_bs = int(bs)

    def end_graph_decode(self) -> None:
        self._graph_bs = None

    # ----------------------------------------------------------------- plan
    def prepare(self, batch) -> None:
        """Per-token slot ranges for every layer of this batch (flashinfer.py:201-210),
        and the shared-prefix plan of its query groups (one kernel, reused by
        every layer's attention)."""
        if batch.kv_indices is None:
            self._plan = None
            return
        if batch.is_prefill:
            self._plan = self._plan_prefill(batch)
        else:
            self._plan = self._plan_decode(batch)
        n = int(self._plan["start"].numel())
        bufs = self._graph_bufs.get(self._graph_bs) if self._graph_bs is not None else None
        gp = None
        if bufs is not None and not batch.is_prefill:
            gp = bufs["group_prefix"][: max(plan_size(n, self.num_qo_heads, self.num_kv_heads), 1)]
        self._plan["group_prefix"] = attention_plan(self._plan["indices"], self._plan["start"],
                                                    self._plan["len"], self.num_qo_heads,
                                                    self.num_kv_heads, out=gp)

    def _plan_decode(self, batch) -> Dict[str, torch.Tensor]:
        n = int(batch.n_rows)
        seq = batch.seq_lens.view(-1)[:n].to(device=self.device, dtype=torch.int32)
        kv = batch.kv_indices.view(-1)
        if kv.dtype != torch.int32:
            kv = kv.to(dtype=torch.int32)
        bufs = self._graph_bufs.get(self._graph_bs) if self._graph_bs is not None else None
        if bufs is not None:
            # indptr[0] stays 0 (zeros at creation); the cumsum fills [1:]
            torch.cumsum(seq, dim=0, out=bufs["indptr"][1 : n + 1])
            bufs["kv_len"][:n].copy_(seq)
            nidx = int(kv.numel())
            if nidx > 0 and kv.data_ptr() != bufs["indices"].data_ptr():
                bufs["indices"][:nidx].copy_(kv, non_blocking=True)
            return {"indices": bufs["indices"], "start": bufs["indptr"][:n], "len": bufs["kv_len"][:n]}
        indptr = batch.kv_indptr
        if indptr is None:
            indptr = torch.zeros(n + 1, dtype=torch.int32, device=self.device)
            torch.cumsum(seq, dim=0, out=indptr[1:])
        indptr = indptr.view(-1).to(device=self.device, dtype=torch.int32)
        return {"indices": kv.contiguous(), "start": indptr[:n].contiguous(), "len": seq.contiguous()}

    def _plan_prefill(self, batch) -> Dict[str, torch.Tensor]:
        """Causal prefill (flashinfer.py:351-378, :409-422): token j of a row with
        prefix P sees the row's first P + j + 1 slots."""
        n = int(batch.n_rows)
        seq = [int(x) for x in batch.seq_lens_cpu.view(-1)[:n].tolist()]
        ext = [int(e) for e in (batch.extend_seq_lens or [1] * n)]
        prefix = batch.extend_prefix_lens or [s - e for s, e in zip(seq, ext)]
        start: List[int] = []
        length: List[int] = []
        off = 0
        for i in range(n):
            for j in range(ext[i]):
                start.append(off)
                length.append(int(prefix[i]) + j + 1)
            off += seq[i]
        kv = batch.kv_indices.view(-1).to(device=self.device, dtype=torch.int32).contiguous()
        return {
            "indices": kv,
            "start": torch.tensor(start, dtype=torch.int32).to(self.device),
            "len": torch.tensor(length, dtype=torch.int32).to(self.device),
        }

    # ------------------------------------------------------------------ run
    @torch.compiler.disable
    def forward(self, q: torch.Tensor, k: torch.Tensor, v: torch.Tensor, layer_id: int, batch,
                skip_store: bool = False) -> torch.Tensor:
        """q/k/v: [T, H, D] (k/v kv-heads).  Writes the new KV, then attends
        (flashinfer.py:212-238).  Returns [T, Hq, D] bf16."""
        if not skip_store:
            self.kv_pool.store(layer_id, k, v, batch.out_cache_loc)
        if self._plan is None:
            raise RuntimeError("AttentionBackend.forward before prepare() (kv_indices required)")
        return paged_attention(q, self.kv_pool.k_cache(layer_id), self.kv_pool.v_cache(layer_id),
                               self._plan["indices"], self._plan["start"], self._plan["len"],
                               self.scale, group_prefix=self._plan.get("group_prefix"))


    @torch.compiler.disable
    def forward_quant_fp8(self, q: torch.Tensor, layer_id: int) -> Tuple[torch.Tensor, torch.Tensor]:
        """Attention over the stored KV fused with the o projection's per-token
        e4m3 quant: (codes [T, Hq * D], scales [T, 1]).  The new KV must be
        stored already (the fused QK-norm/RoPE/KV write does it)."""
        if self._plan is None:
            raise RuntimeError("AttentionBackend.forward_quant_fp8 before prepare() (kv_indices required)")
        return paged_attention_quant_fp8(q, self.kv_pool.k_cache(layer_id), self.kv_pool.v_cache(layer_id),
                                         self._plan["indices"], self._plan["start"], self._plan["len"],
                                         self.scale, group_prefix=self._plan.get("group_prefix"))


def plan_size(T: int, hq: int, hk: int) -> int:
    """Entries of an attention plan for T query tokens (groups of 32 / (hq / hk))."""
    n = int(load().fr_paged_attention_plan_size(int(T), int(hq), int(hk)))
    if n < 0:
        raise ValueError(f"unsupported head ratio {hq}/{hk}")
    return n


def attention_plan(kv_indices: torch.Tensor, kv_start: torch.Tensor, kv_len: torch.Tensor,
                   hq: int, hk: int, out: Optional[torch.Tensor] = None) -> torch.Tensor:
    """The shared slot prefix (rounded down to 32) of each group of 32 / (hq /
    hk) consecutive query tokens: computed once per batch, passed to every
    layer's ``paged_attention`` as ``group_prefix``."""
    require_device(kv_indices, kv_start, kv_len)
    T = int(kv_start.numel())
    n = plan_size(T, hq, hk)
    if out is None:
        out = torch.empty(max(n, 1), dtype=torch.int32, device=kv_start.device)
    if out.dtype != torch.int32 or not out.is_contiguous() or out.numel() < n:
        raise ValueError("plan buffer must be contiguous int32 with plan_size entries")
    call("fr_paged_attention_plan", kv_indices.data_ptr(), kv_start.data_ptr(), kv_len.data_ptr(),
         T, int(hq), int(hk), out.data_ptr(), stream_of(kv_start))
    return out


def _check_plan(group_prefix: Optional[torch.Tensor], T: int, hq: int, hk: int) -> int:
    """The plan's device pointer (0 for none) after checking it holds the
    entries the kernels read for T tokens."""
    if group_prefix is None:
        return 0
    n = plan_size(T, hq, hk)
    if group_prefix.dtype != torch.int32 or not group_prefix.is_contiguous() or group_prefix.numel() < n:
        raise ValueError(f"group_prefix must be a contiguous int32 plan of at least {n} entries "
                         "(attention_plan over the same slot lists)")
    require_device(group_prefix)
    return group_prefix.data_ptr()


def _check_attention_inputs(q, k_cache, v_cache, kv_indices, kv_start, kv_len):
    require_device(q, k_cache, v_cache, kv_indices, kv_start, kv_len)
    if q.dtype != torch.bfloat16:
        raise TypeError("paged_attention takes bf16 queries")
    if k_cache.dtype != torch.float8_e4m3fn or v_cache.dtype != torch.float8_e4m3fn:
        raise TypeError("paged_attention reads an e4m3 KV pool")
    for t in (kv_indices, kv_start, kv_len):
        if t.dtype != torch.int32 or not t.is_contiguous():
            raise TypeError("kv_indices / kv_start / kv_len must be contiguous int32")
    T, Hq, D = q.shape
    slots, Hk, Dk = k_cache.shape
    if Dk != D or v_cache.shape != k_cache.shape or q.stride(2) != 1:
        raise ValueError("q / cache shapes disagree")
    if k_cache.stride(2) != 1 or v_cache.stride(2) != 1:
        raise ValueError("caches need a unit inner stride")
    if kv_start.numel() < T or kv_len.numel() < T:
        raise ValueError("one kv_start / kv_len entry per query token")
    return T, Hq, D, slots, Hk


def paged_attention_quant_fp8(q: torch.Tensor, k_cache: torch.Tensor, v_cache: torch.Tensor,
                              kv_indices: torch.Tensor, kv_start: torch.Tensor, kv_len: torch.Tensor,
                              scale: float, group_prefix: Optional[torch.Tensor] = None,
                              out: Optional[torch.Tensor] = None, out_scale: Optional[torch.Tensor] = None
                              ) -> Tuple[torch.Tensor, torch.Tensor]:
    """``per_token_quant_fp8(paged_attention(...).reshape(T, -1))`` in one
    kernel: the o projection's e4m3 input ``[T, Hq * D]`` and its scales
    ``[T, 1]`` (qwen3.py:131-134 -> linear.py:118-151), bit-for-bit the two
    steps' result.  Head layouts the fused kernel does not take (more than 8
    kv heads, 8 query heads per kv head) run the two steps."""
    T, Hq, D, slots, Hk = _check_attention_inputs(q, k_cache, v_cache, kv_indices, kv_start, kv_len)
    if out is None:
        out = torch.empty(T, Hq * D, dtype=torch.float8_e4m3fn, device=q.device)
    if out_scale is None:
        out_scale = torch.empty(T, 1, dtype=torch.float32, device=q.device)
    if (out.dtype != torch.float8_e4m3fn or out.dim() != 2 or out.shape[0] != T or out.shape[1] != Hq * D
            or out.stride(1) != 1):
        raise ValueError("out must be [T, Hq * D] float8_e4m3fn with a unit inner stride")
    if out_scale.dtype != torch.float32 or out_scale.numel() != T or not out_scale.is_contiguous():
        raise ValueError("out_scale must hold T contiguous fp32 values")
    require_device(out, out_scale)
    try:
        call("fr_paged_attention_quant_fp8",
             q.data_ptr(), q.stride(0), q.stride(1),
             k_cache.data_ptr(), k_cache.stride(0), k_cache.stride(1),
             v_cache.data_ptr(), v_cache.stride(0), v_cache.stride(1),
             slots, kv_indices.data_ptr(), kv_start.data_ptr(), kv_len.data_ptr(),
             out.data_ptr(), out.stride(0), out_scale.data_ptr(),
             T, Hq, Hk, D, float(scale), _check_plan(group_prefix, T, Hq, Hk), stream_of(q))
    except Unsupported:
        from flashrec_amd.kernel.sglops import per_token_quant_fp8

        o = paged_attention(q, k_cache, v_cache, kv_indices, kv_start, kv_len, scale, group_prefix=group_prefix)
        codes, s = per_token_quant_fp8(o.reshape(T, Hq * D))
        out.copy_(codes)
        out_scale.copy_(s.reshape(out_scale.shape))
    return out, out_scale


def paged_attention(q: torch.Tensor, k_cache: torch.Tensor, v_cache: torch.Tensor,
                    kv_indices: torch.Tensor, kv_start: torch.Tensor, kv_len: torch.Tensor,
                    scale: float, out: Optional[torch.Tensor] = None,
                    group_prefix: Optional[torch.Tensor] = None) -> torch.Tensor:
    """softmax(q k^T * scale) v over each query token's slot list.

    q: [T, Hq, 128] bf16 (unit inner stride); k_cache / v_cache: [slots, Hk,
    128] float8_e4m3fn; kv_indices / kv_start / kv_len: int32 on the device.
    group_prefix: the plan of ``attention_plan`` for the same slot lists, or
    None (each call then finds the shared prefixes itself).
    """
    T, Hq, D, slots, Hk = _check_attention_inputs(q, k_cache, v_cache, kv_indices, kv_start, kv_len)
    if out is None:
        out = torch.empty(T, Hq, D, dtype=torch.bfloat16, device=q.device)
    call("fr_paged_attention_fp8",
         q.data_ptr(), q.stride(0), q.stride(1),
         k_cache.data_ptr(), k_cache.stride(0), k_cache.stride(1),
         v_cache.data_ptr(), v_cache.stride(0), v_cache.stride(1),
         slots, kv_indices.data_ptr(), kv_start.data_ptr(), kv_len.data_ptr(),
         out.data_ptr(), out.stride(0), out.stride(1),
         T, Hq, Hk, D, float(scale), _check_plan(group_prefix, T, Hq, Hk), stream_of(q))
    return out
