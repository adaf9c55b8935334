"""One decode step of a Qwen3-shaped decoder on the FP8 path, composed from
the drop-in operators in the call order of the reference model.

Reference: python/flashrec/models/qwen3.py:36-136 (attention block), :138-171
(MLP), :173-223 (decoder layer, fused RMSNorm->fp8 path), :225-320 (model:
layers, final norm), and python/flashrec/logits.py:118-166 (SID-restricted
lm_head + log_softmax; fp8 here).  Weights are either random (bf16 N(0, 0.02)
linear weights quantised per output channel with the path's own quantiser,
norm weights 1 + N(0, 0.1)) or loaded from a safetensors checkpoint by
``flashrec_amd.weight.load_weights``.  The batch is beam
decode: ``requests`` prompts of ``prefix`` tokens whose KV is written once and
shared by each request's ``beams`` rows, plus ``step`` decoded tokens per row.

Everything a step launches is graph-capturable (no allocation inside the
kernels, no host reads of device data): ``capture()`` records the whole step
into one HIP graph, the path's answer to the reference's CUDA-graph decode
(python/flashrec/engine/graph.py:224-355).
"""

from __future__ import annotations

from dataclasses import dataclass
from typing import List, Optional

import torch

from flashrec_amd.attention.paged import AttentionBackend
from flashrec_amd.kernel.qk_rope_kv import fused_qk_norm_rope_store_fp8
from flashrec_amd.kernel.sglops import per_token_quant_fp8
from flashrec_amd.kernel.silu_fp8 import silu_and_mul_per_token_quant_fp8
from flashrec_amd.kvcache.pool import TokenToKVPool
from flashrec_amd.layers.linear import Linear
from flashrec_amd.layers.norm import RMSNorm
from flashrec_amd.layers.rotary import RotaryEmbedding
from flashrec_amd.logits import RestrictedLMHead


@dataclass
class Qwen3Shape:
    """Qwen3-1.7B shape (the config-4 decode step: 28 layers, 16 q / 8 kv heads of 128)."""

    hidden: int = 2048
    intermediate: int = 6144
    layers: int = 28
    q_heads: int = 16
    kv_heads: int = 8
    head_dim: int = 128
    eps: float = 1e-6
    rope_theta: float = 1e6
    max_position: int = 4096
    sid_tokens: int = 8192
    vocab: int = 151936
    tie_word_embeddings: bool = True


class _Batch:
    """The ForwardBatch fields (python/flashrec/core.py:80-104) a decode step reads."""

    def __init__(self, **kw):
        self.__dict__.update(kw)

    @property
    def n_rows(self) -> int:
        return int(self.seq_lens.numel())


class _Layer:
    """One decoder layer's weights, empty until loaded or initialised."""

    def __init__(self, shape: Qwen3Shape, layer_id: int):
        h, d = shape.hidden, shape.head_dim
        nq, nk = shape.q_heads, shape.kv_heads
        self.layer_id = layer_id
        self.qkv_proj = Linear(h, (nq + 2 * nk) * d)
        self.o_proj = Linear(nq * d, h)
        self.gate_up_proj = Linear(h, 2 * shape.intermediate)
        self.down_proj = Linear(shape.intermediate, h)
        self.input_layernorm = RMSNorm(h, shape.eps)
        self.post_attention_layernorm = RMSNorm(h, shape.eps)
        self.q_norm = RMSNorm(d, shape.eps)
        self.k_norm = RMSNorm(d, shape.eps)

    def linears(self):
        """(reference module name under ``layers.<i>.``, module)."""
        return (("self_attn.qkv_proj", self.qkv_proj), ("self_attn.o_proj", self.o_proj),
                ("mlp.gate_up_proj", self.gate_up_proj), ("mlp.down_proj", self.down_proj))

    def norms(self):
        return (("input_layernorm", self.input_layernorm),
                ("post_attention_layernorm", self.post_attention_layernorm),
                ("self_attn.q_norm", self.q_norm), ("self_attn.k_norm", self.k_norm))


class Qwen3FP8Weights:
    """The decoder's parameters under the reference's module names
    (qwen3.py:225-320): what ``flashrec_amd.weight.load_weights`` fills.
    Construction allocates nothing on the device."""

    def __init__(self, shape: Qwen3Shape):
        self.shape = shape
        self.layers: List[_Layer] = [_Layer(shape, i) for i in range(shape.layers)]
        self.final_norm = RMSNorm(shape.hidden, shape.eps)
        self.embed: Optional[torch.Tensor] = None
        self.lm_head_weight: Optional[torch.Tensor] = None
        self.tie_word_embeddings = shape.tie_word_embeddings

    def named_linears(self):
        for L in self.layers:
            for name, lin in L.linears():
                yield f"layers.{L.layer_id}.{name}", lin

    def named_norms(self):
        for L in self.layers:
            for name, n in L.norms():
                yield f"layers.{L.layer_id}.{name}", n
        yield "norm", self.final_norm

    @classmethod
    def random(cls, shape: Qwen3Shape, gen: torch.Generator, device) -> "Qwen3FP8Weights":
        """bf16 N(0, 0.02) linear weights quantised per output channel by the
        path's quantiser; norm weights 1 + N(0, 0.1); tied embedding N(0, 0.02)."""
        w = cls(shape)

        def norm_weight(n):
            return torch.nn.Parameter(
                (1.0 + 0.1 * torch.randn(n, generator=gen, device=device)).to(torch.bfloat16),
                requires_grad=False)

        for L in w.layers:
            for _, lin in L.linears():
                lin.load((torch.randn(lin.out_features, lin.in_features, generator=gen, device=device)
                          * 0.02).to(torch.bfloat16), quantize_fp8=True)
            for _, n in L.norms():
                n.weight = norm_weight(n.hidden_size)
        w.final_norm.weight = norm_weight(shape.hidden)
        w.embed = (torch.randn(shape.vocab, shape.hidden, generator=gen, device=device) * 0.02
                   ).to(torch.bfloat16)
        w.lm_head_weight = w.embed
        return w


class Qwen3FP8DecodeStep:
    """Qwen3-shaped fp8 decoder (random init, or a checkpoint via
    ``from_pretrained``) plus a synthetic decode batch over a shared-prefix KV pool."""

    def __init__(self, shape: Qwen3Shape, requests: int, beams: int, prefix: int, step: int = 1,
                 device: Optional[torch.device] = None, seed: int = 4,
                 weights: Optional[Qwen3FP8Weights] = None, trie_items: int = 0,
                 trie_levels: int = 3, trie_codes: int = 256):
        self.shape = shape
        self.device = device or torch.device("cuda")
        dev = self.device
        gen = torch.Generator(device=dev).manual_seed(seed)
        if weights is None:
            weights = Qwen3FP8Weights.random(shape, gen, dev)
        for name, lin in weights.named_linears():
            if not lin._use_fp8:
                raise ValueError(f"{name} holds no fp8 weight: load with quantize_fp8=True")
        if weights.lm_head_weight is None:
            raise ValueError("no lm_head weight (and embeddings are not tied)")
        self.weights = weights
        self.layers = weights.layers
        # prearranged weights (and the gate_up weights with gate/up rows
        # interleaved for the SiLU-and-mul epilogue), built once here rather
        # than inside a captured step
        for L in self.layers:
            for lin in (L.qkv_proj, L.o_proj, L.down_proj):
                lin.prepare()
            L.gate_up_proj._glu_operands()
        self.final_norm = weights.final_norm
        self.embed = weights.lm_head_weight
        self.rotary = RotaryEmbedding(shape.head_dim, shape.max_position, shape.rope_theta, device=dev)
        # the head reads the SID rows of the lm_head weight (logits.py:110-114),
        # here the top of the vocabulary
        sid_lo = shape.vocab - shape.sid_tokens
        self.sid_ids = list(range(sid_lo, sid_lo + shape.sid_tokens))
        self.lm_head = RestrictedLMHead(self.sid_ids, fp8=True)
        # the batch (KV pool contents, hidden states) comes from its own
        # stream of random numbers, so it is the same for any weights
        gen = torch.Generator(device=dev).manual_seed(seed + 1000)

        # ---- KV pool: each request's prompt KV once, then `step` decoded
        # slots per beam row (slot 0 is the pool's dummy)
        rows = requests * beams
        self.rows = rows
        slots = 1 + requests * prefix + rows * (step + 1)
        self.pool = TokenToKVPool(shape.layers, slots, shape.kv_heads, shape.head_dim,
                                  torch.float8_e4m3fn, dev)
        for layer in range(shape.layers):
            for cache in (self.pool.k[layer], self.pool.v[layer]):
                cache.copy_(torch.randn(cache.shape, generator=gen, device=dev).to(torch.float8_e4m3fn))
        prefix_slots = 1 + torch.arange(requests * prefix, device=dev, dtype=torch.int32).view(requests, prefix)
        own0 = 1 + requests * prefix
        own = own0 + torch.arange(rows * (step + 1), device=dev, dtype=torch.int32).view(rows, step + 1)
        req_of_row = torch.arange(rows, device=dev) // beams
        kv = torch.cat([prefix_slots[req_of_row], own], dim=1)  # [rows, prefix + step + 1]
        seq = prefix + step + 1
        self.seq_len = seq
        self.batch = _Batch(
            is_prefill=False,
            seq_lens=torch.full((rows,), seq, dtype=torch.int32, device=dev),
            seq_lens_cpu=torch.full((rows,), seq, dtype=torch.int32),
            kv_indices=kv.reshape(-1).contiguous(),
            kv_indptr=None,
            positions=torch.full((rows,), seq - 1, dtype=torch.int64, device=dev),
            out_cache_loc=own[:, -1].to(torch.int64).contiguous(),
            extend_seq_lens=None,
            extend_prefix_lens=None,
        )
        self.attn = AttentionBackend(self.pool, shape.q_heads, shape.kv_heads, shape.head_dim)
        self.attn.prepare(self.batch)
        self.hidden_in = (torch.randn(rows, shape.hidden, generator=gen, device=dev)).to(torch.bfloat16)
        self._graph: Optional[torch.cuda.CUDAGraph] = None
        self._out = None
        # probe(layer_id, stage, *tensors): called at each stage boundary of a
        # layer when set (tests compare every stage with the oracle); it must
        # copy what it keeps, later stages update some tensors in place
        self.probe = None
        self.trie = None
        if trie_items > 0:
            self._init_beam(requests, beams, trie_items, trie_levels, trie_codes, gen, step)

    # ------------------------------------------------------------ one layer
    def _attention(self, L: _Layer, q_fp8, a_scale, residual: Optional[torch.Tensor] = None) -> torch.Tensor:
        """qwen3.py:65-136, fused fp8 path.  With ``residual`` the o projection
        adds its output into the residual stream in its epilogue (the add of
        the next fused add + RMSNorm) and returns the updated stream."""
        s = self.shape
        t = int(q_fp8.shape[0])
        qkv = L.qkv_proj.forward_fp8(q_fp8, a_scale, (t, s.hidden), torch.bfloat16)
        self._tap(L, "qkv", qkv)
        heads = qkv.view(t, s.q_heads + 2 * s.kv_heads, s.head_dim)
        q = heads[:, : s.q_heads]
        k = heads[:, s.q_heads: s.q_heads + s.kv_heads]
        v = heads[:, s.q_heads + s.kv_heads:]
        stored = fused_qk_norm_rope_store_fp8(
            q, k, v, self.batch.positions, self.batch.out_cache_loc, L.q_norm.weight, L.k_norm.weight,
            L.q_norm.eps, self.rotary.cos_sin_cache, self.pool.k[L.layer_id], self.pool.v[L.layer_id])
        if not stored:
            raise RuntimeError("fused QK-norm/RoPE/KV write rejected its inputs")
        self._tap(L, "rope", q)
        # q stays a strided view of qkv: the attention kernel takes row and head strides
        if self.probe is None:
            # attention fused with the o projection's per-token e4m3 quant
            # (bit-for-bit the two steps below, which a probe needs apart)
            a8, a_scale = self.attn.forward_quant_fp8(q, L.layer_id)
            if residual is not None:
                return L.o_proj.forward_fp8_residual(a8, a_scale, residual)
            out = L.o_proj.forward_fp8(a8, a_scale, (t, s.q_heads * s.head_dim), torch.bfloat16)
        else:
            o = self.attn.forward(q, k, v, L.layer_id, self.batch, skip_store=True)
            self._tap(L, "attn", o)
            out = L.o_proj(o.reshape(t, -1))
        self._tap(L, "o", out)
        return out

    def _tap(self, L: _Layer, stage: str, *tensors) -> None:
        if self.probe is not None:
            self.probe(L.layer_id, stage, *tensors)

    def _layer(self, L: _Layer, x: torch.Tensor, residual: Optional[torch.Tensor]):
        """qwen3.py:197-210 (fused RMSNorm->fp8 path) and the MLP of :146-171."""
        if self.probe is None:
            return self._layer_folded(L, x, residual)
        if residual is None:
            residual = x
            q_fp8, a_scale = L.input_layernorm.quant_fp8(x)
        else:
            q_fp8, a_scale, residual = L.input_layernorm.quant_fp8(x, residual)
        self._tap(L, "ln_in", q_fp8, a_scale, residual)
        hidden = self._attention(L, q_fp8, a_scale)
        q_fp8, a_scale, residual = L.post_attention_layernorm.quant_fp8(hidden, residual)
        self._tap(L, "ln_post", q_fp8, a_scale, residual)
        t = int(q_fp8.shape[0])
        gu = L.gate_up_proj.forward_fp8(q_fp8, a_scale, (t, self.shape.hidden), torch.bfloat16)
        self._tap(L, "gate_up", gu)
        y_fp8, y_scale = silu_and_mul_per_token_quant_fp8(gu)
        self._tap(L, "silu", y_fp8, y_scale)
        hidden = L.down_proj.forward_fp8(y_fp8, y_scale, (t, self.shape.intermediate), torch.bfloat16)
        self._tap(L, "down", hidden)
        return hidden, residual

    def _layer_folded(self, L: _Layer, x: Optional[torch.Tensor], residual: Optional[torch.Tensor]):
        """The same layer with each residual add folded into the GEMM that
        produces the addend (o_proj, down_proj: fr_fp8_scaled_mm_residual),
        so both RMSNorms run without their add, and SiLU-and-mul folded into
        the gate_up GEMM (fr_fp8_scaled_mm_silu): bit-for-bit ``_layer``, whose
        fused add + RMSNorm rounds the GEMM output and then the sum the same
        way.  Takes and returns (None, residual) once the stream holds the
        sum; the first layer starts from (x, None) as ``_layer`` does."""
        if residual is None:
            residual = x
        q_fp8, a_scale = L.input_layernorm.quant_fp8(residual)
        residual = self._attention(L, q_fp8, a_scale, residual)
        q_fp8, a_scale = L.post_attention_layernorm.quant_fp8(residual)
        # SiLU-and-mul in the gate_up GEMM's epilogue (half-width bf16 rows),
        # then the per-token quant: bit-for-bit silu_and_mul_per_token_quant_fp8
        # of the full gate_up output
        h = L.gate_up_proj.forward_fp8_silu(q_fp8, a_scale)
        y_fp8, y_scale = per_token_quant_fp8(h)
        residual = L.down_proj.forward_fp8_residual(y_fp8, y_scale, residual)
        return None, residual

    def forward(self, x: Optional[torch.Tensor] = None, layers: Optional[int] = None) -> torch.Tensor:
        """Decoder layers, final norm, SID-restricted fp8 lm_head -> logprobs [rows, sid_tokens]."""
        logprobs, _ = self.lm_head.compute(self._hidden_out(x, layers), self.embed)
        return logprobs

    def _hidden_out(self, x: Optional[torch.Tensor] = None, layers: Optional[int] = None,
                    quant: bool = False):
        """Decoder layers and the final norm: the lm_head's input (with
        ``quant``, as per-token e4m3 codes and scales from the fused
        RMSNorm -> e4m3, the rows the fp8 head would quantise)."""
        x = self.hidden_in if x is None else x
        residual = None
        # the residual stream is updated in place by the fused add-norms: start
        # from a copy so replays see the same input
        x = x.clone()
        for L in self.layers[: layers if layers is not None else len(self.layers)]:
            x, residual = self._layer(L, x, residual)
        if x is None:  # folded layers: the stream already holds the last sum
            return self.final_norm.quant_fp8(residual) if quant else self.final_norm(residual)
        if quant:
            q, s, _ = self.final_norm.quant_fp8(x, residual)
            return q, s
        y, _ = self.final_norm(x, residual)
        return y

    # ---------------------------------------------------------- graph
    # ---------------------------------------------------------- beam tail
    def _init_beam(self, requests: int, beams: int, items: int, levels: int, codes: int,
                   gen: torch.Generator, step: int) -> None:
        """A random trie of ``items`` SIDs of ``levels`` codes each (level l's
        code c is token sid_lo + l*codes + c) as the dense allow / next tables
        of python/flashrec/search/trie.py:208-251 (next_node int32, leaves ->
        -1 = unconstrained, missing children -> the invalid row), and beam
        state one level deep: each beam has taken a random valid first code."""
        dev = self.device
        vsz = levels * codes
        if vsz > self.shape.sid_tokens:
            raise ValueError("trie codes exceed the SID head")
        sids = torch.randint(0, codes, (items, levels), generator=gen, device=dev)
        # node ids: root 0, then the distinct prefixes of each depth in order
        node_of = [torch.zeros(items, dtype=torch.int64, device=dev)]
        n_nodes = 1
        key = torch.zeros(items, dtype=torch.int64, device=dev)
        for d in range(1, levels):
            key = key * codes + sids[:, d - 1]
            uniq, inv = torch.unique(key, return_inverse=True)
            node_of.append(n_nodes + inv)
            n_nodes += int(uniq.numel())
        invalid = n_nodes
        allow = torch.zeros(n_nodes + 1, vsz, dtype=torch.bool, device=dev)
        nxt = torch.full((n_nodes + 1, vsz), invalid, dtype=torch.int32, device=dev)
        for d in range(levels):
            rel = d * codes + sids[:, d]
            allow[node_of[d], rel] = True
            child = node_of[d + 1].to(torch.int32) if d + 1 < levels else torch.full_like(rel, -1, dtype=torch.int32)
            nxt[node_of[d], rel] = child
        n, bw = requests, beams
        first = sids[torch.randint(0, items, (n, bw), generator=gen, device=dev), 0]
        self.trie = dict(allow=allow, next=nxt, invalid=invalid, base=self.sid_ids[0], levels=levels,
                         codes=codes, n_nodes=n_nodes)
        self.beam_n, self.beam_bw = n, bw
        self.beam_cand = min(2 * bw, self.shape.sid_tokens)  # beam_candidates (core.py:76-78)
        self.cand_ids = torch.tensor(self.sid_ids, dtype=torch.int64, device=dev)
        self.beam_cum = torch.sort(torch.randn(n, bw, generator=gen, device=dev) - 3.0, dim=-1,
                                   descending=True).values
        self.beam_nodes = nxt[0, first].to(torch.int64)
        width = max(levels, step + 1)
        self.beam_tokens = torch.zeros(n, bw, width, dtype=torch.int64, device=dev)
        self.beam_tokens[:, :, 0] = self.sid_ids[0] + first
        self.beam_col = torch.ones(n, dtype=torch.int32, device=dev)
        from flashrec_amd.kernel.beam_trie import GenrecFusedWorkspace

        self.beam_ws = GenrecFusedWorkspace()
        self._topk_vals = torch.empty(n, bw, self.beam_cand, dtype=torch.float32, device=dev)
        self._topk_tok = torch.empty(n, bw, self.beam_cand, dtype=torch.int64, device=dev)

    def beam_step(self, logprobs: torch.Tensor, from_logits: bool = False):
        """The step's tail (scheduler.py:1469-1561): per-row top-C of the SID
        log-probs with the candidate-id gather, then the fused trie mask +
        top-K + token-row expand + node advance for every request.  With
        ``from_logits`` the input is the head's logits and the log-softmax is
        folded into the top-C (the same log-probs, never written out)."""
        from flashrec_amd.kernel.beam_trie import genrec_mask_topk_expand, row_topk

        if self.trie is None:
            raise RuntimeError("built without a trie (trie_items=0)")
        n, bw, c = self.beam_n, self.beam_bw, self.beam_cand
        vals, _, toks = row_topk(logprobs.view(n, bw, -1), c, self.cand_ids,
                                 out=(self._topk_vals, None), out_tokens=self._topk_tok, need_idx=False,
                                 log_softmax=from_logits)
        tr = self.trie
        return genrec_mask_topk_expand(
            self.beam_cum, vals, toks, select_k=bw, node_ids=self.beam_nodes, allow_table=tr["allow"],
            token_base=tr["base"], token_ids=self.beam_tokens, col=self.beam_col, next_node=tr["next"],
            invalid_node=tr["invalid"], workspace=self.beam_ws)

    def forward_beam(self):
        """forward() then beam_step(): one whole decode step of beam search,
        with the final norm writing the fp8 head's e4m3 input directly and the
        head's log-softmax folded into the beam tail's top-C."""
        q, s = self._hidden_out(quant=True)
        logits, _ = self.lm_head.compute_logits_fp8(q, s, self.embed)
        return self.beam_step(logits, from_logits=True)

    @classmethod
    def from_pretrained(cls, model_path: str, requests: int, beams: int, prefix: int, step: int = 1,
                        device: Optional[torch.device] = None, seed: int = 4,
                        sid_tokens: Optional[int] = None) -> "Qwen3FP8DecodeStep":
        """Shape from config.json and weights from safetensors (bf16 weights
        quantised on load, fp8 ones kept with their scales)."""
        from flashrec_amd.weight import load_hf_config, load_weights

        shape = load_hf_config(model_path)
        if sid_tokens is not None:
            shape.sid_tokens = int(sid_tokens)
        shape.sid_tokens = min(shape.sid_tokens, shape.vocab)
        shape.max_position = max(shape.max_position, prefix + step + 1)
        dev = device or torch.device("cuda")
        w = Qwen3FP8Weights(shape)
        load_weights(w, model_path, dev, torch.bfloat16, quantize_fp8=True)
        return cls(shape, requests, beams, prefix, step, dev, seed, weights=w)

    def capture(self, beam: bool = False) -> None:
        """Record forward() (with ``beam``, forward_beam()) into one HIP graph
        after a warm-up run that lets the lm_head quantise its slice and the
        allocator and workspaces settle."""
        fn = self.forward_beam if beam else self.forward
        s = torch.cuda.Stream()
        s.wait_stream(torch.cuda.current_stream())
        with torch.cuda.stream(s):
            fn()
        torch.cuda.current_stream().wait_stream(s)
        torch.cuda.synchronize()
        g = torch.cuda.CUDAGraph()
        with torch.cuda.graph(g):
            self._out = fn()
        self._graph = g

    def replay(self):
        assert self._graph is not None and self._out is not None
        self._graph.replay()
        return self._out

