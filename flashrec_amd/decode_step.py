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
from flashrec_amd.kernel.silu_fp8 import silu_and_mul_per_token_quant_fp8
from flashrec_amd.kvcache.pool import TokenToKVPool
from flashrec_amd.layers.linear import Linear
from flashrec_amd.layers.norm import RMSNorm
from flashrec_amd.layers.rotary import RotaryEmbedding
from flashrec_amd.logits import RestrictedLMHead


@dataclass
class Qwen3Shape:
    """Qwen3-1.7B shape."""

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
                 weights: Optional[Qwen3FP8Weights] = None):
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
        self._out: Optional[torch.Tensor] = None

    # ------------------------------------------------------------ one layer
    def _attention(self, L: _Layer, q_fp8, a_scale) -> torch.Tensor:
        """qwen3.py:65-136, fused fp8 path."""
        s = self.shape
        t = int(q_fp8.shape[0])
        qkv = L.qkv_proj.forward_fp8(q_fp8, a_scale, (t, s.hidden), torch.bfloat16)
        heads = qkv.view(t, s.q_heads + 2 * s.kv_heads, s.head_dim)
        q = heads[:, : s.q_heads]
        k = heads[:, s.q_heads: s.q_heads + s.kv_heads]
        v = heads[:, s.q_heads + s.kv_heads:]
        stored = fused_qk_norm_rope_store_fp8(
            q, k, v, self.batch.positions, self.batch.out_cache_loc, L.q_norm.weight, L.k_norm.weight,
            L.q_norm.eps, self.rotary.cos_sin_cache, self.pool.k[L.layer_id], self.pool.v[L.layer_id])
        if not stored:
            raise RuntimeError("fused QK-norm/RoPE/KV write rejected its inputs")
        o = self.attn.forward(q.contiguous(), k, v, L.layer_id, self.batch, skip_store=True)
        return L.o_proj(o.reshape(t, -1))

    def _layer(self, L: _Layer, x: torch.Tensor, residual: Optional[torch.Tensor]):
        """qwen3.py:197-210 (fused RMSNorm->fp8 path) and the MLP of :146-171."""
        if residual is None:
            residual = x
            q_fp8, a_scale = L.input_layernorm.quant_fp8(x)
        else:
            q_fp8, a_scale, residual = L.input_layernorm.quant_fp8(x, residual)
        hidden = self._attention(L, q_fp8, a_scale)
        q_fp8, a_scale, residual = L.post_attention_layernorm.quant_fp8(hidden, residual)
        t = int(q_fp8.shape[0])
        gu = L.gate_up_proj.forward_fp8(q_fp8, a_scale, (t, self.shape.hidden), torch.bfloat16)
        y_fp8, y_scale = silu_and_mul_per_token_quant_fp8(gu)
        hidden = L.down_proj.forward_fp8(y_fp8, y_scale, (t, self.shape.intermediate), torch.bfloat16)
        return hidden, residual

    def forward(self, x: Optional[torch.Tensor] = None, layers: Optional[int] = None) -> torch.Tensor:
        """Decoder layers, final norm, SID-restricted fp8 lm_head -> logprobs [rows, sid_tokens]."""
        x = self.hidden_in if x is None else x
        residual = None
        # the residual stream is updated in place by the fused add-norms: start
        # from a copy so replays see the same input
        x = x.clone()
        for L in self.layers[: layers if layers is not None else len(self.layers)]:
            x, residual = self._layer(L, x, residual)
        y, _ = self.final_norm(x, residual)
        logprobs, _ = self.lm_head.compute(y, self.embed)
        return logprobs

    # ---------------------------------------------------------- graph
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

    def capture(self) -> None:
        """Record forward() into one HIP graph (after a warm-up run that lets
        the lm_head quantise its slice and the allocator settle)."""
        s = torch.cuda.Stream()
        s.wait_stream(torch.cuda.current_stream())
        with torch.cuda.stream(s):
            self.forward()
        torch.cuda.current_stream().wait_stream(s)
        torch.cuda.synchronize()
        g = torch.cuda.CUDAGraph()
        with torch.cuda.graph(g):
            self._out = self.forward()
        self._graph = g

    def replay(self) -> torch.Tensor:
        assert self._graph is not None and self._out is not None
        self._graph.replay()
        return self._out

