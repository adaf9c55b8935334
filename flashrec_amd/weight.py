"""Checkpoint loading into the FP8 path, mirroring ``flashrec.models.weight``.

Reference: python/flashrec/models/weight.py:19-68 (``merge_gate_up_weights``,
``merge_qkv_weights``), :71-88 (``load_hf_config``), :91-113 (safetensors
iteration, scale keys), :116-263 (``load_weights``).  Same key mapping, merge
order, scale expansion and dtype rules:

* ``*.weight_scale`` / ``*.weight_scale_inv`` tensors are read in a first pass
  that deserialises nothing else, and are used as given (the reference does
  not invert ``weight_scale_inv``; neither does this loader).
* q/k/v and gate/up are concatenated on the output dimension without
  requantising; a per-tensor scale is expanded per original matrix before
  the concatenation, so the fused layer keeps one scale per source matrix
  (``as_channel_scale``); block-wise scales raise ``ValueError``.
* fp8 weights are kept as stored; bf16/fp16/fp32 weights are cast to the
  compute dtype and, with ``quantize_fp8``, quantised per output channel by
  the HIP quantiser.

Layout choice for a 288 GB device: a fused matrix is allocated once on the
device and each source matrix is copied straight from the host tensor into
its row range, so neither a host-side concatenation nor a second device copy
of the parts is ever made.
"""

from __future__ import annotations

import json
import logging
from pathlib import Path
from typing import Dict, Iterator, List, Optional, Sequence, Tuple

import torch
from safetensors import safe_open

from flashrec_amd.layers.linear import Linear, as_channel_scale

logger = logging.getLogger(__name__)

_FP8 = (torch.float8_e4m3fn,)


def _merge_rows(parts: Sequence[torch.Tensor], device: Optional[torch.device]) -> torch.Tensor:
    """Concatenate ``[N_i, K]`` matrices on dim 0 into one tensor allocated on
    ``device`` (default: the first part's), copying each part into its rows."""
    dev = torch.device(device) if device is not None else parts[0].device
    n = sum(int(p.shape[0]) for p in parts)
    out = torch.empty((n,) + tuple(parts[0].shape[1:]), dtype=parts[0].dtype, device=dev)
    r = 0
    for p in parts:
        rows = int(p.shape[0])
        out[r: r + rows].copy_(p)
        r += rows
    return out


def merge_gate_up_weights(
    gate_w: torch.Tensor,
    up_w: torch.Tensor,
    gate_scale: Optional[torch.Tensor] = None,
    up_scale: Optional[torch.Tensor] = None,
    device: Optional[torch.device] = None,
) -> Tuple[torch.Tensor, Optional[torch.Tensor]]:
    """``[gate; up]`` on the output dim, not requantised (weight.py:19-41).

    ``device`` (an addition) names where the merged matrix is allocated; by
    default the parts' device, as in the reference."""
    if tuple(gate_w.shape) != tuple(up_w.shape):
        raise ValueError(f"gate/up shape mismatch: {tuple(gate_w.shape)} vs {tuple(up_w.shape)}")
    weight = _merge_rows([gate_w, up_w], device)
    scale = None
    if gate_scale is not None and up_scale is not None:
        n = int(gate_w.shape[0])
        scale = torch.cat([as_channel_scale(gate_scale, n, weight.device),
                           as_channel_scale(up_scale, n, weight.device)], dim=0)
    return weight, scale


def merge_qkv_weights(
    q_w: torch.Tensor,
    k_w: torch.Tensor,
    v_w: torch.Tensor,
    q_scale: Optional[torch.Tensor] = None,
    k_scale: Optional[torch.Tensor] = None,
    v_scale: Optional[torch.Tensor] = None,
    device: Optional[torch.device] = None,
) -> Tuple[torch.Tensor, Optional[torch.Tensor]]:
    """``[q; k; v]`` on the output dim, not requantised (weight.py:44-68)."""
    if q_w.shape[1] != k_w.shape[1] or q_w.shape[1] != v_w.shape[1]:
        raise ValueError(
            f"qkv in-dim mismatch: {tuple(q_w.shape)} / {tuple(k_w.shape)} / {tuple(v_w.shape)}")
    weight = _merge_rows([q_w, k_w, v_w], device)
    scale = None
    if q_scale is not None and k_scale is not None and v_scale is not None:
        scale = torch.cat([as_channel_scale(s, int(w.shape[0]), weight.device)
                           for w, s in ((q_w, q_scale), (k_w, k_scale), (v_w, v_scale))], dim=0)
    return weight, scale


def load_hf_config(model_path: str):
    """config.json -> model shape (weight.py:71-88; same keys and defaults)."""
    from flashrec_amd.decode_step import Qwen3Shape

    cfg = json.loads((Path(model_path) / "config.json").read_text(encoding="utf-8"))
    return Qwen3Shape(
        hidden=int(cfg["hidden_size"]),
        intermediate=int(cfg["intermediate_size"]),
        layers=int(cfg["num_hidden_layers"]),
        q_heads=int(cfg["num_attention_heads"]),
        kv_heads=int(cfg["num_key_value_heads"]),
        head_dim=int(cfg.get("head_dim") or cfg["hidden_size"] // cfg["num_attention_heads"]),
        vocab=int(cfg["vocab_size"]),
        eps=float(cfg.get("rms_norm_eps", 1e-6)),
        rope_theta=float(cfg.get("rope_theta", 1000000)),
        max_position=int(cfg.get("max_position_embeddings", 40960)),
        tie_word_embeddings=bool(cfg.get("tie_word_embeddings", True)),
    )


def _checkpoint_files(model_path: str) -> List[Path]:
    root = Path(model_path)
    index = root / "model.safetensors.index.json"
    if index.is_file():
        weight_map = json.loads(index.read_text())["weight_map"]
        return [root / name for name in sorted(set(weight_map.values()))]
    single = root / "model.safetensors"
    return [single] if single.is_file() else []


def _iter_safetensors(model_path: str, key_filter=None) -> Iterator[Tuple[str, torch.Tensor]]:
    """(key, host tensor); ``key_filter`` runs before a tensor is read (weight.py:91-110)."""
    for path in _checkpoint_files(model_path):
        with safe_open(str(path), framework="pt", device="cpu") as f:
            for key in f.keys():
                if key_filter is not None and not key_filter(key):
                    continue
                yield key, f.get_tensor(key)


def _is_scale_key(key: str) -> bool:
    return key.endswith(".weight_scale") or key.endswith(".weight_scale_inv")


def _layer_module(key: str) -> Optional[str]:
    """'model.layers.3.self_attn.q_proj.weight' -> 'layers.3.self_attn.q_proj'."""
    if not key.startswith("model.layers."):
        return None
    layer_id, _, tail = key[len("model.layers."):].partition(".")
    return f"layers.{layer_id}." + tail.rsplit(".", 1)[0]


def _load_linear(lin: Linear, w: torch.Tensor, scale: Optional[torch.Tensor], device,
                 compute_dtype: torch.dtype, quantize_fp8: bool) -> None:
    """weight.py:186-194 (and :230-237, :253-260): dtype rule, then Linear.load."""
    if w.dtype not in _FP8 and w.dtype != compute_dtype:
        w = w.to(dtype=compute_dtype)
    w = w.to(device=device)
    lin.load(w, quantize_fp8=quantize_fp8 and w.dtype not in _FP8, weight_scale=scale)


def load_weights(model, model_path: str, device: torch.device, compute_dtype: torch.dtype,
                 quantize_fp8: bool = False) -> None:
    """Load a HF safetensors checkpoint into ``model`` (weight.py:116-263).

    ``model`` exposes ``named_linears()`` and ``named_norms()`` (reference
    module names such as ``layers.0.self_attn.qkv_proj`` and ``norm``), and
    the attributes ``embed``, ``lm_head_weight`` and ``tie_word_embeddings``.
    """
    device = torch.device(device)
    linears: Dict[str, Linear] = dict(model.named_linears())
    norms = dict(model.named_norms())

    scale_map: Dict[str, torch.Tensor] = {}
    for key, tensor in _iter_safetensors(model_path, key_filter=_is_scale_key):
        mod = _layer_module(key)
        if mod is not None:
            scale_map[mod] = tensor.to(device=device)

    pending_gate_up: Dict[str, Dict[str, torch.Tensor]] = {}
    pending_qkv: Dict[str, Dict[str, torch.Tensor]] = {}
    for key, t in _iter_safetensors(model_path):
        if _is_scale_key(key):
            continue
        if key == "model.embed_tokens.weight":
            model.embed = t.to(device=device, dtype=compute_dtype)
            continue
        if key == "lm_head.weight":
            model.lm_head_weight = t.to(device=device, dtype=compute_dtype)
            continue
        if key == "model.norm.weight":
            norms["norm"].weight = torch.nn.Parameter(t.to(device=device, dtype=compute_dtype),
                                                      requires_grad=False)
            continue
        if not key.startswith("model.layers.") or not key.endswith(".weight"):
            continue
        mod = _layer_module(key)
        parent, _, which = mod.rpartition(".")
        if mod.endswith(".mlp.gate_proj") or mod.endswith(".mlp.up_proj"):
            # host tensors wait for their partner, then go to the device once,
            # straight into the fused matrix
            pending_gate_up.setdefault(parent + ".", {})[which] = t
            continue
        if mod.endswith((".self_attn.q_proj", ".self_attn.k_proj", ".self_attn.v_proj")):
            pending_qkv.setdefault(parent + ".", {})[which] = t
            continue
        if mod in linears:
            _load_linear(linears[mod], t, scale_map.get(mod), device, compute_dtype, quantize_fp8)
            continue
        if mod in norms:
            norms[mod].weight = torch.nn.Parameter(t.to(device=device, dtype=compute_dtype),
                                                   requires_grad=False)

    for prefix, parts in pending_qkv.items():
        dest = prefix + "qkv_proj"
        if dest not in linears:
            logger.warning("no qkv_proj module for %s", prefix)
            continue
        if any(p not in parts for p in ("q_proj", "k_proj", "v_proj")):
            logger.warning("incomplete q/k/v weights for %s", prefix)
            continue
        w, scale = merge_qkv_weights(parts["q_proj"], parts["k_proj"], parts["v_proj"],
                                     scale_map.get(prefix + "q_proj"), scale_map.get(prefix + "k_proj"),
                                     scale_map.get(prefix + "v_proj"), device=device)
        _load_linear(linears[dest], w, scale, device, compute_dtype, quantize_fp8)

    for prefix, parts in pending_gate_up.items():
        dest = prefix + "gate_up_proj"
        if dest not in linears:
            logger.warning("no gate_up_proj module for %s", prefix)
            continue
        if "gate_proj" not in parts or "up_proj" not in parts:
            logger.warning("incomplete gate/up weights for %s", prefix)
            continue
        w, scale = merge_gate_up_weights(parts["gate_proj"], parts["up_proj"],
                                         scale_map.get(prefix + "gate_proj"),
                                         scale_map.get(prefix + "up_proj"), device=device)
        _load_linear(linears[dest], w, scale, device, compute_dtype, quantize_fp8)

    if model.lm_head_weight is None and model.tie_word_embeddings:
        model.lm_head_weight = model.embed
