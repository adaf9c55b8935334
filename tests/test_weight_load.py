"""Checkpoint loading (flashrec_amd/weight.py) on the CPU.

The merge tests restate the known answers of the reference's own tests
(tests/test_mlp.py:28-71: merged layout, per-tensor scale expansion per source
matrix, block-wise rejection).  The loader tests write small safetensors
checkpoints (single file and sharded with an index) and check every fused
matrix and scale against the parts that were written; fp8 checkpoints load
with no kernel call, so these run without a GPU.
"""

import json
import logging

import pytest
import torch
from safetensors.torch import save_file

from flashrec_amd.decode_step import Qwen3FP8Weights, Qwen3Shape
from flashrec_amd.layers.linear import Linear, as_channel_scale
from flashrec_amd.weight import load_hf_config, load_weights, merge_gate_up_weights, merge_qkv_weights

F8 = torch.float8_e4m3fn


def test_merge_shapes():
    gate, up = torch.randn(6, 4), torch.randn(6, 4)
    gs, us = torch.ones(6), torch.full((6,), 2.0)
    w, scale = merge_gate_up_weights(gate, up, gs, us)
    assert tuple(w.shape) == (12, 4)
    assert torch.equal(w[:6], gate) and torch.equal(w[6:], up)
    assert torch.equal(scale[:6], gs) and torch.equal(scale[6:], us)


def test_merge_expands_per_tensor_scales():
    q, k, v = torch.randn(2048, 2048), torch.randn(1024, 2048), torch.randn(1024, 2048)
    w, scale = merge_qkv_weights(q, k, v, torch.tensor(2.0), torch.tensor(3.0), torch.tensor(4.0))
    assert tuple(w.shape) == (4096, 2048)
    assert torch.equal(w[2048:3072], k)
    assert tuple(scale.shape) == (4096,)
    assert torch.equal(scale[:2048], torch.full((2048,), 2.0))
    assert torch.equal(scale[2048:3072], torch.full((1024,), 3.0))
    assert torch.equal(scale[3072:], torch.full((1024,), 4.0))
    lin = Linear(2048, 4096)
    lin.load(torch.empty(4096, 2048, dtype=F8), weight_scale=scale)
    assert tuple(lin._fp8_scale.shape) == (4096,)
    _, gscale = merge_gate_up_weights(torch.randn(6, 4), torch.randn(6, 4), torch.tensor(0.5), torch.tensor(1.5))
    assert gscale.tolist() == [0.5] * 6 + [1.5] * 6


def test_merge_rejects_mismatch_and_blockwise():
    with pytest.raises(ValueError, match="block-wise"):
        as_channel_scale(torch.ones(3), 4096)
    with pytest.raises(ValueError, match="gate/up shape mismatch"):
        merge_gate_up_weights(torch.randn(6, 4), torch.randn(5, 4))
    with pytest.raises(ValueError, match="in-dim mismatch"):
        merge_qkv_weights(torch.randn(4, 8), torch.randn(2, 8), torch.randn(2, 6))
    # one missing scale: no merged scale (weight.py:31,59)
    _, s = merge_gate_up_weights(torch.randn(2, 2), torch.randn(2, 2), torch.tensor(1.0), None)
    assert s is None


def test_merge_keeps_fp8_codes():
    g = torch.Generator().manual_seed(1)
    parts = [torch.randn(n, 32, generator=g).to(F8) for n in (8, 4, 4)]
    w, _ = merge_qkv_weights(*parts)
    assert w.dtype == F8
    assert torch.equal(w.view(torch.uint8), torch.cat(parts).view(torch.uint8))


SHAPE = dict(hidden_size=64, intermediate_size=96, num_hidden_layers=2, num_attention_heads=4,
             num_key_value_heads=2, head_dim=16, vocab_size=300, rms_norm_eps=1e-5,
             rope_theta=10000.0, max_position_embeddings=128)


def _checkpoint(tmp_path, tie=True, shards=1, per_tensor=True, drop=None, scale_inv_key=False):
    """An fp8 checkpoint with split q/k/v and gate/up, as HF/ModelOpt write it."""
    cfg = dict(SHAPE, tie_word_embeddings=tie)
    (tmp_path / "config.json").write_text(json.dumps(cfg))
    g = torch.Generator().manual_seed(3)
    h, d, nq, nk, inter = 64, 16, 4, 2, 96
    t = {}
    for i in range(2):
        p = f"model.layers.{i}."
        dims = {"self_attn.q_proj": (nq * d, h), "self_attn.k_proj": (nk * d, h),
                "self_attn.v_proj": (nk * d, h), "self_attn.o_proj": (h, nq * d),
                "mlp.gate_proj": (inter, h), "mlp.up_proj": (inter, h), "mlp.down_proj": (h, inter)}
        for j, (name, (n, k)) in enumerate(dims.items()):
            t[p + name + ".weight"] = torch.randn(n, k, generator=g).to(F8)
            sk = ".weight_scale_inv" if (scale_inv_key and j == 0) else ".weight_scale"
            t[p + name + sk] = (torch.tensor(0.5 + j + i) if per_tensor
                                else torch.rand(n, generator=g) + 0.1)
        for name, n in (("input_layernorm", h), ("post_attention_layernorm", h),
                        ("self_attn.q_norm", d), ("self_attn.k_norm", d)):
            t[p + name + ".weight"] = torch.randn(n, generator=g).to(torch.bfloat16)
    t["model.embed_tokens.weight"] = torch.randn(300, h, generator=g).to(torch.bfloat16)
    t["model.norm.weight"] = torch.randn(h, generator=g).to(torch.bfloat16)
    if not tie:
        t["lm_head.weight"] = torch.randn(300, h, generator=g).to(torch.bfloat16)
    if drop:
        del t[drop]
    keys = sorted(t)
    if shards == 1:
        save_file(t, str(tmp_path / "model.safetensors"))
    else:
        wmap = {}
        for s in range(shards):
            name = f"model-{s + 1:05d}-of-{shards:05d}.safetensors"
            part = {k: t[k] for k in keys[s::shards]}
            save_file(part, str(tmp_path / name))
            wmap.update({k: name for k in part})
        (tmp_path / "model.safetensors.index.json").write_text(json.dumps({"weight_map": wmap}))
    return t


def _load(tmp_path):
    shape = load_hf_config(str(tmp_path))
    w = Qwen3FP8Weights(shape)
    load_weights(w, str(tmp_path), torch.device("cpu"), torch.bfloat16, quantize_fp8=True)
    return shape, w


def _expect(t, i, names, n_rows):
    p = f"model.layers.{i}."
    w = torch.cat([t[p + n + ".weight"] for n in names]).view(torch.uint8)
    s = []
    for n, rows in zip(names, n_rows):
        sc = t.get(p + n + ".weight_scale", t.get(p + n + ".weight_scale_inv"))
        s.append(sc.float().reshape(-1).expand(rows) if sc.numel() == 1 else sc.float())
    return w, torch.cat(s)


@pytest.mark.parametrize("shards,per_tensor,scale_inv", [(1, True, False), (3, False, True)])
def test_loader_fuses_and_expands(tmp_path, shards, per_tensor, scale_inv):
    t = _checkpoint(tmp_path, shards=shards, per_tensor=per_tensor, scale_inv_key=scale_inv)
    shape, w = _load(tmp_path)
    assert (shape.hidden, shape.intermediate, shape.layers, shape.q_heads, shape.kv_heads,
            shape.head_dim, shape.vocab) == (64, 96, 2, 4, 2, 16, 300)
    assert shape.eps == 1e-5 and shape.rope_theta == 10000.0 and shape.max_position == 128
    for L in w.layers:
        i = L.layer_id
        cases = ((L.qkv_proj, ("self_attn.q_proj", "self_attn.k_proj", "self_attn.v_proj"), (64, 32, 32)),
                 (L.gate_up_proj, ("mlp.gate_proj", "mlp.up_proj"), (96, 96)),
                 (L.o_proj, ("self_attn.o_proj",), (64,)),
                 (L.down_proj, ("mlp.down_proj",), (64,)))
        for lin, names, rows in cases:
            ew, es = _expect(t, i, names, rows)
            assert lin._use_fp8
            # [K, N] column-major view of the stored [N, K] codes
            assert lin._fp8_weight.shape == (lin.in_features, lin.out_features)
            assert lin._fp8_weight.stride() == (1, lin.in_features)
            assert torch.equal(lin._fp8_weight.t().contiguous().view(torch.uint8), ew)
            assert torch.equal(lin._fp8_scale, es)
        assert torch.equal(L.q_norm.weight, t[f"model.layers.{i}.self_attn.q_norm.weight"])
        assert torch.equal(L.post_attention_layernorm.weight,
                           t[f"model.layers.{i}.post_attention_layernorm.weight"])
    assert torch.equal(w.final_norm.weight, t["model.norm.weight"])
    assert torch.equal(w.embed, t["model.embed_tokens.weight"])
    assert w.lm_head_weight is w.embed


def test_loader_untied_head_and_missing_part(tmp_path, caplog):
    t = _checkpoint(tmp_path, tie=False, drop="model.layers.1.self_attn.v_proj.weight")
    with caplog.at_level(logging.WARNING, logger="flashrec_amd.weight"):
        _, w = _load(tmp_path)
    assert torch.equal(w.lm_head_weight, t["lm_head.weight"])
    assert not w.layers[1].qkv_proj._use_fp8          # left unloaded
    assert w.layers[0].qkv_proj._use_fp8
    assert any("incomplete q/k/v" in r.message for r in caplog.records)


def test_config_defaults(tmp_path):
    cfg = {k: v for k, v in SHAPE.items() if k not in ("head_dim", "rms_norm_eps", "rope_theta",
                                                       "max_position_embeddings")}
    (tmp_path / "config.json").write_text(json.dumps(cfg))
    s = load_hf_config(str(tmp_path))
    assert isinstance(s, Qwen3Shape)
    assert s.head_dim == 16 and s.eps == 1e-6 and s.rope_theta == 1000000.0
    assert s.max_position == 40960 and s.tie_word_embeddings is True
