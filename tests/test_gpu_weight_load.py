"""Checkpoint -> device weights -> decode step, on the GPU.

Round trip: a random-init step's fp8 weights are written as a split
(q/k/v, gate/up) ModelOpt-style checkpoint with per-channel scales, loaded
back through ``Qwen3FP8DecodeStep.from_pretrained``, and the two steps must
give bit-identical log-probs on the same batch.  A bf16 checkpoint loaded with
quantisation must give, for every fused matrix, the oracle quantiser's codes
and scales of the concatenated bf16 parts (per-channel quantisation commutes
with the row concatenation)."""

import json

import pytest
import torch
from safetensors.torch import save_file

from oracle import ops

pytestmark = pytest.mark.gpu

CFG = dict(hidden_size=512, intermediate_size=1024, num_hidden_layers=2, num_attention_heads=4,
           num_key_value_heads=2, head_dim=128, vocab_size=2048, rms_norm_eps=1e-6,
           rope_theta=1000000.0, max_position_embeddings=512, tie_word_embeddings=True)


def _shape():
    from flashrec_amd.decode_step import Qwen3Shape

    return Qwen3Shape(hidden=512, intermediate=1024, layers=2, q_heads=4, kv_heads=2,
                      max_position=512, sid_tokens=512, vocab=2048)


def _split(lin, rows):
    w = lin._fp8_weight.t().contiguous().cpu()
    s = lin._fp8_scale.cpu()
    out, r = [], 0
    for n in rows:
        out.append((w[r: r + n].contiguous(), s[r: r + n].contiguous()))
        r += n
    return out


def test_fp8_checkpoint_round_trip(dev, tmp_path):
    from flashrec_amd.decode_step import Qwen3FP8DecodeStep

    a = Qwen3FP8DecodeStep(_shape(), requests=2, beams=16, prefix=40, step=1, device=dev, seed=11)
    t = {}
    for L in a.layers:
        p = f"model.layers.{L.layer_id}."
        for name, (w, s) in zip(("self_attn.q_proj", "self_attn.k_proj", "self_attn.v_proj"),
                                _split(L.qkv_proj, (512, 256, 256))):
            t[p + name + ".weight"], t[p + name + ".weight_scale"] = w, s
        for name, (w, s) in zip(("mlp.gate_proj", "mlp.up_proj"), _split(L.gate_up_proj, (1024, 1024))):
            t[p + name + ".weight"], t[p + name + ".weight_scale"] = w, s
        for name, lin in (("self_attn.o_proj", L.o_proj), ("mlp.down_proj", L.down_proj)):
            (w, s), = _split(lin, (lin.out_features,))
            t[p + name + ".weight"], t[p + name + ".weight_scale"] = w, s
        for name, n in L.norms():
            t[p + name + ".weight"] = n.weight.detach().cpu()
    t["model.norm.weight"] = a.final_norm.weight.detach().cpu()
    t["model.embed_tokens.weight"] = a.embed.cpu()
    save_file(t, str(tmp_path / "model.safetensors"))
    (tmp_path / "config.json").write_text(json.dumps(CFG))

    b = Qwen3FP8DecodeStep.from_pretrained(str(tmp_path), requests=2, beams=16, prefix=40, step=1,
                                           device=dev, seed=11, sid_tokens=512)
    assert torch.equal(a.hidden_in, b.hidden_in)
    ya, yb = a.forward(), b.forward()
    torch.cuda.synchronize()
    assert torch.equal(ya, yb)


def test_bf16_checkpoint_quantised_on_load(dev, tmp_path):
    from flashrec_amd.decode_step import Qwen3FP8Weights
    from flashrec_amd.weight import load_hf_config, load_weights

    (tmp_path / "config.json").write_text(json.dumps(CFG))
    g = torch.Generator().manual_seed(5)
    t = {}
    dims = {"self_attn.q_proj": (512, 512), "self_attn.k_proj": (256, 512), "self_attn.v_proj": (256, 512),
            "self_attn.o_proj": (512, 512), "mlp.gate_proj": (1024, 512), "mlp.up_proj": (1024, 512),
            "mlp.down_proj": (512, 1024)}
    for i in range(2):
        for name, (n, k) in dims.items():
            w = torch.randn(n, k, generator=g) * 0.02
            w[0, :] *= 50  # one loud channel per matrix: the scales differ per row
            t[f"model.layers.{i}.{name}.weight"] = w.to(torch.bfloat16)
    t["model.embed_tokens.weight"] = torch.randn(2048, 512, generator=g).to(torch.bfloat16)
    save_file(t, str(tmp_path / "model.safetensors"))
    w = Qwen3FP8Weights(load_hf_config(str(tmp_path)))
    load_weights(w, str(tmp_path), dev, torch.bfloat16, quantize_fp8=True)
    torch.cuda.synchronize()
    for L in w.layers:
        p = f"model.layers.{L.layer_id}."
        for lin, names in ((L.qkv_proj, ("self_attn.q_proj", "self_attn.k_proj", "self_attn.v_proj")),
                           (L.gate_up_proj, ("mlp.gate_proj", "mlp.up_proj")),
                           (L.o_proj, ("self_attn.o_proj",)), (L.down_proj, ("mlp.down_proj",))):
            q, s = ops.quantize_weight_fp8(torch.cat([t[p + n + ".weight"] for n in names]))
            assert torch.equal(lin._fp8_weight.t().contiguous().cpu().view(torch.uint8), q.view(torch.uint8))
            assert torch.equal(lin._fp8_scale.cpu(), s)
    assert w.lm_head_weight is w.embed and w.embed.device.type == "cuda"
