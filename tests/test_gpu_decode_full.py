"""Config 4 at its full size: the 28-layer Qwen3-1.7B-shaped fp8 decode step
over 4096 beam rows (8 requests x 512 beams, 128-token shared prefix), the
8192-token SID head and the beam tail over a 3-level x 256-code trie.

Checks: every output finite; log-softmax rows sum to 1; every stage of
layers 0 and 27 on all 4096 rows against the oracle, each stage fed the
GPU's own input to it (so each operator is held to its own bar inside the
composition); the head on sampled rows; the beam tail against the oracle on
the step's own log-probs, with every pick a valid trie child; and the
HIP-graph replay of the whole step equal to its eager run.
"""

import pytest
import torch

from helpers import assert_fp8_parity, assert_rope_parity, code_flip_stats, codes, max_abs_rel
from oracle import beam, ops

pytestmark = pytest.mark.gpu

CHECKED_LAYERS = (0, 27)


@pytest.fixture(scope="module")
def step(dev):
    from flashrec_amd.decode_step import Qwen3FP8DecodeStep, Qwen3Shape

    m = Qwen3FP8DecodeStep(Qwen3Shape(), requests=8, beams=512, prefix=128, step=2, device=dev, seed=4,
                           trie_items=200000, trie_levels=3, trie_codes=256)
    yield m
    del m
    torch.cuda.empty_cache()


def _gemm_rel(lin, q8, sa, got):
    ref = ops.fp8_scaled_mm(q8, lin._fp8_weight.cpu(), sa, lin._fp8_scale.cpu())
    return max_abs_rel(got, ref)


def _check_layer(m, L, taps, x_in, r_in):
    """Every stage of one decoder layer on all 4096 rows against the oracle,
    each fed the GPU's own input to that stage (qwen3.py:65-210 order)."""
    s = m.shape
    b = m.batch
    t = m.rows
    eps = s.eps
    tag = f"layer {L.layer_id}"
    # (add +) RMSNorm -> fp8
    w_in = L.input_layernorm.weight.cpu()
    q8, sa, res = taps["ln_in"]
    if r_in is None:
        q_ref, s_ref = ops.rmsnorm_per_token_quant_fp8(x_in, w_in, eps)
    else:
        q_ref, s_ref, res_ref = ops.fused_add_rmsnorm_per_token_quant_fp8(x_in, r_in, w_in, eps)
        assert torch.equal(res.view(torch.int16), res_ref.view(torch.int16)), f"{tag} input residual"
    assert_fp8_parity(q8, sa, q_ref, s_ref, label=f"{tag} input norm")
    # qkv GEMM
    qkv = taps["qkv"][0]
    e = _gemm_rel(L.qkv_proj, q8, sa, qkv)
    # QK-norm + RoPE + fp8 KV write, from the GPU's qkv
    heads = qkv.view(t, s.q_heads + 2 * s.kv_heads, s.head_dim)
    q, k, v = heads[:, :s.q_heads], heads[:, s.q_heads:s.q_heads + s.kv_heads], heads[:, s.q_heads + s.kv_heads:]
    kc_gpu = m.pool.k[L.layer_id].cpu()
    vc_gpu = m.pool.v[L.layer_id].cpu()
    kc_ref = kc_gpu.clone()
    vc_ref = vc_gpu.clone()
    loc = b.out_cache_loc.cpu()
    qn_w, kn_w = L.q_norm.weight.cpu(), L.k_norm.weight.cpu()
    q_rot_ref = ops.qk_norm_rope_store_fp8(q, k, v, b.positions.cpu(), loc, qn_w, kn_w, eps,
                                           m.rotary.cos_sin_cache.cpu(), kc_ref, vc_ref)
    q_rot = taps["rope"][0]
    assert_rope_parity(q_rot, q_rot_ref, ops.rmsnorm(q, qn_w, eps))
    assert torch.equal(codes(vc_gpu[loc]), codes(vc_ref[loc])), f"{tag} V pages"
    frac, dist = code_flip_stats(kc_gpu[loc], kc_ref[loc])
    assert frac < 1e-3 and dist <= 1, (tag, "K pages", frac, dist)
    # paged attention over the GPU's pool (shared prefix + own slots)
    seq = m.seq_len
    start = torch.arange(t, dtype=torch.int32) * seq
    ln = torch.full((t,), seq, dtype=torch.int32)
    att_ref = ops.paged_attention(q_rot, kc_gpu, vc_gpu, b.kv_indices.cpu(), start, ln, s.head_dim ** -0.5)
    att = taps["attn"][0]
    err = ((att.float() - att_ref.float()).abs().amax(-1) / att_ref.float().abs().amax(-1).clamp(min=1e-6))
    e_att = err.max().item()
    assert e_att < 1e-2, (tag, "attention", e_att)
    # o: per-token quant (bit-exact op) + GEMM
    qa, sa_o = ops.per_token_quant_fp8(att.reshape(t, -1))
    e_o = _gemm_rel(L.o_proj, qa, sa_o, taps["o"][0])
    # residual add + RMSNorm -> fp8
    q8p, sap, resp = taps["ln_post"]
    q_ref, s_ref, res_ref = ops.fused_add_rmsnorm_per_token_quant_fp8(
        taps["o"][0], res, L.post_attention_layernorm.weight.cpu(), eps)
    assert torch.equal(resp.view(torch.int16), res_ref.view(torch.int16)), f"{tag} residual"
    assert_fp8_parity(q8p, sap, q_ref, s_ref, label=f"{tag} post-attention norm")
    # MLP
    gu = taps["gate_up"][0]
    e_gu = _gemm_rel(L.gate_up_proj, q8p, sap, gu)
    y8, ys = taps["silu"]
    y_ref, ys_ref = ops.silu_and_mul_per_token_quant_fp8(gu)
    assert_fp8_parity(y8, ys, y_ref, ys_ref, label=f"{tag} silu")
    e_dn = _gemm_rel(L.down_proj, y8, ys, taps["down"][0])
    print(f"{tag}: qkv {e:.2e}, attention {e_att:.2e}, o {e_o:.2e}, gate_up {e_gu:.2e}, down {e_dn:.2e}")
    for name, val in (("qkv", e), ("o", e_o), ("gate_up", e_gu), ("down", e_dn)):
        assert val < 1e-2, (tag, name, val)


def test_full_step_every_stage(step):
    m = step
    assert m.rows == 4096 and len(m.layers) == 28 and m.seq_len == 131
    taps = {}

    def probe(layer_id, stage, *tensors):
        if layer_id in CHECKED_LAYERS:
            taps.setdefault(layer_id, {})[stage] = [tt.detach().cpu().clone() for tt in tensors]

    x = m.hidden_in.clone()
    residual = None
    inputs = {}
    m.probe = probe
    try:
        for L in m.layers:
            if L.layer_id in CHECKED_LAYERS:
                inputs[L.layer_id] = (x.cpu(), None if residual is None else residual.cpu())
            x, residual = m._layer(L, x, residual)
            if L.layer_id in CHECKED_LAYERS:
                torch.cuda.synchronize()
                _check_layer(m, L, taps[L.layer_id], *inputs[L.layer_id])
            assert torch.isfinite(x).all() and torch.isfinite(residual).all(), f"layer {L.layer_id}"
    finally:
        m.probe = None
    y, _ = m.final_norm(x, residual)
    lp, ids = m.lm_head.compute(y, m.embed)
    assert lp.shape == (4096, 8192) and torch.isfinite(lp).all()
    torch.testing.assert_close(lp.exp().sum(-1).cpu(), torch.ones(4096), atol=1e-4, rtol=0)
    assert ids.cpu().tolist() == m.sid_ids
    # the fp8 head on the GPU's final hidden rows
    w = m.embed.cpu()[m.sid_ids[0]: m.sid_ids[0] + 8192]
    rows = torch.randperm(4096, generator=torch.Generator().manual_seed(12))[:256]
    ref = ops.restricted_logprobs_fp8(y.cpu()[rows], w)
    assert (lp.cpu()[rows] - ref).abs().max().item() < 2e-3
    # forward() composes exactly these calls
    assert torch.equal(m.forward(), lp)


def test_full_beam_tail_and_graph_replay(step):
    m = step
    lp = m.forward()
    got = m.beam_step(lp)
    n, bw, c = m.beam_n, m.beam_bw, m.beam_cand
    assert (n, bw, c) == (8, 512, 1024)
    tr = m.trie
    rv, _, rt = beam.row_topk(lp.cpu().view(n, bw, -1), c, m.cand_ids.cpu())
    ref = beam.genrec_mask_topk_expand(m.beam_cum.cpu(), rv, rt, bw, m.beam_nodes.cpu(), tr["allow"].cpu(),
                                       tr["base"], m.beam_tokens.cpu(), m.beam_col.cpu(),
                                       tr["next"].cpu().long(), tr["invalid"])
    for name, a, b in zip(("vals", "parents", "tokens", "indices", "token_ids", "node_ids"),
                          (got.vals, got.parents, got.tokens, got.indices, got.token_ids, got.node_ids), ref):
        assert torch.equal(a.cpu(), b), name
    # every pick is a child of its parent beam's trie node (level-1 codes)
    vals = got.vals.cpu()
    ok = vals > float("-inf")
    assert ok.float().mean().item() > 0.5
    parents = got.parents.cpu().long()
    node_of_parent = torch.gather(m.beam_nodes.cpu(), 1, parents)
    rel = got.tokens.cpu().long() - tr["base"]
    allow = tr["allow"].cpu()
    assert allow[node_of_parent[ok], rel[ok]].all()
    # one HIP graph for the whole step (layers, head, beam tail): every replay
    # equals the eager run
    eager = [t.clone() for t in (got.vals, got.tokens, got.token_ids, got.node_ids)]
    m.capture(beam=True)
    for i in range(2):
        torch.cuda.synchronize()
        out = m.replay()
        torch.cuda.synchronize()
        for a, b in zip((out.vals, out.tokens, out.token_ids, out.node_ids), eager):
            assert torch.equal(a, b), f"replay {i}"
