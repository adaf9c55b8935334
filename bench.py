"""Benchmark of the MI355X FP8 path (one JSON line on stdout).

Headline (``value``): the W8A8 gate_up GEMM of config 1 at M=4096 beam rows
(K=2048, N=12288, bf16 out) in TFLOP/s, one launch per step, with operands
already resident in HBM and rotated over enough copies (> 512 MB) that no
step is served from the 256 MB MALL.  ``extra`` carries the other kernels of
the path at their configuration sizes (GB/s for the bandwidth-bound ones,
TFLOP/s for GEMMs), each with its roofline fraction.  ``cpu_baseline`` times
the reference's CPU torch path for the same GEMM on a bounded row sample.

    python bench.py [--steps K] [--warmup W] [--gpus 1] [--no-cpu] [--quick]
"""

from __future__ import annotations

import argparse
import json
import math
import os
import sys
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
if ROOT not in sys.path:
    sys.path.insert(0, ROOT)

import torch  # noqa: E402

PEAK_FP8_TFLOPS = 5000.0  # MI355X dense fp8 MFMA
PEAK_HBM_GBS = 8000.0  # MI355X HBM3E
MALL_DEFEAT_BYTES = 600 * 2**20


def _timed(fn, steps: int, warmup: int, settle_s: float = 0.0) -> float:
    """Average ms per call of ``fn(i)`` over ``steps`` calls, HIP events on the
    current stream (the stream every kernel of the path is launched on).
    ``settle_s``: before the ``warmup`` calls, call ``fn`` (untimed) for that
    long, so the timed calls run at the clock the GPU settles to under this
    load rather than on its ramp up from idle (a few ms of calls would
    otherwise read 3-5 % slow, the first measurement of a process)."""
    t_end = time.perf_counter() + settle_s
    i = 0
    while time.perf_counter() < t_end:
        for _ in range(16):
            fn(i)
            i += 1
        torch.cuda.synchronize()
    for i in range(warmup):
        fn(i)
    torch.cuda.synchronize()
    start = torch.cuda.Event(enable_timing=True)
    end = torch.cuda.Event(enable_timing=True)
    start.record()
    for i in range(steps):
        fn(i)
    end.record()
    torch.cuda.synchronize()
    return start.elapsed_time(end) / steps


def _graph_timed(fn, reps: int, iters: int = 20) -> float:
    """Average ms per call of ``fn(i)`` (i cycling over ``reps`` buffers) from
    one HIP-graph replay of ``iters`` captured calls: the kernels' own time,
    without the Python launch overhead that dominates calls of a few us."""
    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(s):
        for i in range(reps):
            fn(i)
    torch.cuda.current_stream().wait_stream(s)
    torch.cuda.synchronize()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        for i in range(iters):
            fn(i % reps)
    g.replay()
    torch.cuda.synchronize()
    start = torch.cuda.Event(enable_timing=True)
    end = torch.cuda.Event(enable_timing=True)
    start.record()
    g.replay()
    end.record()
    torch.cuda.synchronize()
    return start.elapsed_time(end) / iters


def _copies(nbytes: int) -> int:
    return max(2, math.ceil(MALL_DEFEAT_BYTES / max(1, nbytes)))


def _gemm_case(dev, m, n, k, steps, warmup, seed, rotate=True, silu=False, layout="prearranged", settle_s=0.0):
    """W8A8 GEMM TFLOP/s over rotated operands.  ``layout``: "prearranged",
    the weights as ``Linear`` keeps them for its calls (rearranged once at
    load, untimed; ``fp8_scaled_mm_prearranged``), or "plain", the ``[K, N]``
    column-major view ``fp8_scaled_mm`` takes.  ``silu``: the SiLU-and-mul
    epilogue variant (half-width bf16 output; random weights, so their
    gate/up order does not matter)."""
    from flashrec_amd.kernel.sglops import (fp8_scaled_mm, fp8_scaled_mm_prearranged, fp8_scaled_mm_silu,
                                            per_token_quant_fp8, prearrange_fp8_weight)
    from flashrec_amd.layers.linear import quantize_weight_fp8

    g = torch.Generator(device=dev).manual_seed(seed)
    reps = _copies(m * k + n * k) if rotate else 1
    acts, weights = [], []
    for _ in range(reps):
        x = torch.randn(m, k, device=dev, generator=g, dtype=torch.float32).to(torch.bfloat16)
        w = (0.02 * torch.randn(n, k, device=dev, generator=g, dtype=torch.float32)).to(torch.bfloat16)
        acts.append(per_token_quant_fp8(x))
        q, s = quantize_weight_fp8(w)
        weights.append((prearrange_fp8_weight(q.t()) if layout == "prearranged" else q.t(), s))
        del x, w, q
    out = torch.empty(m, n // 2 if silu else n, dtype=torch.bfloat16, device=dev)

    def step(i):
        qa, sa = acts[i % reps]
        qw, sw = weights[i % reps]
        if layout == "prearranged":
            fp8_scaled_mm_prearranged(qa, qw, sa, sw, torch.bfloat16, out=out, silu=silu)
        elif silu:
            fp8_scaled_mm_silu(qa, qw, sa, sw, out)
        else:
            fp8_scaled_mm(qa, qw, sa, sw, torch.bfloat16)

    ms = _timed(step, steps, warmup, settle_s)
    del acts, weights, out
    flops = 2.0 * m * n * k
    return ms, flops / (ms * 1e-3) / 1e12


def _vendor_gemm_case(dev, m, n, k, steps, warmup, seed, rowwise=True):
    """The vendor library on the same shape, for comparison only: torch._scaled_mm
    (hipBLASLt on ROCm) with e4m3 operands rotated as in _gemm_case, per-row /
    per-column scales (``rowwise``, the path's own scaling) or one scale per
    tensor.  Returns (ms, TFLOP/s), or None when the build refuses the call."""
    g = torch.Generator(device=dev).manual_seed(seed)
    reps = _copies(m * k + n * k)
    ops = []
    for _ in range(reps):
        a = torch.randn(m, k, device=dev, generator=g).to(torch.float8_e4m3fn)
        b = (0.02 * torch.randn(n, k, device=dev, generator=g)).to(torch.float8_e4m3fn).t()
        if rowwise:
            sa = torch.rand(m, 1, device=dev, generator=g) + 0.5
            sb = torch.rand(1, n, device=dev, generator=g) + 0.5
        else:
            sa = torch.tensor(1.0, device=dev)
            sb = torch.tensor(1.0, device=dev)
        ops.append((a, b, sa, sb))

    def step(i):
        a, b, sa, sb = ops[i % reps]
        torch._scaled_mm(a, b, scale_a=sa, scale_b=sb, out_dtype=torch.bfloat16)

    try:
        step(0)
    except (RuntimeError, NotImplementedError):
        return None
    ms = _timed(step, steps, warmup)
    del ops
    return ms, 2.0 * m * n * k / (ms * 1e-3) / 1e12


def _decode_step_case(dev):
    """Config 4: the 28-layer decode step at 4096 beam rows (8 requests x 512
    beams over a 128-token shared prompt), one HIP-graph replay per step;
    its paged attention kernel timed alone over the same batch."""
    from flashrec_amd.attention import paged_attention, paged_attention_quant_fp8
    from flashrec_amd.decode_step import Qwen3FP8DecodeStep, Qwen3Shape

    shape = Qwen3Shape()
    m = Qwen3FP8DecodeStep(shape, requests=8, beams=512, prefix=128, step=2, device=dev,
                           trie_items=200000, trie_levels=3, trie_codes=256)
    m.capture(beam=True)
    for _ in range(3):
        m.replay()
    torch.cuda.synchronize()
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    n = 10
    e0.record()
    for _ in range(n):
        m.replay()
    e1.record()
    torch.cuda.synchronize()
    ms = e0.elapsed_time(e1) / n
    rows, h, inter = m.rows, shape.hidden, shape.intermediate
    qkv_n = (shape.q_heads + 2 * shape.kv_heads) * shape.head_dim
    gemm_flops = shape.layers * 2 * rows * (h * qkv_n + shape.q_heads * shape.head_dim * h
                                            + h * 2 * inter + inter * h)
    gemm_flops += 2 * rows * h * shape.sid_tokens
    out = {"config4_decode_step": {
        "ms": round(ms, 4), "GEMM_TFLOP/s": round(gemm_flops / (ms * 1e-3) / 1e12, 1),
        "gemm_tflop_per_step": round(gemm_flops / 1e12, 3), "layers": shape.layers, "rows": rows,
        "kv_len": m.seq_len, "timing": "one HIP graph per step, mean of 10 replays",
        "includes": "28 layers, fp8 SID lm_head + log_softmax, per-row top-1024 candidates, "
                    "3-level x 256 trie mask + top-512 per request + expand/advance",
        "trie_nodes": m.trie["n_nodes"]}}
    lp = torch.log_softmax(torch.randn(rows, shape.sid_tokens, device=dev), dim=-1)
    ms_b = _graph_timed(lambda _i: m.beam_step(lp), 1)
    out["config4_beam_tail"] = {"ms": round(ms_b, 5), "rows": rows, "candidates_per_row": m.beam_cand,
                                "select_k": m.beam_bw, "kernels": "row_topk + genrec (2 kernels)"}
    ms_f = _graph_timed(lambda _i: m.beam_step(lp, from_logits=True), 1)
    out["config4_beam_tail_from_logits"] = {
        "ms": round(ms_f, 5), "what": "the same tail taking the head's logits, the log-softmax folded into "
                                      "the row top-k (the decode step's form; replaces log_softmax + row_topk)"}
    p = m.attn._plan
    q = torch.randn(rows, shape.q_heads, shape.head_dim, device=dev).to(torch.bfloat16)
    o = torch.empty_like(q)
    k0, v0 = m.pool.k[0], m.pool.v[0]

    def step(_i):
        paged_attention(q, k0, v0, p["indices"], p["start"], p["len"], shape.head_dim ** -0.5, out=o,
                        group_prefix=p["group_prefix"])

    ms_a = _graph_timed(step, 1)
    flops = 4.0 * rows * shape.q_heads * m.seq_len * shape.head_dim
    out["config4_decode_attention"] = {"ms": round(ms_a, 5), "TFLOP/s": round(flops / (ms_a * 1e-3) / 1e12, 1),
                                       "bound": "bf16 MFMA + gather latency", "rows": rows, "kv_len": m.seq_len}
    codes = torch.empty(rows, shape.q_heads * shape.head_dim, dtype=torch.float8_e4m3fn, device=dev)
    scales = torch.empty(rows, 1, dtype=torch.float32, device=dev)

    def step_q(_i):
        paged_attention_quant_fp8(q, k0, v0, p["indices"], p["start"], p["len"], shape.head_dim ** -0.5,
                                  group_prefix=p["group_prefix"], out=codes, out_scale=scales)

    ms_aq = _graph_timed(step_q, 1)
    out["config4_decode_attention_quant"] = {
        "ms": round(ms_aq, 5), "rows": rows, "kv_len": m.seq_len,
        "what": "attention fused with the o projection's per-token e4m3 quant (the decode step's path)"}
    del m
    torch.cuda.empty_cache()
    return out


def _mfma_ceiling(dev, iters=40000):
    """Sustained rate of the GEMM's fp8 MFMA with register operands and no
    memory traffic (fr_calib_mfma_ceiling), one wave per SIMD on every CU,
    with constant and with random e4m3 operands, and the shader clock the
    kernel ran at (s_memtime over s_memrealtime): what the matrix cores reach
    on this board under its power management."""
    from flashrec_amd._lib import call

    cus = torch.cuda.get_device_properties(dev).multi_processor_count
    clocks = torch.zeros(2 * cus, dtype=torch.int64, device=dev)
    sink = torch.zeros(256, dtype=torch.float32, device=dev)
    st = torch.cuda.current_stream(dev).cuda_stream
    out = {}
    for name, rnd in (("constant_operands", 0), ("random_operands", 1)):
        call("fr_calib_mfma_ceiling", cus, 200, rnd, clocks.data_ptr(), sink.data_ptr(), st)
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        e0.record()
        call("fr_calib_mfma_ceiling", cus, iters, rnd, clocks.data_ptr(), sink.data_ptr(), st)
        e1.record()
        torch.cuda.synchronize()
        ms = e0.elapsed_time(e1)
        c = clocks.view(cus, 2).double().cpu()
        ghz = float((c[:, 0] / c[:, 1]).mean()) * 0.1
        flops = cus * 4 * iters * 4 * 2.0 * 32 * 32 * 64
        out[name] = {"TFLOP/s": round(flops / (ms * 1e-3) / 1e12, 1), "sclk_GHz": round(ghz, 3),
                     "frac_of_5PF": round(flops / (ms * 1e-3) / 1e12 / PEAK_FP8_TFLOPS, 4)}
    out["what"] = ("v_mfma_scale_f32_32x32x64_f8f6f4 on register operands, 4 chains per wave, one wave per "
                   "SIMD, no memory traffic; mean over the launch (HIP events)")
    return out


def _bw_case(fn_factory, dev, nbytes, reps):
    step, cleanup = fn_factory()
    ms = _graph_timed(step, reps)
    cleanup()
    return ms, nbytes / (ms * 1e-3) / 1e9


def _copy_same_bytes(dev, nbytes, reps):
    """A device-to-device copy moving the same bytes (nbytes/2 read, nbytes/2
    written), timed and rotated like the case: what a launch of this size
    reaches when it does nothing but stream."""
    half = max(nbytes // 2, 1)
    src = [torch.empty(half, dtype=torch.uint8, device=dev) for _ in range(reps)]
    dst = [torch.empty_like(t) for t in src]
    ms = _graph_timed(lambda i: dst[i].copy_(src[i]), reps)
    del src, dst
    return ms


def _rms_case(dev, m, h, rotate):
    from flashrec_amd.kernel.rms_fp8 import rmsnorm_per_token_quant_fp8

    nbytes = m * h * 2 + h * 2 + m * h + m * 4
    reps = _copies(nbytes) if rotate else 1

    def factory():
        xs = [torch.randn(m, h, device=dev).to(torch.bfloat16) for _ in range(reps)]
        gamma = (1 + 0.1 * torch.randn(h, device=dev)).to(torch.bfloat16)

        def step(i):
            rmsnorm_per_token_quant_fp8(xs[i % reps], gamma, 1e-6)

        return step, lambda: xs.clear()

    return factory, nbytes, reps


def _quant_case(dev, m, k):
    from flashrec_amd.kernel.sglops import per_token_quant_fp8

    nbytes = m * k * 2 + m * k + m * 4
    reps = _copies(nbytes)

    def factory():
        xs = [torch.randn(m, k, device=dev).to(torch.bfloat16) for _ in range(reps)]

        def step(i):
            per_token_quant_fp8(xs[i % reps])

        return step, lambda: xs.clear()

    return factory, nbytes, reps


def _silu_case(dev, m, d, rotate):
    from flashrec_amd.kernel.silu_fp8 import silu_and_mul_per_token_quant_fp8

    nbytes = m * 2 * d * 2 + m * d + m * 4
    reps = _copies(nbytes) if rotate else 1

    def factory():
        xs = [torch.randn(m, 2 * d, device=dev).to(torch.bfloat16) for _ in range(reps)]

        def step(i):
            silu_and_mul_per_token_quant_fp8(xs[i % reps])

        return step, lambda: xs.clear()

    return factory, nbytes, reps


def _rope_case(dev, t, hq, hk, d, slots, rotate):
    from flashrec_amd.kernel.qk_rope_kv import fused_qk_norm_rope_store_fp8
    from flashrec_amd.layers.rotary import build_cos_sin_cache

    nbytes = t * hq * d * 2 * 2 + 2 * t * hk * d * 2 + 2 * t * hk * d + 2 * t * 8 + 2 * d * 2
    reps = _copies(nbytes) if rotate else 1

    def factory():
        g = torch.Generator().manual_seed(3)
        bufs = []
        for _ in range(reps):
            q = torch.randn(t, hq, d, device=dev).to(torch.bfloat16)
            k = torch.randn(t, hk, d, device=dev).to(torch.bfloat16)
            v = torch.randn(t, hk, d, device=dev).to(torch.bfloat16)
            bufs.append((q, k, v))
        per_req = max(1, t // 8)
        prompt = torch.randint(64, 257, (8,), generator=g)
        step_no = torch.randint(0, 5, (8,), generator=g)
        pos = (prompt + step_no)[torch.clamp(torch.arange(t) // per_req, max=7)].to(dev)
        loc = (torch.randperm(slots - 1, generator=g)[:t] + 1).to(dev)
        cache = build_cos_sin_cache(d, 4096, 1e6).to(dev)
        kc = torch.zeros(slots, hk, d, dtype=torch.float8_e4m3fn, device=dev)
        vc = torch.zeros_like(kc)
        w = torch.ones(d, dtype=torch.bfloat16, device=dev)

        def step(i):
            q, k, v = bufs[i % reps]
            fused_qk_norm_rope_store_fp8(q, k, v, pos, loc, w, w, 1e-6, cache, kc, vc)

        return step, lambda: bufs.clear()

    return factory, nbytes, reps


def cpu_baseline(target_s: float = 3.0, runs: int = 3):
    """The reference's CPU torch path for the headline GEMM (torch._scaled_mm +
    per-row/per-channel rescale, python/flashrec/kernel/sglops.py:111-139) on a
    row sample of config 1 sized to ~``target_s`` seconds per run (at most all
    4096 rows), median of ``runs``; TFLOP/s."""
    from oracle import inputs, ops

    torch.set_num_threads(os.cpu_count() or 1)
    g = torch.Generator().manual_seed(1)
    x = torch.randn(4096, 2048, generator=g).to(torch.bfloat16)
    qa_all, sa_all = ops.per_token_quant_fp8(x)
    qw, sw = ops.quantize_weight_fp8(inputs.config1_weight())
    b = qw.t()
    ops.fp8_scaled_mm_torch_cpu(qa_all[:32], b, sa_all[:32], sw, torch.bfloat16)  # warm-up
    t0 = time.perf_counter()
    ops.fp8_scaled_mm_torch_cpu(qa_all[:64], b, sa_all[:64], sw, torch.bfloat16)  # probe
    probe = (time.perf_counter() - t0) / 64
    rows = int(min(4096, max(32, 32 * round(target_s / max(probe, 1e-9) / 32))))
    qa, sa = qa_all[:rows], sa_all[:rows]
    times = []
    while len(times) < runs or (sum(times) < 10.0 and len(times) < 30):
        t0 = time.perf_counter()
        ops.fp8_scaled_mm_torch_cpu(qa, b, sa, sw, torch.bfloat16)
        times.append(time.perf_counter() - t0)
    runs = len(times)
    sec = sorted(times)[len(times) // 2]
    flops = 2.0 * rows * 12288 * 2048
    return {
        "value": round(flops / sec / 1e12, 6),
        "unit": "TFLOP/s",
        "cores": torch.get_num_threads(),
        "kind": "port",
        "sample": f"gate_up W8A8 GEMM, {rows} of 4096 rows x N=12288 x K=2048 through "
                  f"torch._scaled_mm on CPU (reference sglops.py:111-139), median of {runs} "
                  f"runs of {sec:.2f} s; os.cpu_count()={os.cpu_count()}",
        "seconds_per_sample": round(sec, 3),
    }


def cpu_decode_step_extrapolated():
    """Config 4 on the host, as the baseline plan asks: one Qwen3-1.7B-shaped
    decoder layer at 4096 rows through the reference's CPU path (the oracle's
    restatement: RMSNorm->fp8, qkv / o / gate_up / down through
    torch._scaled_mm as sglops.py:111-139 runs it, QK-norm + RoPE + fp8 KV
    store, the bf16 gather + SDPA decode of flashinfer.py:380-431, SiLU->fp8),
    x 28 layers, plus the fp8 SID lm_head and log_softmax."""
    from oracle import ops

    torch.set_num_threads(os.cpu_count() or 1)
    g = torch.Generator().manual_seed(4)
    T, H, I, Hq, Hk, D, eps = 4096, 2048, 6144, 16, 8, 128, 1e-6
    reqs, prefix = 8, 128

    def wq(n, k):
        return ops.quantize_weight_fp8((0.02 * torch.randn(n, k, generator=g)).to(torch.bfloat16))

    (wqkv, sqkv), (wo, so), (wgu, sgu), (wd, sd) = wq((Hq + 2 * Hk) * D, H), wq(H, Hq * D), wq(2 * I, H), wq(H, I)
    nw = [(1 + 0.1 * torch.randn(n, generator=g)).to(torch.bfloat16) for n in (H, H, D, D)]
    slots = 1 + reqs * prefix + T
    kc = torch.randn(slots, Hk, D, generator=g).to(torch.float8_e4m3fn)
    vc = torch.randn(slots, Hk, D, generator=g).to(torch.float8_e4m3fn)
    pre = 1 + torch.arange(reqs * prefix, dtype=torch.int64).view(reqs, prefix)
    own = 1 + reqs * prefix + torch.arange(T, dtype=torch.int64)
    rows = torch.cat([pre.repeat_interleave(T // reqs, 0), own[:, None]], 1)  # [T, prefix + 1]
    kv_indices = rows.reshape(-1).to(torch.int32)
    kv_indptr = torch.arange(T + 1, dtype=torch.int64) * (prefix + 1)
    positions = torch.full((T,), prefix, dtype=torch.int64)
    cache = ops.cos_sin_cache(D, 4096, 1e6)
    x = torch.randn(T, H, generator=g).to(torch.bfloat16)
    residual = torch.randn(T, H, generator=g).to(torch.bfloat16)
    lm_w = (0.02 * torch.randn(8192, H, generator=g)).to(torch.bfloat16)

    def layer():
        t0 = time.perf_counter()
        q8, s8, res = ops.fused_add_rmsnorm_per_token_quant_fp8(x, residual, nw[0], eps)
        qkv = ops.fp8_scaled_mm_torch_cpu(q8, wqkv.t(), s8, sqkv, torch.bfloat16).view(T, Hq + 2 * Hk, D)
        q = ops.qk_norm_rope_store_fp8(qkv[:, :Hq], qkv[:, Hq:Hq + Hk], qkv[:, Hq + Hk:], positions, own,
                                       nw[2], nw[3], eps, cache, kc, vc)
        o = ops.sdpa_reference_style(q, kc, vc, kv_indices, kv_indptr)
        o8, os8 = ops.per_token_quant_fp8(o.reshape(T, Hq * D))
        h = ops.fp8_scaled_mm_torch_cpu(o8, wo.t(), os8, so, torch.bfloat16)
        q8, s8, res = ops.fused_add_rmsnorm_per_token_quant_fp8(h, res, nw[1], eps)
        gu = ops.fp8_scaled_mm_torch_cpu(q8, wgu.t(), s8, sgu, torch.bfloat16)
        y8, ys = ops.silu_and_mul_per_token_quant_fp8(gu)
        ops.fp8_scaled_mm_torch_cpu(y8, wd.t(), ys, sd, torch.bfloat16)
        return time.perf_counter() - t0

    def head():
        t0 = time.perf_counter()
        lw8, lws = ops.quantize_weight_fp8(lm_w)
        a8, a_s = ops.per_token_quant_fp8(residual)
        logits = ops.fp8_scaled_mm_torch_cpu(a8, lw8.t(), a_s, lws, torch.float32)
        torch.log_softmax(logits.float(), dim=-1)
        return time.perf_counter() - t0

    # the baseline plan's protocol: one warm-up, then the median of 5 runs
    layer_s = sorted([layer() for _ in range(6)][1:])[2]
    head_s = sorted([head() for _ in range(6)][1:])[2]
    return {"seconds_extrapolated": round(28 * layer_s + head_s, 3), "layer_s": round(layer_s, 3),
            "lm_head_s": round(head_s, 3), "layers": 28, "cores": torch.get_num_threads(),
            "runs": "median of 5 after 1 warm-up",
            "note": "one decoder layer on the host counted 28 times, plus the fp8 SID lm_head; the "
                    "trie mask / beam tail is not included"}


def main() -> int:
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=50)
    ap.add_argument("--warmup", type=int, default=10)
    ap.add_argument("--no-cpu", action="store_true", help="skip the CPU baseline")
    ap.add_argument("--quick", action="store_true", help="headline GEMM only")
    ap.add_argument("--copy-calibration", action="store_true",
                    help="only run 20 copies of a 256 MiB buffer (rocprof FETCH/WRITE_SIZE scale)")
    ap.add_argument("--mfma-ceiling", action="store_true",
                    help="only measure the fp8 MFMA rate on register operands (constant and random)")
    ap.add_argument("--decode-only", action="store_true",
                    help="only the config-4 decode step entries (for a kernel trace of the step)")
    args = ap.parse_args()
    if args.decode_only:
        from flashrec_amd._lib import load

        load()
        print(json.dumps(_decode_step_case(torch.device("cuda:0"))))
        return 0
    if args.mfma_ceiling:
        from flashrec_amd._lib import load

        load()
        print(json.dumps(_mfma_ceiling(torch.device("cuda:0"))))
        return 0
    if args.copy_calibration:
        src = torch.empty(256 * 2**20, dtype=torch.uint8, device="cuda")
        dst = torch.empty_like(src)
        for _ in range(20):
            dst.copy_(src)
        torch.cuda.synchronize()
        print(json.dumps({"copy_bytes_read_per_launch": 256 * 2**20,
                          "copy_bytes_written_per_launch": 256 * 2**20}))
        return 0
    if args.gpus != 1:
        print(f"bench.py measures one GPU; --gpus {args.gpus} is not supported "
              "(the FP8 path is measured on one GPU: its kernels shard by beam rows, one KV pool per GPU)", file=sys.stderr)
        return 2
    from flashrec_amd._lib import load

    load()
    dev = torch.device("cuda:0")
    torch.backends.cuda.matmul.allow_tf32 = False

    m, n, k = 4096, 12288, 2048
    settle_s = 0.25
    ms, tflops = _gemm_case(dev, m, n, k, args.steps, args.warmup, seed=1, settle_s=settle_s)
    traffic = None
    prof = os.path.join(ROOT, "profiles", "gemm_fp8_config1_traffic.json")
    if os.path.exists(prof):
        with open(prof) as f:
            traffic = json.load(f).get("hbm_bytes_per_launch")
    result = {
        "metric": "FP8 GEMM TFLOPS + quant/KV-write GB/s at 512-4096 beam rows; % of roofline",
        "value": round(tflops, 2),
        "unit": "TFLOP/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "settle_s": settle_s,
        "ms_per_step": round(ms, 5),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "e4m3 (fp32 accumulate, bf16 out)",
        "data": "synthetic (seeded N(0,1) activations, N(0,0.02) weights; operands rotated over >512 MB)",
        "config": {"workload": "config1 gate_up W8A8 GEMM", "M": m, "N": n, "K": k,
                   "a": "e4m3 per-token scale",
                   "b": "e4m3 per-channel scale, prearranged once at load as Linear keeps it "
                        "(the plain [K, N] column-major layout: extra.config1_gemm_plain_layout)"},
        "roofline": {"bound": "mfma", "achieved": round(tflops, 2), "peak": PEAK_FP8_TFLOPS,
                     "unit": "TFLOP/s", "frac": round(tflops / PEAK_FP8_TFLOPS, 4),
                     "traffic": traffic},
    }
    extra = {}
    if not args.quick:
        steps, warm = max(20, args.steps), args.warmup
        extra["mfma_ceiling"] = _mfma_ceiling(dev)
        msp, tfp = _gemm_case(dev, m, n, k, steps, warm, seed=1, layout="plain")
        extra["config1_gemm_plain_layout"] = {
            "ms": round(msp, 5), "TFLOP/s": round(tfp, 2), "frac": round(tfp / PEAK_FP8_TFLOPS, 4),
            "what": "the headline shape through fp8_scaled_mm on the [K, N] column-major weight view "
                    "(both operands staged through LDS)"}
        ms1, tf1 = _gemm_case(dev, 512, 12288, 2048, steps, warm, seed=11)
        extra["config1_gemm_M512"] = {"ms": round(ms1, 5), "TFLOP/s": round(tf1, 2),
                                      "frac": round(tf1 / PEAK_FP8_TFLOPS, 4)}
        for name, rw in (("vendor_hipblaslt_config1_rowwise", True), ("vendor_hipblaslt_config1_tensorwise", False)):
            vend = _vendor_gemm_case(dev, 4096, 12288, 2048, steps, warm, seed=7, rowwise=rw)
            if vend is not None:
                extra[name] = {"ms": round(vend[0], 5), "TFLOP/s": round(vend[1], 2),
                               "frac": round(vend[1] / PEAK_FP8_TFLOPS, 4),
                               "what": "torch._scaled_mm (hipBLASLt) on the headline shape, same operand "
                                       "rotation; for comparison, not this library"}
        msb, tfb = _gemm_case(dev, 8192, 8192, 8192, steps, warm, seed=9)
        extra["gemm_8192_cube"] = {"ms": round(msb, 5), "TFLOP/s": round(tfb, 2),
                                   "frac": round(tfb / PEAK_FP8_TFLOPS, 4)}
        mss, tfs = _gemm_case(dev, 4096, 12288, 2048, steps, warm, seed=3, silu=True)
        extra["config1_gate_up_silu_gemm"] = {
            "ms": round(mss, 5), "TFLOP/s": round(tfs, 2), "frac": round(tfs / PEAK_FP8_TFLOPS, 4),
            "what": "the headline GEMM with SiLU-and-mul in its epilogue (the decode step's gate_up)"}
        ms2, tf2 = _gemm_case(dev, 4096, 2048, 6144, steps, warm, seed=2)
        extra["config2_down_gemm"] = {"ms": round(ms2, 5), "TFLOP/s": round(tf2, 2),
                                      "frac": round(tf2 / PEAK_FP8_TFLOPS, 4)}
        for name, (mm, nn, kk) in {"config4_qkv_gemm": (4096, 4096, 2048),
                                   "config4_o_gemm": (4096, 2048, 2048),
                                   "config4_lm_head_gemm": (4096, 8192, 2048)}.items():
            msx, tfx = _gemm_case(dev, mm, nn, kk, steps, warm, seed=5)
            extra[name] = {"ms": round(msx, 5), "TFLOP/s": round(tfx, 2),
                           "frac": round(tfx / PEAK_FP8_TFLOPS, 4)}
        cases = {
            "config0_rms_fp8_M512": _rms_case(dev, 512, 2048, rotate=False),
            "config0_rms_fp8_M4096": _rms_case(dev, 4096, 2048, rotate=True),
            "rms_fp8_M65536": _rms_case(dev, 65536, 2048, rotate=True),
            "config2_silu_fp8": _silu_case(dev, 4096, 6144, rotate=True),
            "config3_qk_rope_kv": _rope_case(dev, 4096, 16, 8, 128, 65536, rotate=True),
            "qk_rope_kv_T32768": _rope_case(dev, 32768, 16, 8, 128, 65536, rotate=True),
            "per_token_quant_M65536": _quant_case(dev, 65536, 2048),
            "silu_fp8_M16384": _silu_case(dev, 16384, 6144, rotate=True),
        }
        result["extra_timing"] = ("GEMMs: HIP events around back-to-back launches; bandwidth kernels: "
                                  "one HIP-graph replay of 20 launches; inputs rotated over >512 MB "
                                  "except the 3 MB config-0 case; copy_ms_same_bytes: a device copy of the "
                                  "same bytes timed the same way (the streaming limit at that size)")
        for name, (factory, nbytes, reps) in cases.items():
            msb, gbs = _bw_case(factory, dev, nbytes, reps)
            extra[name] = {"ms": round(msb, 5), "GB/s": round(gbs, 1),
                           "frac": round(gbs / PEAK_HBM_GBS, 4), "bytes": nbytes}
            torch.cuda.empty_cache()
            extra[name]["copy_ms_same_bytes"] = round(_copy_same_bytes(dev, nbytes, reps), 5)
            torch.cuda.empty_cache()
        extra.update(_decode_step_case(dev))
        result["extra"] = extra
    if not args.no_cpu:
        result["cpu_baseline"] = cpu_baseline()
        if not args.quick:
            result["cpu_baseline"]["config4_decode_step"] = cpu_decode_step_extrapolated()
    print(json.dumps(result), flush=True)
    return 0


if __name__ == "__main__":
    sys.exit(main())
