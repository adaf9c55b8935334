"""Attention fused with the o projection's per-token e4m3 quant
(``paged_attention_quant_fp8`` -> ``fr_paged_attention_quant_fp8``).

Bar: bit-exact against the two steps it replaces, the attention kernel
(itself held to the oracle in test_gpu_attention.py) followed by
``per_token_quant_fp8`` on its bf16 output, codes and scales alike, on the
shared-prefix (MFMA) groups, the token-by-token groups, partial last groups,
empty rows, strided queries and output rows, with and without the plan, and
at config 4's full size.  Head layouts the fused kernel refuses take the two
steps and must give the same bits too."""

import pytest
import torch

from oracle import ops

pytestmark = pytest.mark.gpu

E4M3 = torch.float8_e4m3fn
SCALE = 128 ** -0.5


def _pool(slots, hk, seed, spread=1.0):
    g = torch.Generator().manual_seed(seed)
    k = (torch.randn(slots, hk, 128, generator=g) * spread).to(E4M3)
    v = (torch.randn(slots, hk, 128, generator=g)).to(E4M3)
    return k, v


def _rows(lens, slots, g, prefix=None):
    rows = []
    for n in lens:
        own = torch.randint(1, slots, (n,), generator=g, dtype=torch.int32)
        rows.append(own if prefix is None else torch.cat([prefix, own]))
    idx = torch.cat(rows)
    ln = torch.tensor([int(r.numel()) for r in rows], dtype=torch.int32)
    start = torch.zeros(len(rows), dtype=torch.int32)
    start[1:] = torch.cumsum(ln[:-1], 0)
    return idx, start, ln


def _same(dev, q, k, v, idx, start, ln, plan=False, out_pad=0, label=""):
    from flashrec_amd.attention import attention_plan, paged_attention, paged_attention_quant_fp8
    from flashrec_amd.kernel.sglops import per_token_quant_fp8

    t, hq, d = q.shape
    hk = k.shape[1]
    dq, dk, dv, di, ds, dl = [x.to(dev) for x in (q, k, v, idx, start, ln)]
    if q.stride(1) != d:  # keep a strided query view strided on the device
        dq = q.to(dev)
    gp = attention_plan(di, ds, dl, hq, hk) if plan else None
    att = paged_attention(dq, dk, dv, di, ds, dl, SCALE, group_prefix=gp)
    ref_q, ref_s = per_token_quant_fp8(att.reshape(t, hq * d))
    out = None
    if out_pad:
        out = torch.empty(t, hq * d + out_pad, dtype=E4M3, device=dev)[:, : hq * d]
    got_q, got_s = paged_attention_quant_fp8(dq, dk, dv, di, ds, dl, SCALE, group_prefix=gp, out=out)
    torch.cuda.synchronize()
    assert got_q.shape == (t, hq * d) and got_s.shape == (t, 1)
    assert torch.equal(got_q.view(torch.uint8).cpu(), ref_q.view(torch.uint8).cpu()), f"codes {label}"
    assert torch.equal(got_s.view(torch.int32).cpu(), ref_s.view(torch.int32).cpu()), f"scales {label}"
    return att, got_q, got_s


@pytest.mark.parametrize("hq,hk", [(16, 8), (8, 8), (16, 4), (16, 2), (4, 1)])
@pytest.mark.parametrize("plan", [False, True])
def test_shared_prefix_beams(dev, hq, hk, plan):
    """Beams of two requests over 128-slot shared prefixes plus 3 own slots
    (the config-4 pattern); 45 tokens, so the last group is partial."""
    slots = 4096
    k, v = _pool(slots, hk, 30 + hq + hk, spread=2.0)
    g = torch.Generator().manual_seed(31)
    pre1 = torch.randperm(slots - 1, generator=g)[:128].to(torch.int32) + 1
    pre2 = torch.randperm(slots - 1, generator=g)[:128].to(torch.int32) + 1
    i1, s1, l1 = _rows([3] * 32, slots, g, pre1)
    i2, s2, l2 = _rows([3] * 13, slots, g, pre2)
    idx = torch.cat([i1, i2])
    start = torch.cat([s1, s2 + int(i1.numel())])
    ln = torch.cat([l1, l2])
    q = (torch.randn(45, hq, 128, generator=g) * 2).to(torch.bfloat16)
    _same(dev, q, k, v, idx, start, ln, plan=plan, label=f"{hq}/{hk}")


@pytest.mark.parametrize("hq,hk", [(16, 8), (16, 2), (8, 8)])
def test_token_path_ragged(dev, hq, hk):
    """No shared prefix: every group goes token by token; 1 .. 1000 keys."""
    lens = [1, 2, 7, 8, 9, 63, 64, 65, 128, 130, 257, 1000, 5, 17, 33, 40, 31, 3]
    slots = 4096
    k, v = _pool(slots, hk, 40 + hq)
    g = torch.Generator().manual_seed(41)
    idx, start, ln = _rows(lens, slots, g)
    q = torch.randn(len(lens), hq, 128, generator=g).to(torch.bfloat16)
    _same(dev, q, k, v, idx, start, ln, label=f"{hq}/{hk}")


def test_empty_rows_and_out_of_pool(dev):
    """Rows with no visible slot quantize zeros: scale 1e-12 / 448, codes 0."""
    slots, hk, hq = 256, 2, 4
    k, v = _pool(slots, hk, 50)
    idx = torch.tensor([3, 999, 5, -4, 7, 1 << 30, 9], dtype=torch.int32)
    start = torch.tensor([0, 0, 7, 1], dtype=torch.int32)
    ln = torch.tensor([7, 0, 0, 1], dtype=torch.int32)
    q = torch.randn(4, hq, 128).to(torch.bfloat16)
    _, codes, scales = _same(dev, q, k, v, idx, start, ln)
    assert (codes.view(torch.uint8).cpu()[1:] == 0).all()
    floor = torch.tensor(1e-12, dtype=torch.float32) / 448.0
    assert torch.equal(scales.cpu()[1:], floor.expand(3, 1))


def test_strided_queries_and_output_rows(dev):
    """q a view into the fused qkv rows; codes written into a wider buffer."""
    t, hq, hk, slots = 37, 16, 8, 1024
    k, v = _pool(slots, hk, 60)
    g = torch.Generator().manual_seed(61)
    qkv = torch.randn(t, (hq + 2 * hk) * 128, generator=g).to(torch.bfloat16).to(dev)
    q = qkv[:, : hq * 128].view(t, hq, 128)
    pre = torch.randperm(slots - 1, generator=g)[:64].to(torch.int32) + 1
    idx, start, ln = _rows([int(n) for n in torch.randint(0, 40, (t,), generator=g)], slots, g, pre)
    _same(dev, q, k, v, idx, start, ln, plan=True, out_pad=64)


@pytest.mark.parametrize("hq,hk", [(16, 16), (8, 1)])
def test_unfused_layouts_take_the_two_steps(dev, hq, hk):
    """More than 8 kv heads, or 8 query heads per kv head: the wrapper runs
    attention + quant itself (same bits)."""
    from flashrec_amd import _lib

    slots = 1024
    k, v = _pool(slots, hk, 70 + hq)
    g = torch.Generator().manual_seed(71)
    pre = torch.randperm(slots - 1, generator=g)[:64].to(torch.int32) + 1
    idx, start, ln = _rows([2] * 20, slots, g, pre)
    q = torch.randn(20, hq, 128, generator=g).to(torch.bfloat16)
    d = [x.to(dev) for x in (q, k, v, idx, start, ln)]
    codes = torch.empty(20, hq * 128, dtype=E4M3, device=dev)
    sc = torch.empty(20, dtype=torch.float32, device=dev)
    rc = _lib.load().fr_paged_attention_quant_fp8(
        d[0].data_ptr(), d[0].stride(0), d[0].stride(1), d[1].data_ptr(), d[1].stride(0), d[1].stride(1),
        d[2].data_ptr(), d[2].stride(0), d[2].stride(1), slots, d[3].data_ptr(), d[4].data_ptr(), d[5].data_ptr(),
        codes.data_ptr(), codes.stride(0), sc.data_ptr(), 20, hq, hk, 128, SCALE, None,
        torch.cuda.current_stream().cuda_stream)
    assert rc == _lib.FR_EUNSUPPORTED
    _same(dev, q, k, v, idx, start, ln, label=f"{hq}/{hk}")


def test_config4_full_size(dev):
    """8 requests x 512 beams over 128-slot prompts + 3 own slots, 16 / 8
    heads, 65536-slot pool: bit-exact with the two steps; the attention
    itself against the oracle on sampled rows."""
    slots, hq, hk = 65536, 16, 8
    k, v = _pool(slots, hk, 80)
    g = torch.Generator().manual_seed(81)
    perm = torch.randperm(slots - 1, generator=g).to(torch.int32) + 1
    idx_l, start_l, ln_l, off = [], [], [], 0
    for r in range(8):
        pre = perm[r * 128:(r + 1) * 128]
        own = perm[1024 + r * 512 * 3: 1024 + (r + 1) * 512 * 3].view(512, 3)
        for b in range(512):
            idx_l.append(torch.cat([pre, own[b]]))
    idx = torch.cat(idx_l)
    ln = torch.full((4096,), 131, dtype=torch.int32)
    start = torch.arange(4096, dtype=torch.int32) * 131
    q = torch.randn(4096, hq, 128, generator=g).to(torch.bfloat16)
    att, _, _ = _same(dev, q, k, v, idx, start, ln, plan=True, label="config 4")
    rows = torch.randperm(4096, generator=g)[:64]
    ref = torch.stack([ops.paged_attention(q[r: r + 1], k, v, idx, start[r: r + 1], ln[r: r + 1], SCALE)[0]
                       for r in rows.tolist()])
    err = ((att.cpu()[rows].float() - ref.float()).abs().amax(-1) / ref.float().abs().amax(-1).clamp(min=1e-6))
    assert err.max().item() < 1e-2
