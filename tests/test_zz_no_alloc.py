"""fr_genrec_mask_topk_expand_noalloc (the fused beam step with its scratch in
a static device array) against fr_genrec_mask_topk_expand (caller-provided
scratch), both called through the C ABI on the same inputs: bit-exact on
every output, on two calls in a row, the second with a smaller input (the
static array keeps the first call's lists; nothing of them may leak)."""

import pytest
import torch

from flashrec_amd import _lib

pytestmark = pytest.mark.gpu


def _inputs(dev, n, bw, c, vocab, n_nodes, seed):
    g = torch.Generator().manual_seed(seed)
    cum = torch.randn(n, bw, generator=g) * 3
    lp = torch.sort(torch.randn(n, bw, c, generator=g), dim=-1, descending=True).values
    base = 500
    tok = base + torch.randint(0, vocab, (n, bw, c), generator=g)
    nodes = torch.randint(0, n_nodes, (n, bw), generator=g)
    allow = (torch.rand(n_nodes, vocab, generator=g) < 0.5).to(torch.uint8)
    nxt = torch.randint(0, n_nodes, (n_nodes, vocab), generator=g).to(torch.int32)
    ti = torch.randint(0, 50000, (n, bw, 4), generator=g)
    col = torch.randint(0, 4, (n,), generator=g).to(torch.int32)
    return [t.to(dev).contiguous() for t in (cum, lp, tok, nodes, allow, nxt, ti, col)], base


def _outputs(dev, n, bw, k):
    return [torch.full((n, k), -7.0, device=dev), torch.full((n, k), -7, dtype=torch.int64, device=dev),
            torch.full((n, k), -7, dtype=torch.int64, device=dev),
            torch.full((n, k), -7, dtype=torch.int64, device=dev),
            torch.full((n, bw, 4), -7, dtype=torch.int64, device=dev),
            torch.full((n, bw), -7, dtype=torch.int64, device=dev)]


def _call(lib, dev, ins, base, outs, n, bw, c, k, scratch=None):
    cum, lp, tok, nodes, allow, nxt, ti, col = ins
    vals, parents, toks, idx, ti_out, nodes_out = outs
    stream = torch.cuda.current_stream(dev).cuda_stream
    n_nodes, vsz = allow.shape
    common = (cum.data_ptr(), lp.data_ptr(), tok.data_ptr(), nodes.data_ptr(), allow.data_ptr(),
              ti.data_ptr(), ti_out.data_ptr(), nxt.data_ptr(), nodes_out.data_ptr(), None, col.data_ptr(),
              base, n_nodes, vsz, n_nodes, n, bw, c, k, 4, 1, 1, 1, 1, stream)
    head = (vals.data_ptr(), parents.data_ptr(), toks.data_ptr(), idx.data_ptr())
    if scratch is None:
        return lib.fr_genrec_mask_topk_expand_noalloc(*head, *common)
    return lib.fr_genrec_mask_topk_expand(*head, scratch.data_ptr(), scratch.numel(), *common)


@pytest.mark.parametrize("order", ["alone", "after_other_calls"])
def test_noalloc_matches_scratch_entry_point(dev, order):
    lib = _lib.load()
    if order == "after_other_calls":
        # a call of the scratch entry point on another size first: the static
        # array is separate from any caller buffer
        ins, base = _inputs(dev, 3, 64, 32, 300, 50, seed=99)
        sc = torch.empty(int(lib.fr_genrec_scratch_bytes(3, 64, 32)), dtype=torch.uint8, device=dev)
        assert _call(lib, dev, ins, base, _outputs(dev, 3, 64, 32), 3, 64, 32, 32, scratch=sc) == _lib.FR_OK
    # two calls in a row, the second smaller (fewer requests, beams, candidates, K)
    for n, bw, c, k, seed in ((8, 512, 1024, 512, 1), (3, 100, 64, 40, 2)):
        ins, base = _inputs(dev, n, bw, c, 768, 400, seed)
        need = int(lib.fr_genrec_scratch_bytes(n, bw, k))
        assert 0 < need <= _lib.GENREC_NOALLOC_SCRATCH_BYTES
        scratch = torch.empty(need, dtype=torch.uint8, device=dev)
        want = _outputs(dev, n, bw, k)
        got = _outputs(dev, n, bw, k)
        assert _call(lib, dev, ins, base, want, n, bw, c, k, scratch=scratch) == _lib.FR_OK
        assert _call(lib, dev, ins, base, got, n, bw, c, k) == _lib.FR_OK
        torch.cuda.synchronize()
        for a, b in zip(got, want):
            assert torch.equal(a, b), (n, bw, c, k)
        assert (want[0] > float("-inf")).any()


def test_noalloc_rejects_requests_past_its_capacity(dev):
    lib = _lib.load()
    n, bw, c, k = 64, 1024, 1024, 1024  # 64 x 64 slices x 1025 keys x 8 B = 32 MiB
    assert lib.fr_genrec_scratch_bytes(n, bw, k) > _lib.GENREC_NOALLOC_SCRATCH_BYTES
    ins, base = _inputs(dev, 1, 1, 1, 8, 2, seed=3)  # pointers only: nothing is launched
    outs = _outputs(dev, 1, 1, 1)
    assert _call(lib, dev, ins, base, outs, n, bw, c, k) == _lib.FR_ETOOLARGE
