"""fr_log_softmax_f32 (the SID head's log-probs) against torch's fp32
log_softmax on the CPU: the register-resident path (N = 8192, 4096) and the
generic one, in place and strided, with -inf and NaN rows."""

import pytest
import torch

pytestmark = pytest.mark.gpu


@pytest.mark.parametrize("m,n", [(4096, 8192), (37, 4096), (5, 1000), (3, 8192)])
def test_matches_torch(dev, m, n):
    from flashrec_amd.kernel.sglops import log_softmax_f32

    g = torch.Generator().manual_seed(m + n)
    x = torch.randn(m, n, generator=g) * 4
    got = log_softmax_f32(x.to(dev)).cpu()
    ref = torch.log_softmax(x, dim=-1)
    assert (got - ref).abs().max().item() < 2e-5
    assert torch.allclose(got.exp().sum(-1), torch.ones(m), atol=1e-4)


def test_in_place_strided_and_special_rows(dev):
    from flashrec_amd.kernel.sglops import log_softmax_f32

    g = torch.Generator().manual_seed(3)
    big = torch.randn(6, 8192 + 64, generator=g)
    big[1, :] = float("-inf")          # all -inf: NaN, as torch
    big[2, 100] = float("nan")         # NaN anywhere: NaN row
    big[3, 5:] = float("-inf")         # mostly masked: the five finite entries renormalise
    x = big[:, :8192]
    ref = torch.log_softmax(x, dim=-1)
    d = big.to(dev)
    view = d[:, :8192]
    log_softmax_f32(view, out=view)    # in place through a strided view
    got = d.cpu()[:, :8192]
    assert torch.equal(torch.isnan(got), torch.isnan(ref))
    fin = torch.isfinite(ref)
    assert (got[fin] - ref[fin]).abs().max().item() < 2e-5
    assert torch.equal(got[~fin & ~torch.isnan(ref)], ref[~fin & ~torch.isnan(ref)])
    assert torch.equal(d.cpu()[:, 8192:], big[:, 8192:])  # the tail past N untouched
