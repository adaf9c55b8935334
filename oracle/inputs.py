"""Seeded synthetic inputs for the five benchmark configurations (CPU tensors).

TEST INFRASTRUCTURE ONLY.  Generated on the CPU with ``torch.Generator``
(seed = config index) so the oracle and the HIP kernels see identical inputs.
"""

from __future__ import annotations

import torch

QWEN3_1P7B = dict(hidden=2048, intermediate=6144, heads=16, kv_heads=8, head_dim=128, layers=28,
                  eps=1e-6, rope_theta=1e6)


def _gen(seed: int) -> torch.Generator:
    return torch.Generator().manual_seed(seed)


def config0(m: int = 512, h: int = 2048, seed: int = 0):
    """RMSNorm->FP8 input: x ~ N(0,1) bf16 with 1% of channels x20, gamma = 1 + N(0, 0.1)."""
    g = _gen(seed)
    x = torch.randn(m, h, generator=g)
    cols = torch.randperm(h, generator=g)[: max(1, h // 100)]
    x[:, cols] *= 20.0
    gamma = 1.0 + 0.1 * torch.randn(h, generator=g)
    return x.to(torch.bfloat16), gamma.to(torch.bfloat16), 1e-6


def weight(n: int, k: int, seed: int, std: float = 0.02) -> torch.Tensor:
    g = _gen(seed)
    return (std * torch.randn(n, k, generator=g)).to(torch.bfloat16)


def config1_weight(n: int = 12288, k: int = 2048) -> torch.Tensor:
    """gate_up weight, N(0, 0.02) bf16 [12288, 2048]."""
    return weight(n, k, seed=1)


def config2(m: int = 4096, d: int = 6144, n_out: int = 2048):
    """SiLU input [m, 2d] ~ N(0,1) bf16 and down-proj weight N(0, 0.02) [n_out, d]."""
    g = _gen(2)
    x = torch.randn(m, 2 * d, generator=g).to(torch.bfloat16)
    w = (0.02 * torch.randn(n_out, d, generator=g)).to(torch.bfloat16)
    return x, w


def config3(t: int = 4096, hq: int = 16, hk: int = 8, d: int = 128, slots: int = 65536,
            requests: int = 8, seed: int = 3):
    """QK-RoPE + KV write inputs.

    positions: per-request prompt length U[64, 256] plus a decode step 0..4;
    loc: the first t entries of a seeded permutation of slots 1..slots-1
    (slot 0 is the pool's dummy page).
    """
    g = _gen(seed)
    q = torch.randn(t, hq, d, generator=g).to(torch.bfloat16)
    k = torch.randn(t, hk, d, generator=g).to(torch.bfloat16)
    v = torch.randn(t, hk, d, generator=g).to(torch.bfloat16)
    per_req = max(1, t // requests)
    prompt = torch.randint(64, 257, (requests,), generator=g)
    step = torch.randint(0, 5, (requests,), generator=g)
    req_of_row = torch.clamp(torch.arange(t) // per_req, max=requests - 1)
    positions = (prompt + step)[req_of_row].to(torch.int64)
    loc = (torch.randperm(slots - 1, generator=g)[:t] + 1).to(torch.int64)
    return q, k, v, positions, loc
