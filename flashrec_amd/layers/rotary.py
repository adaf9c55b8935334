"""RotaryEmbedding mirroring ``flashrec.layers.rotary`` (python/flashrec/layers/rotary.py).

The ``cos_sin_cache`` is ``[max_position, head_dim]`` fp32, cos half then sin
half, computed with the reference's exact torch formula (rotary.py:21-34) on
the CPU and then moved to the device, so its values do not depend on the
device's libm.  ``forward`` applies NeoX rotate-half RoPE in place through
the HIP kernel.
"""

from __future__ import annotations

import torch
import torch.nn as nn

from flashrec_amd.kernel.sglops import apply_rope_inplace, rope_inplace_any


def build_cos_sin_cache(head_dim: int, max_position: int, base: float) -> torch.Tensor:
    inv_freq = 1.0 / (base ** (torch.arange(0, head_dim, 2, dtype=torch.float32) / head_dim))
    t = torch.arange(max_position, dtype=torch.float32)
    freqs = torch.einsum("i,j->ij", t, inv_freq)
    return torch.cat((freqs.cos(), freqs.sin()), dim=-1)


class RotaryEmbedding(nn.Module):
    def __init__(self, head_dim: int, max_position: int, base: float, device=None):
        super().__init__()
        self.head_dim = int(head_dim)
        cache = build_cos_sin_cache(self.head_dim, int(max_position), float(base))
        if device is not None:
            cache = cache.to(device=device)
        self.register_buffer("cos_sin_cache", cache, persistent=False)

    def forward(self, positions: torch.Tensor, query: torch.Tensor, key: torch.Tensor):
        """In-place RoPE of query [T, Hq*D] / key [T, Hk*D]; returns (query, key)."""
        if not apply_rope_inplace(positions, query, key, self.head_dim, self.cos_sin_cache):
            rope_inplace_any(positions, query, key, self.head_dim, self.cos_sin_cache)
        return query, key
