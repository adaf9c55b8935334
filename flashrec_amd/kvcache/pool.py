"""Paged fp8 KV pool mirroring ``TokenToKVPool`` (python/flashrec/kvcache/pool.py:66-145).

Per layer, ``k[layer]`` / ``v[layer]`` are ``[num_tokens, num_kv_heads,
head_dim]`` tensors (page size 1); slot 0 is a dummy page that is never
allocated (pool.py:69, :95-96).  ``store`` converts bf16 K/V to the pool's
e4m3 and scatters them to ``loc`` in one HIP kernel.
"""

from __future__ import annotations

from typing import List, Optional, Sequence, Union

import torch

from flashrec_amd.kernel.sglops import store_kv_cache


def _as_cpu_ids(indices) -> List[int]:
    if indices is None:
        return []
    if isinstance(indices, torch.Tensor):
        return [int(i) for i in indices.detach().reshape(-1).cpu().tolist()]
    return [int(i) for i in indices]


class TokenToKVPool:
    def __init__(
        self,
        num_layers: int,
        num_tokens: int,
        num_kv_heads: int,
        head_dim: int,
        dtype: torch.dtype,
        device: torch.device,
    ):
        self.num_layers = num_layers
        self.num_tokens = int(num_tokens)
        self.num_kv_heads = num_kv_heads
        self.head_dim = head_dim
        self.dtype = dtype
        self.device = device
        self.row_dim = num_kv_heads * head_dim
        shape = (self.num_tokens, num_kv_heads, head_dim)
        self.k = [torch.zeros(shape, dtype=dtype, device=device) for _ in range(num_layers)]
        self.v = [torch.zeros(shape, dtype=dtype, device=device) for _ in range(num_layers)]
        # padded slot 0 is never allocated to a live request
        self._free: List[int] = list(range(1, self.num_tokens))
        self.last_alloc_cpu: List[int] = []

    def available_size(self) -> int:
        return len(self._free)

    def alloc(self, n: int) -> Optional[torch.Tensor]:
        n = int(n)
        if n <= 0:
            self.last_alloc_cpu = []
            return torch.empty(0, dtype=torch.int64, device=self.device)
        if n > len(self._free):
            self.last_alloc_cpu = []
            return None
        idx = self._free[-n:]
        del self._free[-n:]
        self.last_alloc_cpu = idx
        return torch.tensor(idx, dtype=torch.int64).to(self.device)

    def free(self, indices: Optional[Union[torch.Tensor, Sequence[int]]]) -> None:
        ids = [i for i in _as_cpu_ids(indices) if i > 0]
        if ids:
            self._free.extend(ids)

    def store(self, layer_id: int, k: torch.Tensor, v: torch.Tensor, loc: torch.Tensor) -> None:
        """``k_cache[loc] = k.to(dtype)`` and the same for v (pool.py:121-139)."""
        loc = loc.view(-1).to(dtype=torch.int64)
        n = int(loc.numel())
        if n == 0:
            return
        k = k.reshape(n, self.row_dim)
        v = v.reshape(n, self.row_dim)
        store_kv_cache(
            self.k[layer_id].view(-1, self.row_dim),
            self.v[layer_id].view(-1, self.row_dim),
            loc,
            k,
            v,
        )

    def k_cache(self, layer_id: int) -> torch.Tensor:
        return self.k[layer_id]

    def v_cache(self, layer_id: int) -> torch.Tensor:
        return self.v[layer_id]
