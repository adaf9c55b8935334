"""Paged KV pool and request-slot pool: drop-ins for
``flashrec.kvcache.pool.TokenToKVPool`` (python/flashrec/kvcache/pool.py:66-145)
and ``ReqToTokenPool`` (pool.py:148-182), so the module can replace the
reference's whole ``flashrec.kvcache.pool``.

Interface kept: ``TokenToKVPool(num_layers, num_tokens, num_kv_heads,
head_dim, dtype, device)`` with per-layer ``k`` / ``v`` lists of
``[num_tokens, num_kv_heads, head_dim]`` tensors (page size 1),
``available_size()``, ``alloc(n)`` (a device int64 tensor of slot ids, or
``None`` when fewer than ``n`` slots are free), ``free(ids)``, ``store(layer,
k, v, loc)``, ``k_cache(layer)``, ``v_cache(layer)`` and ``last_alloc_cpu``.
Slot 0 is the padding slot that graph-captured batches point their unused
rows at, so it is never handed out and freeing it is a no-op.
``ReqToTokenPool(max_reqs, max_seq_len, device)`` keeps the int32
``req_to_token`` table ``[max_reqs, max_seq_len]`` and hands out request rows
1 .. max_reqs-1 with the same ``available_size`` / ``alloc`` / ``free`` /
``last_alloc_cpu`` contract (row 0 is the dummy row pointing at KV slot 0).

Design here:

* Free slots are a host-side LIFO stack held in a numpy array (push and pop
  of a run of ids are slice copies, no Python list per id).
* Allocated ids reach the device through ``_PinnedUpload``: the ids are
  written into pinned host memory and copied with a non-blocking H2D on the
  current stream, so ``alloc`` never waits for the work already queued on
  that stream (a pageable copy would, pool.py:3-6).  The pinned area is a
  ring; before a region is rewritten, the event recorded after the copy that
  last read it is waited for (normally long complete).  Each call returns a
  freshly allocated device tensor, so ids handed out earlier are never
  overwritten by later uploads.
* ``store`` writes through the HIP scatter kernels: bf16 or e4m3 K/V rows
  into an e4m3 pool (torch's ``.to(float8_e4m3fn)`` rounding), or bf16 rows
  into a bf16 pool.
"""

from __future__ import annotations

from collections import deque
from typing import Deque, List, Optional, Sequence, Tuple, Union

import numpy as np
import torch

from flashrec_amd.kernel.sglops import store_kv_cache

_POOL_DTYPES = (torch.float8_e4m3fn, torch.bfloat16)


def _host_ids(indices) -> np.ndarray:
    """Slot ids from a tensor (any device), a sequence or None, as int64."""
    if indices is None:
        return np.empty(0, dtype=np.int64)
    if isinstance(indices, torch.Tensor):
        return indices.detach().reshape(-1).to(device="cpu", dtype=torch.int64).numpy()
    return np.asarray(list(indices), dtype=np.int64).reshape(-1)


class _PinnedUpload:
    """Non-blocking host-to-device upload of small int64 id arrays."""

    def __init__(self, device: torch.device, capacity: int = 1 << 16):
        self.device = device
        self.capacity = int(capacity)
        self._host: Optional[torch.Tensor] = None  # pinned, allocated on first use
        self._cursor = 0
        # copies still possibly reading the ring: (start, end, event)
        self._inflight: Deque[Tuple[int, int, torch.cuda.Event]] = deque()

    def _reserve(self, n: int) -> int:
        if self._host is None or n > self.capacity:
            self._drain()
            self.capacity = max(self.capacity, 1 << (n - 1).bit_length())
            self._host = torch.empty(self.capacity, dtype=torch.int64, pin_memory=True)
            self._cursor = 0
        start = self._cursor if self._cursor + n <= self.capacity else 0
        end = start + n
        # in ring order the oldest copies sit right after the cursor: retire
        # every one whose range meets [start, end)
        while self._inflight and self._inflight[0][0] < end and start < self._inflight[0][1]:
            self._inflight.popleft()[2].synchronize()
        self._cursor = end
        return start

    def _drain(self) -> None:
        while self._inflight:
            self._inflight.popleft()[2].synchronize()

    def __call__(self, ids: np.ndarray) -> torch.Tensor:
        n = int(ids.size)
        if self.device.type != "cuda" or n == 0:
            return torch.from_numpy(np.array(ids, dtype=np.int64)).to(self.device)
        start = self._reserve(n)
        staged = self._host[start:start + n]
        staged.numpy()[:] = ids
        out = torch.empty(n, dtype=torch.int64, device=self.device)
        out.copy_(staged, non_blocking=True)
        done = torch.cuda.Event()
        done.record(torch.cuda.current_stream(self.device))
        self._inflight.append((start, start + n, done))
        return out


class _FreeStack:
    """Host-side LIFO of free ids ``1 .. n-1`` (0 is the padding id): ``take``
    pops the top ``k`` ids in stack order (the reference's ``free[-k:]``),
    ``give`` pushes ids back in the order given."""

    def __init__(self, n: int):
        self._stack = np.arange(1, int(n), dtype=np.int64)
        self._top = self._stack.size

    def __len__(self) -> int:
        return self._top

    def take(self, k: int) -> np.ndarray:
        taken = self._stack[self._top - k:self._top].copy()
        self._top -= k
        return taken

    def give(self, ids: np.ndarray) -> None:
        need = self._top + ids.size
        if need > self._stack.size:
            grown = np.empty(max(need, 2 * self._stack.size), dtype=np.int64)
            grown[:self._top] = self._stack[:self._top]
            self._stack = grown
        self._stack[self._top:need] = ids
        self._top = need


class _IdAllocator:
    """``available_size`` / ``alloc`` / ``free`` / ``last_alloc_cpu`` over a
    ``_FreeStack``, ids uploaded through ``_PinnedUpload`` (shared by both
    pools: the reference's two pools have the same allocation contract,
    pool.py:100-119 and :160-182)."""

    def _init_ids(self, n: int, device: torch.device) -> None:
        self._free_ids = _FreeStack(n)
        self._upload = _PinnedUpload(device)
        self.last_alloc_cpu: List[int] = []

    def available_size(self) -> int:
        return len(self._free_ids)

    def alloc(self, n: int) -> Optional[torch.Tensor]:
        """``n`` free ids on the pool's device, or ``None`` if fewer are free."""
        n = int(n)
        if n > len(self._free_ids):
            self.last_alloc_cpu = []
            return None
        if n <= 0:
            self.last_alloc_cpu = []
            return torch.empty(0, dtype=torch.int64, device=self.device)
        taken = self._free_ids.take(n)
        self.last_alloc_cpu = taken.tolist()
        return self._upload(taken)

    def free(self, indices: Optional[Union[torch.Tensor, Sequence[int]]]) -> None:
        """Return ids to the pool (the padding id 0 and negative ids are ignored)."""
        ids = _host_ids(indices)
        ids = ids[ids > 0]
        if ids.size:
            self._free_ids.give(ids)


class ReqToTokenPool(_IdAllocator):
    """Request rows of the ``req_to_token`` table (int32 KV slot ids per
    request position); row 0 is the dummy row (python/flashrec/kvcache/pool.py:148-182)."""

    def __init__(self, max_reqs: int, max_seq_len: int, device: torch.device):
        self.max_reqs = int(max_reqs)
        self.max_seq_len = int(max_seq_len)
        self.device = torch.device(device)
        self.req_to_token = torch.zeros((self.max_reqs, self.max_seq_len), dtype=torch.int32,
                                        device=self.device)
        self._init_ids(self.max_reqs, self.device)


class TokenToKVPool(_IdAllocator):
    """Per-layer K and V pages ``[num_tokens, num_kv_heads, head_dim]``; slot 0 is padding."""

    def __init__(self, num_layers: int, num_tokens: int, num_kv_heads: int, head_dim: int,
                 dtype: torch.dtype, device: torch.device):
        if dtype not in _POOL_DTYPES:
            raise TypeError(f"KV pool dtype must be float8_e4m3fn or bfloat16, got {dtype}")
        if int(num_tokens) < 1:
            raise ValueError("the pool needs at least the padding slot")
        self.num_layers = int(num_layers)
        self.num_tokens = int(num_tokens)
        self.num_kv_heads = int(num_kv_heads)
        self.head_dim = int(head_dim)
        self.dtype = dtype
        self.device = torch.device(device)
        self.row_dim = self.num_kv_heads * self.head_dim
        page_shape = (self.num_tokens, self.num_kv_heads, self.head_dim)
        self.k: List[torch.Tensor] = []
        self.v: List[torch.Tensor] = []
        for _ in range(self.num_layers):
            self.k.append(torch.zeros(page_shape, dtype=dtype, device=self.device))
            self.v.append(torch.zeros(page_shape, dtype=dtype, device=self.device))
        self._init_ids(self.num_tokens, self.device)

    def store(self, layer_id: int, k: torch.Tensor, v: torch.Tensor, loc: torch.Tensor) -> None:
        """``k_cache[loc] = k``, ``v_cache[loc] = v`` in the pool's dtype (pool.py:121-139)."""
        loc = loc.reshape(-1)
        rows = int(loc.numel())
        if rows == 0:
            return
        store_kv_cache(self.k[layer_id].view(self.num_tokens, self.row_dim),
                       self.v[layer_id].view(self.num_tokens, self.row_dim),
                       loc, k.reshape(rows, self.row_dim), v.reshape(rows, self.row_dim))

    def k_cache(self, layer_id: int) -> torch.Tensor:
        return self.k[layer_id]

    def v_cache(self, layer_id: int) -> torch.Tensor:
        return self.v[layer_id]
