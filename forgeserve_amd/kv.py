"""Contiguous KV cache (kv.py:10-33 in the reference), kept in device memory in the pool layout.

A view stores the keys/values of one attention layer for B rows of equal length. Here it is a
one-block-per-row pool: keys (B, n_kv_heads, capacity, head_dim) and values stored dim-major
(B, n_kv_heads, head_dim, capacity) with capacity a multiple of 16, so the same attention kernel
serves contiguous and paged caches with bit-identical results. `update` appends at the current
length (kv.py:21-24); `truncate` only moves the length (kv.py:26-29), so speculative rollback copies
nothing. `.k`/`.v` are (B, n_kv_heads, length, head_dim) views, as in the reference.
"""

from typing import Optional, Tuple

import torch

from . import ops


def _round16(n: int) -> int:
    return -(-n // 16) * 16


class ContiguousKV:
    def __init__(self):
        self._k: Optional[torch.Tensor] = None   # (B, H, cap, D)
        self._vt: Optional[torch.Tensor] = None  # (B, H, D, cap)
        self._len = 0
        self._tables: Optional[torch.Tensor] = None

    # ---- reference surface -----------------------------------------------------------------------
    @property
    def length(self) -> int:
        return self._len

    @property
    def k(self) -> Optional[torch.Tensor]:
        return None if self._k is None else self._k[:, :, : self._len]

    @property
    def v(self) -> Optional[torch.Tensor]:
        return None if self._vt is None else self._vt[:, :, :, : self._len].transpose(2, 3)

    def update(self, k: torch.Tensor, v: torch.Tensor) -> Tuple[torch.Tensor, torch.Tensor]:
        """Append k, v (B, n_kv_heads, T, head_dim) and return every key/value so far."""
        b, h, t, d = k.shape
        self._reserve(b, h, d, t, k.dtype, k.device)
        slots = (self._len + torch.arange(t, device=k.device, dtype=torch.int32)).expand(b, t).contiguous()
        if k.stride() != v.stride() or k.stride(3) != 1:
            k, v = k.contiguous(), v.contiguous()
        ops.paged_kv_write(k, v, slots, self._tables, self.layout())
        self._len += t
        return self.k, self.v

    def truncate(self, n: int) -> None:
        """Keep only the first n positions (speculative rollback)."""
        if self._k is not None:
            self._len = min(self._len, max(0, n))

    # ---- device path used by the model -------------------------------------------------------------
    def layout(self):
        return ops.kv_layout(self._k, self._vt.transpose(2, 3))

    def _reserve(self, b: int, h: int, d: int, t: int, dtype, device) -> None:
        need = self._len + t
        if self._k is None:
            cap = _round16(max(need, 16))
            self._k = torch.zeros((b, h, cap, d), dtype=dtype, device=device)
            self._vt = torch.zeros((b, h, d, cap), dtype=dtype, device=device)
            self._tables = torch.arange(b, dtype=torch.int32, device=device).reshape(b, 1)
            return
        if self._k.shape[0] != b or self._k.shape[1] != h or self._k.shape[3] != d:
            raise ValueError(f"cache holds rows of shape {tuple(self._k.shape)}, got (B={b}, H={h}, D={d})")
        cap = self._k.shape[2]
        if need > cap:
            new_cap = _round16(max(need, 2 * cap))
            k2 = torch.zeros((b, h, new_cap, d), dtype=dtype, device=device)
            v2 = torch.zeros((b, h, d, new_cap), dtype=dtype, device=device)
            k2[:, :, : self._len].copy_(self._k[:, :, : self._len])
            v2[:, :, :, : self._len].copy_(self._vt[:, :, :, : self._len])
            self._k, self._vt = k2, v2

    def prepare(self, b: int, t: int, h: int, d: int, dtype, device, positions: torch.Tensor):
        """Make room for t new positions per row; returns (layout, tables, slots, mask positions).

        Keys are appended at slots length..length+t-1 while rotary and the causal mask use the
        given positions (model.py:67, 75); keys that do not exist yet are never visible."""
        self._reserve(b, h, d, t, dtype, device)
        slots = (self._len + torch.arange(t, device=device, dtype=torch.int32)).expand(b, t).reshape(-1)
        mask = positions.clamp(max=self._len + t - 1)
        return self.layout(), self._tables, slots.contiguous(), mask

    def commit(self, t: int) -> None:
        self._len += t


def new_contiguous_cache(n_layers: int):
    return [ContiguousKV() for _ in range(n_layers)]
