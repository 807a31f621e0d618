"""Paged KV cache (paged.py:20-82 in the reference) with the pool resident in HBM.

The pool holds every layer in two allocations: keys (n_layers, num_blocks, n_kv_heads, block_size,
head_dim) and values stored dim-major (n_layers, num_blocks, n_kv_heads, head_dim, block_size).
`pool.k[layer]` and `pool.v[layer]` are (num_blocks, n_kv_heads, block_size, head_dim) views of them,
the reference's shape, so code that indexes the pool directly keeps working. One (block, kv-head)
tile of keys is block_size*head_dim contiguous elements (4 KB at 16 x 128 bf16), and the values of a
block for one dim are block_size contiguous elements: the attention kernel streams both with 16-byte
and 8-byte loads and never gathers.

`key_layout="groups"` stores each (block, kv-head) tile of keys as head_dim/8 groups of 8 dims, each
group holding every slot's 8 dims back to back (n_layers, num_blocks, n_kv_heads, head_dim/8,
block_size, 8). Each 16-byte-per-lane load of a key tile is then one contiguous 1 KB instead of
sixteen 64-byte pieces, which the attention kernels stream faster; the values, the arithmetic and
every result are the same.
`pool.k[layer]` is then a (num_blocks, n_kv_heads, block_size, head_dim/8, 8) view
(`.flatten(-2)` gives the reference's shape, as a copy).

The block allocator and the block tables stay on the host, as in the reference; tables are copied
to the GPU (int32) once per step and shared by every layer's view.
"""

from typing import Iterable, List, Optional, Tuple

import numpy as np
import torch

from . import ops
from .config import ModelConfig
from .parallel import SINGLE, TPContext
from ._lib import to_device


class OutOfBlocks(RuntimeError):
    pass


class BlockList(list):
    """A sequence's block ids: a list (the allocator's currency) that also keeps an int32 copy of
    itself, so the per-step block table of a batch is built with one array copy per row instead of
    converting Python ints. Appends (`+=`, `extend`, `append`) keep the copy current; any other
    mutation marks the copy stale and the next `array()` rebuilds it."""

    __slots__ = ("_arr", "_n", "_ver")

    def __init__(self, blocks: Iterable[int] = ()):
        super().__init__(blocks)
        self._arr = np.array(self, dtype=np.int32)
        self._n = len(self)
        self._ver = 0   # bumped by every mutation other than an append: a copy of a prefix is still valid
                        # while the version is unchanged

    def __iadd__(self, other):
        other = list(other)
        super().__iadd__(other)
        n, m = self._n, len(self)
        if n == m - len(other):   # the copy was current: append to it
            if self._arr.shape[0] < m:
                grown = np.empty(max(2 * self._arr.shape[0], m, 16), dtype=np.int32)
                grown[:n] = self._arr[:n]
                self._arr = grown
            self._arr[n:m] = other
            self._n = m
        return self

    def extend(self, other) -> None:
        self.__iadd__(other)

    def append(self, block: int) -> None:
        self.__iadd__([block])

    def _stale(name):
        def f(self, *a, **kw):
            self._n = -1
            self._ver += 1
            return getattr(list, name)(self, *a, **kw)
        f.__name__ = name
        return f

    __setitem__ = _stale("__setitem__")
    __delitem__ = _stale("__delitem__")
    __imul__ = _stale("__imul__")
    insert = _stale("insert")
    pop = _stale("pop")
    remove = _stale("remove")
    clear = _stale("clear")
    sort = _stale("sort")
    reverse = _stale("reverse")
    del _stale

    @property
    def version(self) -> int:
        """Changes whenever an entry already in the list may have changed (appends keep it)."""
        return self._ver

    def array(self) -> np.ndarray:
        """The ids as an int32 array (a view: valid until the list changes)."""
        if self._n != len(self):
            self._arr = np.array(self, dtype=np.int32)
            self._n = len(self)
        return self._arr[: self._n]


def block_table(lists: List[List[int]], device) -> torch.Tensor:
    """(B, max_blocks) int32 device table of B block lists, zero padded (engine.py:121-124 pads with
    block 0, which the positions mask). Rows that are BlockLists are copied as arrays."""
    arrs = [x.array() if isinstance(x, BlockList) else np.asarray(x, dtype=np.int32) for x in lists]
    width = max([1] + [a.shape[0] for a in arrs])
    t = np.zeros((len(arrs), width), dtype=np.int32)
    for i, a in enumerate(arrs):
        t[i, : a.shape[0]] = a
    return to_device(torch.from_numpy(t), device)


class BlockAllocator:
    """LIFO free list; block 0 is handed out first (paged.py:24-39)."""

    def __init__(self, num_blocks: int):
        self.num_blocks = num_blocks
        self._free = list(range(num_blocks - 1, -1, -1))

    @property
    def num_free(self) -> int:
        return len(self._free)

    def allocate(self, n: int) -> List[int]:
        if n > len(self._free):
            raise OutOfBlocks(f"need {n} blocks, {len(self._free)} free")
        out = self._free[len(self._free) - n:][::-1]
        del self._free[len(self._free) - n:]
        return out

    def release(self, blocks: List[int]) -> None:
        self._free.extend(blocks)


class PagedKVPool:
    """The block pool of every layer (paged.py:42-58). key_layout: "slots" (the reference's key shape,
    the default) or "groups" (keys as 8-dim groups of every slot; see the module docstring)."""

    def __init__(self, cfg: ModelConfig, num_blocks: int, block_size: int = 16, tp: TPContext = SINGLE,
                 dtype=torch.float32, device=None, key_layout: str = "slots"):
        if device is None:
            device = torch.device("cuda", torch.cuda.current_device()) if torch.cuda.is_available() else "cuda"
        h = cfg.n_kv_heads // tp.size
        d = cfg.head_dim
        self.cfg = cfg
        self.block_size = block_size
        self.num_blocks = num_blocks
        self.dtype = dtype
        self.device = torch.device(device)
        if key_layout == "slots":
            self.k_store = torch.zeros((cfg.n_layers, num_blocks, h, block_size, d), dtype=dtype, device=self.device)
            self.k = [self.k_store[i] for i in range(cfg.n_layers)]
        elif key_layout == "groups":
            if d % 8:
                raise ValueError(f"grouped keys need head_dim % 8 == 0 (head_dim {d})")
            self.k_store = torch.zeros((cfg.n_layers, num_blocks, h, d // 8, block_size, 8), dtype=dtype,
                                       device=self.device)
            self.k = [self.k_store[i].transpose(2, 3) for i in range(cfg.n_layers)]
        else:
            raise ValueError(f"key_layout must be 'slots' or 'groups', not {key_layout!r}")
        self.key_layout = key_layout
        self.v_store = torch.zeros((cfg.n_layers, num_blocks, h, d, block_size), dtype=dtype, device=self.device)
        self.v = [self.v_store[i].transpose(-1, -2) for i in range(cfg.n_layers)]
        self.allocator = BlockAllocator(num_blocks)
        self._layouts = None

    def blocks_for(self, n_tokens: int) -> int:
        return -(-n_tokens // self.block_size)

    def layout(self, layer: int):
        if self._layouts is None:
            self._layouts = [ops.kv_layout(self.k[i], self.v[i]) for i in range(len(self.k))]
        return self._layouts[layer]

    def views(self, block_tables: torch.Tensor, positions: torch.Tensor) -> List["PagedLayerView"]:
        """One view per layer for a step. block_tables: (B, max_blocks), positions: (B, T)."""
        step = _Step(self, block_tables, positions)
        return [PagedLayerView(self, layer, block_tables, positions, step) for layer in range(len(self.k))]


class _Step:
    """Device copies of a step's block tables and positions, shared by the views of every layer."""

    def __init__(self, pool: PagedKVPool, tables: torch.Tensor, positions: torch.Tensor):
        if tables.dim() != 2 or positions.dim() != 2 or tables.shape[0] != positions.shape[0]:
            raise ValueError(f"block_tables (B, max_blocks) and positions (B, T): {tuple(tables.shape)}, "
                             f"{tuple(positions.shape)}")
        if tables.device.type == "cpu" and tables.numel() and (int(tables.min()) < 0 or
                                                              int(tables.max()) >= pool.num_blocks):
            raise IndexError(f"block table entries must be in [0, {pool.num_blocks})")
        self.tables = to_device(tables.contiguous(), pool.device, torch.int32)
        self.positions = to_device(positions.contiguous(), pool.device, torch.int32)


class PagedLayerView:
    """What one attention layer sees during one step (paged.py:61-82)."""

    def __init__(self, pool: PagedKVPool, layer: int, block_tables: torch.Tensor, positions: torch.Tensor,
                 step: Optional[_Step] = None):
        self.pool, self.layer, self.tables, self.positions = pool, layer, block_tables, positions
        self._step = step if step is not None else _Step(pool, block_tables, positions)

    @property
    def length(self) -> int:
        raise NotImplementedError("paged views need explicit positions")

    @property
    def plan_key(self):
        """The step this view belongs to: every layer of it attends with the same tables and positions."""
        return self._step

    def update(self, k: torch.Tensor, v: torch.Tensor) -> Tuple[torch.Tensor, torch.Tensor]:
        """Write k, v (B, n_kv_heads, T, head_dim) at their positions, then return every table block of
        every row in table order, (B, n_kv_heads, max_blocks*block_size, head_dim)."""
        if k.stride() != v.stride() or k.stride(3) != 1:
            k, v = k.contiguous(), v.contiguous()
        lay = self.pool.layout(self.layer)
        ops.paged_kv_write(k, v, self._step.positions, self._step.tables, lay)
        return ops.paged_gather(lay, self._step.tables, self.pool.dtype, self.pool.device)

    # ---- device path used by the model -------------------------------------------------------------
    def prepare(self, b: int, t: int, h: int, d: int, dtype, device, positions: torch.Tensor):
        if dtype != self.pool.dtype:
            raise ValueError(f"pool dtype {self.pool.dtype} does not match the model's {dtype}")
        return self.pool.layout(self.layer), self._step.tables, None, positions

    def commit(self, t: int) -> None:
        pass


class PackedPrefill:
    """One prefill step over a pool for several sequences packed back to back, with no padding rows:
    sequence s has lens[s] new tokens at positions starts[s] .. starts[s] + lens[s] - 1, written through
    its block list block_lists[s] (which must cover them). The reference prefills one prompt per step
    with T = its length (engine.py:80-95 through paged.py:71-82); each token's keys, values and
    attention output here are bit-identical to that (the kernels' per-token arithmetic does not depend
    on the other tokens of the step)."""

    packed = True

    def __init__(self, pool: "PagedKVPool", block_lists: List[List[int]], starts: List[int], lens: List[int]):
        if not lens or len(block_lists) != len(lens) or len(starts) != len(lens):
            raise ValueError("packed prefill: one block list, start and length per sequence")
        bs = pool.block_size
        for blocks, st, n in zip(block_lists, starts, lens):
            if n <= 0 or st < 0:
                raise ValueError(f"packed prefill: length {n} at start {st}")
            if len(blocks) * bs < st + n:
                raise ValueError(f"packed prefill: {len(blocks)} blocks of {bs} do not hold positions < {st + n}")
            if any(not 0 <= b_ < pool.num_blocks for b_ in blocks):
                raise IndexError(f"block table entries must be in [0, {pool.num_blocks})")
        self.pool = pool
        self.n_seqs, self.n_tokens, self.T = len(lens), int(sum(lens)), int(max(lens))
        ln = np.asarray(lens, dtype=np.int64)
        cu = np.zeros(len(lens) + 1, dtype=np.int32)
        cu[1:] = np.cumsum(ln)
        pos_tok = np.concatenate([np.arange(st, st + n, dtype=np.int32) for st, n in zip(starts, lens)])
        token_row = np.repeat(np.arange(len(lens), dtype=np.int32), ln)
        pos_pad = np.full((len(lens), self.T), -1, dtype=np.int32)
        for r, (st, n) in enumerate(zip(starts, lens)):
            pos_pad[r, :n] = np.arange(st, st + n, dtype=np.int32)
        dev = pool.device
        self.max_position = int(max(st + n for st, n in zip(starts, lens))) - 1
        self.tables = block_table(block_lists, dev)
        self.cu = to_device(torch.from_numpy(cu), dev)
        self.pos_tok = to_device(torch.from_numpy(pos_tok), dev)
        self.token_row = to_device(torch.from_numpy(token_row), dev)
        self.pos_pad = to_device(torch.from_numpy(pos_pad), dev)
        self.last_rows = to_device(torch.from_numpy(cu[1:].astype(np.int64) - 1), dev)

    def views(self) -> List["PackedLayerView"]:
        return [PackedLayerView(self, layer) for layer in range(len(self.pool.k))]


class PackedLayerView:
    """What one attention layer sees during a packed prefill step."""

    packed = True

    def __init__(self, step: PackedPrefill, layer: int):
        self.step, self.layer = step, layer
        self.layout = step.pool.layout(layer)
