"""Tensor-parallel context, kept as the size-1 case only (parallel.py:7-29 in the reference).

The hot path runs on one GPU: a context of size 1 is a no-op, and larger sizes are refused rather
than silently computing a partial result (no collective is implemented).
"""

import torch


class TPContext:
    def __init__(self, rank: int = 0, size: int = 1, group=None):
        if not 0 <= rank < size:
            raise ValueError("rank must be in [0, size)")
        if size != 1:
            raise NotImplementedError("forgeserve_amd runs on a single GPU: tensor parallelism is not built")
        self.rank, self.size, self.group = rank, size, group
        self.num_all_reduces = 0
        self.all_reduce_elements = 0

    def all_reduce(self, t: torch.Tensor) -> torch.Tensor:
        return t


SINGLE = TPContext()
