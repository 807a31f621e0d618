"""Host-side logic of the package that needs no GPU (the reference's unit tests for it)."""

import pytest

from forgeserve_amd import BlockAllocator, ModelConfig, OutOfBlocks, TPContext


def test_config_validation():
    """tests/test_model.py:8-15 of the reference."""
    with pytest.raises(ValueError):
        ModelConfig(d_model=100, n_heads=3)
    with pytest.raises(ValueError):
        ModelConfig(n_heads=8, n_kv_heads=3)
    cfg = ModelConfig(vocab_size=64, d_model=64, n_layers=3, n_heads=8, n_kv_heads=4, max_seq_len=64)
    with pytest.raises(ValueError):
        cfg.check_tensor_parallel(3)
    cfg.check_tensor_parallel(4)
    assert cfg.ffn_dim == 192 and cfg.head_dim == 8
    assert ModelConfig(d_model=256, ffn_dim=688).ffn_dim == 688


def test_allocator():
    """tests/test_paged.py:10-17 of the reference, plus the exact LIFO order."""
    a = BlockAllocator(4)
    got = a.allocate(3)
    assert got == [0, 1, 2] and a.num_free == 1
    with pytest.raises(OutOfBlocks):
        a.allocate(2)
    a.release(got)
    assert a.num_free == 4
    assert a.allocate(2) == [2, 1]


def test_single_gpu_context():
    t = TPContext()
    assert t.size == 1 and t.rank == 0
    with pytest.raises(ValueError):
        TPContext(rank=1, size=1)
    with pytest.raises(NotImplementedError):
        TPContext(rank=0, size=2)
