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


def test_pool_key_layouts():
    """The two key storages of PagedKVPool and the fs_kv_layout each hands the kernels (host only: the
    pool lives on the CPU here and no kernel runs). Grouped keys: a key's 8-dim group g of slot s at
    s * 8 + g * 8 * block_size inside its (block, head) tile; the same element through pool.k."""
    import torch

    from forgeserve_amd import PagedKVPool

    cfg = ModelConfig(vocab_size=32, d_model=256, n_layers=2, n_heads=4, n_kv_heads=2, max_seq_len=64)
    d, bs = cfg.head_dim, 16
    slots = PagedKVPool(cfg, 6, bs, dtype=torch.bfloat16, device="cpu")
    groups = PagedKVPool(cfg, 6, bs, dtype=torch.bfloat16, device="cpu", key_layout="groups")
    ls, lg = slots.layout(1), groups.layout(1)
    assert (ls.k_slot, ls.k_dim, ls.k_group) == (d, 1, 0)
    assert (lg.k_slot, lg.k_dim, lg.k_group) == (8, 1, 8 * bs)
    assert lg.k_block == ls.k_block == 2 * bs * d and lg.k_head == ls.k_head == bs * d
    assert lg.k == groups.k_store[1].data_ptr() and lg.v_dim == ls.v_dim == bs
    assert tuple(groups.k[0].shape) == (6, 2, bs, d // 8, 8)
    # block 3, head 1, slot 5, dim 21 -> group 2, element 5 of it
    groups.k[1][3, 1, 5, 2, 5] = 7.0
    flat = groups.k_store[1].reshape(-1)
    assert float(flat[3 * lg.k_block + 1 * lg.k_head + 5 * lg.k_slot + 2 * lg.k_group + 5]) == 7.0
    assert float(groups.k[1].flatten(-2)[3, 1, 5, 21]) == 7.0
    with pytest.raises(ValueError):
        PagedKVPool(cfg, 6, bs, device="cpu", key_layout="rows")
    with pytest.raises(ValueError):
        PagedKVPool(ModelConfig(vocab_size=32, d_model=48, n_layers=1, n_heads=4, n_kv_heads=2, max_seq_len=16), 4,
                    device="cpu", key_layout="groups")
