"""Kernel-level parity of the HIP path against the CPU oracle (bit-exact for integer/decision work,
within the stated tolerance for floating point). Every case prints its name before it launches."""

import math

import numpy as np
import pytest
import torch

from forgeserve_amd import _lib, ops
from oracle import reference_cpu as orc

pytestmark = pytest.mark.gpu
DEV = "cuda"


def case(*a):
    print("case:", *a, flush=True)


def rel_err(got, ref):
    return (got.double() - ref.double()).abs().max().item() / max(ref.double().abs().max().item(), 1e-30)


# ---- GEMM -------------------------------------------------------------------------------------------
@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
@pytest.mark.parametrize("m,n,k", [(1, 48, 64), (7, 256, 688), (64, 1000, 256), (65, 384, 512), (448, 640, 4096),
                                   (130, 96, 192), (20, 4096, 1024), (100, 2048, 2048),   # these two split K
                                   (448, 24592, 256),    # 224 x 256 tiles, a partial last column tile
                                   (448, 28672, 256), (448, 6144, 512), (448, 6000, 512)])   # 224 x 224, 224 x 96
def test_gemm_matches_fp64(dtype, m, n, k):
    case("gemm", dtype, m, n, k)
    g = torch.Generator().manual_seed(m * 7 + n)
    a = torch.randn(m, k, generator=g).to(dtype)
    w = (torch.randn(n, k, generator=g) * 0.05).to(dtype)
    ref = a.double() @ w.double().T
    out = ops.gemm(a.to(DEV), w.to(DEV)).cpu()
    tol = 1e-5 if dtype == torch.float32 else 8e-3
    assert rel_err(out, ref) < tol
    if dtype == torch.bfloat16:
        # one rounding of the f32 accumulation: at most one bf16 ulp from the exactly rounded product
        exact = ref.to(torch.bfloat16).float()
        assert ((out.float() - exact).abs() <= exact.abs() * 2 ** -7 + 1e-30).float().mean() > 0.999


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
@pytest.mark.parametrize("n,k", [(384, 512), (2048, 2048), (24576, 256),   # (2048, 2048) splits K four ways
                                 (28672, 256), (6144, 1024),   # 448 rows: 224 x 224 tiles; 224 x 96, K split in two
                                 (70000, 128)])   # 64 rows: 64 x 128 tiles
def test_gemm_rows_do_not_depend_on_the_batch(dtype, n, k):
    """A row's result is bit-identical whether it is computed alone, among 64 rows or among 448."""
    case("gemm invariance", dtype, n, k)
    g = torch.Generator().manual_seed(1)
    a = torch.randn(448, k, generator=g).to(dtype).to(DEV)
    w = (torch.randn(n, k, generator=g) * 0.05).to(dtype).to(DEV)
    full = ops.gemm(a, w)
    mid = ops.gemm(a[:64], w)
    for i in (0, 5, 63):
        assert torch.equal(ops.gemm(a[i: i + 1], w)[0], full[i])
        assert torch.equal(mid[i], full[i])
    assert torch.equal(ops.gemm(a[100:107], w), full[100:107])


@pytest.mark.parametrize("n,k", [(128, 256), (4096, 1024)])   # (4096, 1024) splits K
def test_gemm_residual_epilogue(n, k):
    case("gemm residual", n, k)
    g = torch.Generator().manual_seed(2)
    a = torch.randn(70, k, generator=g).bfloat16().to(DEV)
    w = (torch.randn(n, k, generator=g) * 0.05).bfloat16().to(DEV)
    r = torch.randn(70, n, generator=g).bfloat16().to(DEV)
    fused = ops.gemm(a, w, residual=r)
    two_step = (ops.gemm(a, w).float() + r.float()).bfloat16()   # x + linear(...) rounds twice
    assert torch.equal(fused, two_step)


@pytest.mark.parametrize("m,f,k", [(64, 14336, 4096), (448, 14336, 4096), (1, 8192, 2048), (130, 20000, 256),
                                   (448, 1000, 256)])
def test_gemm_swiglu_equals_gemm_then_silu_mul(m, f, k):
    """The gate|up projection with the SwiGLU gate in its epilogue gives exactly gemm then silu_mul."""
    case("gemm swiglu", m, f, k)
    from forgeserve_amd import _lib
    assert _lib.load().fs_gemm_splits(2 * f, k, _lib.BF16) == 1   # the fused kernel is the one under test
    g = torch.Generator().manual_seed(m + f)
    a = torch.randn(m, k, generator=g).bfloat16().to(DEV)
    w = (torch.randn(2 * f, k, generator=g) * 0.05).bfloat16().to(DEV)
    fused = ops.gemm_swiglu(a, w)
    two = ops.silu_mul(ops.gemm(a, w))
    assert fused.shape == (m, f)
    assert torch.equal(fused, two)


@pytest.mark.parametrize("m,n,k", [(70, 2048, 2048), (448, 4096, 4096), (64, 1024, 7168), (1, 2048, 2048)])
def test_splitk_add_rmsnorm_equals_gemm_then_norm(m, n, k):
    """A split-K projection reduced inside the residual-add + RMSNorm kernel gives exactly what the
    GEMM with its residual epilogue followed by add_rmsnorm gives (the reduction's and the norm's
    arithmetic, in the same order)."""
    case("splitk add_rmsnorm", m, n, k)
    from forgeserve_amd import _lib
    assert _lib.load().fs_gemm_splits(n, k, 1) > 1
    g = torch.Generator().manual_seed(m + n + k)
    a = torch.randn(m, k, generator=g).bfloat16().to(DEV)
    w = (torch.randn(n, k, generator=g) * 0.03).bfloat16().to(DEV)
    r = torch.randn(m, n, generator=g).bfloat16().to(DEV)
    nw = (1 + 0.1 * torch.randn(n, generator=g)).bfloat16().to(DEV)
    x, y = ops.gemm_add_rmsnorm(a, w, r, nw, 1e-5)
    x_ref = ops.gemm(a, w, residual=r)
    assert torch.equal(x, x_ref)
    assert torch.equal(y, ops.add_rmsnorm(x_ref, nw, 1e-5))


@pytest.mark.parametrize("n,splits", [(4096, 4), (2048, 8), (2048, 2), (1024, 4)])
def test_splitk_add_rmsnorm_rows_do_not_depend_on_the_batch(n, splits):
    """The split-K residual-add + RMSNorm gives a row the same bits in a 448-row call (loads group by
    group) as in a 64-row call (every load issued up front), for the row widths of the 8B and 1B
    models and one that takes the general path."""
    case("splitk add_rmsnorm rows", n, splits)
    from forgeserve_amd import _lib
    from forgeserve_amd._lib import ptr, stream_ptr
    lib = _lib.load()
    g = torch.Generator().manual_seed(n + splits)
    big, small = 448, 64
    parts = torch.randn(splits, big, n, generator=g).to(DEV)
    resid = torch.randn(big, n, generator=g).bfloat16().to(DEV)
    w = (1 + 0.1 * torch.randn(n, generator=g)).bfloat16().to(DEV)
    outs = {}
    for m in (big, small):
        p = parts[:, :m].contiguous()
        x = torch.empty(m, n, dtype=torch.bfloat16, device=DEV)
        y = torch.empty_like(x)
        assert lib.fs_splitk_add_rmsnorm(ptr(p), splits, ptr(resid), n, ptr(x), n, ptr(w), ptr(y), n, m, n, 1e-5,
                                         _lib.BF16, stream_ptr()) == 0
        outs[m] = (x, y)
    torch.cuda.synchronize()
    assert torch.equal(outs[big][0][:small], outs[small][0]) and torch.equal(outs[big][1][:small], outs[small][1])


@pytest.mark.parametrize("m,n,k", [(4133, 4096, 4096), (8192, 4096, 8192), (2600, 6144, 4096),
                                   (3900, 4100, 4096)])   # a partial last column tile
def test_gemm_serial_splits_equal_short_batch_rows(m, n, k):
    """A long batch whose workgroups run the K splits one after the other (no partials) gives every row
    bit for bit as a short batch gives it through the partials and their reduction, residual included,
    and gemm_add_rmsnorm at that length equals its short-batch rows too."""
    case("gemm serial splits", m, n, k)
    from forgeserve_amd import _lib
    lib = _lib.load()
    assert lib.fs_gemm_splits(n, k, _lib.BF16) > 1 and lib.fs_gemm_serial(m, n, k, _lib.BF16) == 1
    assert lib.fs_gemm_workspace_size(m, n, k, _lib.BF16) == 0
    assert lib.fs_gemm_serial(448, n, k, _lib.BF16) == 0   # the short batches below take the partials
    g = torch.Generator().manual_seed(m + n)
    a = torch.randn(m, k, generator=g).bfloat16().to(DEV)
    w = (torch.randn(n, k, generator=g) * 0.03).bfloat16().to(DEV)
    r = torch.randn(m, n, generator=g).bfloat16().to(DEV)
    nw = (1 + 0.1 * torch.randn(n, generator=g)).bfloat16().to(DEV)
    full = ops.gemm(a, w, residual=r)
    x, y = ops.gemm_add_rmsnorm(a, w, r, nw, 1e-5)
    assert torch.equal(x, full)
    for lo in (0, 1000, m - 300):   # the last slice ends in the long batch's ragged last tile
        hi = min(lo + 448, m)
        assert torch.equal(ops.gemm(a[lo:hi], w, residual=r[lo:hi]), full[lo:hi])
        _, ys = ops.gemm_add_rmsnorm(a[lo:hi], w, r[lo:hi], nw, 1e-5)
        assert torch.equal(y[lo:hi], ys)
    # and against float32 products on a few rows (bf16 output: half an ulp of the sum plus the rounding
    # of the product before the residual is added)
    ref = (a[-64:].float() @ w.float().T)
    got = ops.gemm(a, w)[-64:].float()
    assert ((got - ref).abs() <= ref.abs() * 2 ** -8 + 1e-3).all()


@pytest.mark.parametrize("m,n,k,kind", [(4133, 28672, 1024, "swiglu"), (2600, 4096, 14336, "gemm"),
                                        (3000, 1000, 256, "gemm")])
def test_long_batch_rows_equal_short_batch_rows(m, n, k, kind):
    """Long batches take 256-row tiles walked in groups of 8 row tiles (and, here, split-K partials or
    the SwiGLU epilogue); every row equals the same row computed in a short batch, bit for bit."""
    case("gemm long batch", m, n, k, kind)
    from forgeserve_amd import _lib
    assert not _lib.load().fs_gemm_serial(m, n, k, _lib.BF16)   # the partials / unsplit paths
    g = torch.Generator().manual_seed(m + k)
    a = torch.randn(m, k, generator=g).bfloat16().to(DEV)
    w = (torch.randn(n, k, generator=g) * 0.03).bfloat16().to(DEV)
    fn = ops.gemm_swiglu if kind == "swiglu" else ops.gemm
    full = fn(a, w)
    for lo in (0, 1111, m - 200):
        hi = min(lo + 448, m)
        assert torch.equal(fn(a[lo:hi], w), full[lo:hi])


# ---- row ops ------------------------------------------------------------------------------------------
@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
def test_rmsnorm_and_residual(dtype):
    case("rmsnorm", dtype)
    g = torch.Generator().manual_seed(3)
    x = torch.randn(33, 4096, generator=g).to(dtype)
    d = torch.randn(33, 4096, generator=g).to(dtype)
    w = (1 + 0.1 * torch.randn(4096, generator=g)).to(dtype)
    x_out = torch.empty_like(x, device=DEV)
    y = ops.add_rmsnorm(x.to(DEV), w.to(DEV), 1e-5, delta=d.to(DEV), x_out=x_out).cpu()
    xs = x + d
    assert torch.equal(x_out.cpu(), xs)
    ref = orc.rms_norm(xs, w, 1e-5)
    if dtype == torch.float32:
        torch.testing.assert_close(y, ref, atol=1e-5, rtol=1e-5)
    else:   # the sum of squares is ordered differently from torch's: at most one bf16 ulp apart
        assert ((y.float() - ref.float()).abs() <= ref.float().abs() * 2 ** -7 * 1.01).all()


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
def test_silu_mul(dtype):
    case("silu_mul", dtype)
    g = torch.Generator().manual_seed(4)
    gu = (torch.randn(17, 2 * 688, generator=g) * 3).to(dtype)
    h = ops.silu_mul(gu.to(DEV)).cpu()
    ref = torch.nn.functional.silu(gu[:, :688]) * gu[:, 688:]
    if dtype == torch.float32:
        torch.testing.assert_close(h, ref, atol=1e-6, rtol=1e-6)
    else:
        assert ((h.float() - ref.float()).abs() <= ref.float().abs() * 2 ** -7 * 1.01 + 1e-30).all()


def test_rmsnorm_and_silu_general_paths_bf16():
    """The row kernels' general paths (rows that are not whole 16-byte groups) against the reference,
    and silu_mul's two paths bit for bit (the same per-element arithmetic)."""
    case("rmsnorm/silu general paths")
    g = torch.Generator().manual_seed(5)
    x = torch.randn(9, 4100, generator=g).bfloat16()
    w = (1 + 0.1 * torch.randn(4100, generator=g)).bfloat16()
    y = ops.add_rmsnorm(x.to(DEV), w.to(DEV), 1e-5).cpu()
    ref = orc.rms_norm(x, w, 1e-5)
    assert ((y.float() - ref.float()).abs() <= ref.float().abs() * 2 ** -7 * 1.01).all()
    wide = (torch.randn(17, 2 * 688 + 1, generator=g) * 3).bfloat16().to(DEV)
    strided = wide[:, : 2 * 688]                       # leading dimension 1377: the element-wise path
    packed = strided.contiguous()                      # leading dimension 1376: the 16-byte path
    assert torch.equal(ops.silu_mul(strided), ops.silu_mul(packed))


@pytest.mark.parametrize("dtype,d", [(torch.bfloat16, 48), (torch.bfloat16, 52), (torch.float32, 52),
                                     (torch.float32, 4096)])   # 16-byte copies unless a row is 104 bytes
def test_embedding(dtype, d):
    case("embedding", dtype, d)
    w = torch.randn(100, d).to(dtype)
    ids = torch.tensor([[3, 99, 0], [7, 7, 50]])
    assert torch.equal(ops.embedding(ids.to(DEV), w.to(DEV)).cpu(), w[ids.reshape(-1)])
    # an id outside the vocabulary reads nothing and gives a zero row
    got = ops.embedding(torch.tensor([5, -1, 100]).to(DEV), w.to(DEV)).cpu()
    assert torch.equal(got[0], w[5]) and not got[1:].any()


# ---- KV write + rotary ----------------------------------------------------------------------------------
def _keys(pool, layer=0):
    """A pool layer's keys in the reference's (num_blocks, n_kv_heads, block_size, head_dim) shape."""
    return pool.k[layer].flatten(-2) if pool.key_layout == "groups" else pool.k[layer]


@pytest.mark.parametrize("key_layout", ["slots", "groups"])
@pytest.mark.parametrize("dtype,d,bs", [(torch.float32, 8, 4), (torch.float32, 32, 16), (torch.bfloat16, 128, 16),
                                        (torch.bfloat16, 64, 16), (torch.bfloat16, 24, 16)])   # 24: element path
def test_qkv_rope_write(dtype, d, bs, key_layout):
    case("qkv_rope_write", dtype, d, bs, key_layout)
    from forgeserve_amd import PagedKVPool, ModelConfig
    h, hkv, b, t = 8, 2, 3, 5
    cfg = ModelConfig(vocab_size=10, d_model=h * d, n_layers=1, n_heads=h, n_kv_heads=hkv, max_seq_len=200)
    s = orc.Shape.of(cfg)
    cos, sin = orc.rope_tables(s)
    pool = PagedKVPool(cfg, 40, bs, dtype=dtype, device=DEV, key_layout=key_layout)
    perm = torch.randperm(40, generator=torch.Generator().manual_seed(5))
    nbk = -(-44 // bs)                       # positions reach 43
    tables = perm[: b * nbk].reshape(b, nbk)
    pos = torch.tensor([[0, 1, 2, 3, 4], [17, 18, 19, 20, 21], [40, 41, 42, 43, -1]])
    qkv = torch.randn(b * t, (h + 2 * hkv) * d, generator=torch.Generator().manual_seed(6)).to(dtype)
    q = ops.qkv_rope_write(qkv.to(DEV), pos.reshape(-1).int().to(DEV), t, h, cos.to(DEV), sin.to(DEV),
                           tables.int().to(DEV), pool.layout(0)).cpu()
    x = qkv.view(b, t, h + 2 * hkv, d).transpose(1, 2)
    valid = pos.clamp(min=0)
    q_ref = orc.rotate(x[:, :h], cos, sin, valid).transpose(1, 2).reshape(b * t, h * d)
    k_ref = orc.rotate(x[:, h:h + hkv], cos, sin, valid)
    v_ref = x[:, h + hkv:]
    ok = (pos >= 0).reshape(-1)
    assert torch.equal(q[ok], q_ref[ok])
    kp, vp = _keys(pool).cpu(), pool.v[0].cpu()
    for bi in range(b):
        for ti in range(t):
            p = int(pos[bi, ti])
            if p < 0:
                continue
            blk = int(tables[bi, p // bs])
            assert torch.equal(kp[blk, :, p % bs], k_ref[bi, :, ti])
            assert torch.equal(vp[blk, :, p % bs], v_ref[bi, :, ti])


@pytest.mark.parametrize("t,d,partials", [(7, 128, False), (7, 128, True), (2, 64, False), (16, 128, True)])
def test_qkv_rope_write_window_across_blocks(t, d, partials):
    """A verify window's values are written by the window workgroups (tokens of a row in consecutive
    slots, lanes taking consecutive tokens of one dim): windows that cross a block boundary, a padding
    token, T = 2 (a workgroup writes several KV heads) and T = 16 (more tokens than KV heads). Keys and
    values equal the oracle's, and the pool equals the one written token by token (T = 1, each token
    through its row's table)."""
    case("qkv_rope_write window", t, d, partials)
    from forgeserve_amd import PagedKVPool, ModelConfig
    h, hkv, b, bs = 32, 8, 6, 16
    cfg = ModelConfig(vocab_size=10, d_model=h * d, n_layers=1, n_heads=h, n_kv_heads=hkv, max_seq_len=256)
    cos, sin = orc.rope_tables(orc.Shape.of(cfg))
    g = torch.Generator().manual_seed(40 + t)
    nb = 8
    tables = torch.randperm(b * nb, generator=g).reshape(b, nb)
    starts = torch.tensor([14, 31, 0, 60, 95, 47])          # windows across slots 15|16, 31|32, 63|64 ...
    pos = starts[:, None] + torch.arange(t)
    pos[1, -1] = -1                                          # a padding token
    n = (h + 2 * hkv) * d
    qkv = torch.randn(b * t, n, generator=g).bfloat16()
    pools = [PagedKVPool(cfg, b * nb, bs, dtype=torch.bfloat16, device=DEV, key_layout="groups") for _ in range(2)]
    args = (cos.to(DEV), sin.to(DEV))
    flat_pos = pos.reshape(-1).int().to(DEV)
    if partials:   # two split-K partials whose sum rounds to qkv's values
        p0 = torch.randn(b * t, n, generator=g)
        part = torch.stack([p0, qkv.float() - p0]).to(DEV).contiguous()
        lib = _lib.load()
        q = torch.empty((b * t, h * d), dtype=torch.bfloat16, device=DEV)
        tab = tables.int().to(DEV)
        ops.check(lib.fs_qkv_rope_write_partials(part.data_ptr(), 2, b * t, n, t, h, flat_pos.data_ptr(), 0,
                                                 args[0].data_ptr(), args[1].data_ptr(), args[0].shape[0],
                                                 tab.data_ptr(), tab.stride(0), tab.shape[1], pools[0].layout(0),
                                                 q.data_ptr(), q.stride(0), ops.stream_ptr()), "partials")
        qkv = (part[0] + part[1]).bfloat16().cpu()   # the values the kernel adds and rounds
    else:
        q = ops.qkv_rope_write(qkv.to(DEV), flat_pos, t, h, *args, tables.int().to(DEV), pools[0].layout(0))
    q_one = ops.qkv_rope_write(qkv.to(DEV), flat_pos, 1, h, *args, tables.repeat_interleave(t, 0).int().to(DEV),
                               pools[1].layout(0))
    ok = (pos >= 0).reshape(-1).to(DEV)
    assert torch.equal(q[ok], q_one[ok])
    assert torch.equal(pools[0].k_store, pools[1].k_store)
    assert torch.equal(pools[0].v_store, pools[1].v_store)
    x = qkv.view(b, t, h + 2 * hkv, d).transpose(1, 2)
    k_ref = orc.rotate(x[:, h:h + hkv], cos, sin, pos.clamp(min=0))
    v_ref = x[:, h + hkv:]
    kp, vp = _keys(pools[0]).cpu(), pools[0].v[0].cpu()
    nonzero = 0
    for bi in range(b):
        for ti in range(t):
            p = int(pos[bi, ti])
            if p < 0:
                continue
            blk = int(tables[bi, p // bs])
            assert torch.equal(kp[blk, :, p % bs], k_ref[bi, :, ti])
            assert torch.equal(vp[blk, :, p % bs], v_ref[bi, :, ti])
            nonzero += int(v_ref[bi, :, ti].ne(0).sum())
    assert int(pools[0].v_store.ne(0).sum()) == nonzero   # no other slot of the pool was written


# ---- paged attention --------------------------------------------------------------------------------------
def _paged_case(b, t, h, hkv, d, bs, ctx, nblocks, dtype, seed):
    g = torch.Generator().manual_seed(seed)
    maxb = max(-(-c // bs) for c in ctx)
    perm = torch.randperm(nblocks, generator=g)
    tables = torch.zeros(b, maxb, dtype=torch.long)
    used = 0
    for i, c in enumerate(ctx):
        nb = -(-c // bs)
        tables[i, :nb] = perm[used: used + nb]
        used += nb
    k = torch.randn(nblocks, hkv, bs, d, generator=g).to(dtype)
    v = torch.randn(nblocks, hkv, bs, d, generator=g).to(dtype)
    q = torch.randn(b, t, h, d, generator=g).to(dtype)
    pos = torch.tensor([[c - t + i for i in range(t)] for c in ctx])
    return q, k, v, tables, pos


def _oracle_attention(q, k, v, tables, pos, rep):
    """Gather the table blocks (paged.py:80-81) and run the oracle attention in f32."""
    b = q.shape[0]
    nb = tables.shape[1]
    k_all = k.float()[tables].permute(0, 2, 1, 3, 4).reshape(b, k.shape[1], nb * k.shape[2], k.shape[3])
    v_all = v.float()[tables].permute(0, 2, 1, 3, 4).reshape(b, k.shape[1], nb * k.shape[2], k.shape[3])
    out = orc.attention_math(q.float().transpose(1, 2), k_all, v_all, pos, rep)
    return out.transpose(1, 2)


def _run_attention(q, k, v, tables, pos, dtype, bs, key_layout="slots"):
    from forgeserve_amd import PagedKVPool, ModelConfig
    nblocks, hkv, _, d = k.shape
    h = q.shape[2]
    cfg = ModelConfig(vocab_size=8, d_model=h * d, n_layers=1, n_heads=h, n_kv_heads=hkv, max_seq_len=8)
    pool = PagedKVPool(cfg, nblocks, bs, dtype=dtype, device=DEV, key_layout=key_layout)
    pool.k[0].copy_(k.to(DEV).view(pool.k[0].shape))
    pool.v[0].copy_(v.to(DEV))
    out = ops.paged_attention(q.to(DEV), pool.layout(0), tables.int().to(DEV), pos.int().to(DEV),
                              1.0 / math.sqrt(d))
    return out, pool


@pytest.mark.parametrize("d,bs,t", [(8, 4, 3), (32, 16, 5), (16, 7, 2), (128, 16, 1)])
def test_attention_generic_f32(d, bs, t):
    case("attention f32", d, bs, t)
    ctx = [9, 40, 300, 513]
    q, k, v, tables, pos = _paged_case(4, t, 8, 2, d, bs, ctx, 300, torch.float32, d + bs)
    out, _ = _run_attention(q, k, v, tables, pos, torch.float32, bs)
    ref = _oracle_attention(q, k, v, tables, pos, 4)
    torch.testing.assert_close(out.cpu(), ref, atol=1e-5, rtol=1e-5)


@pytest.mark.parametrize("d,t,g", [(128, 5, 4), (128, 7, 4), (64, 5, 4), (128, 1, 4), (128, 9, 4), (64, 3, 8)])
def test_attention_mfma_bf16(d, t, g):
    case("attention bf16 mfma", d, t, g)
    hkv = 2
    ctx = [t + 1, 100, 257, 1000, 4097]
    q, k, v, tables, pos = _paged_case(len(ctx), t, hkv * g, hkv, d, 16, ctx, 600, torch.bfloat16, d * t + g)
    out, _ = _run_attention(q, k, v, tables, pos, torch.bfloat16, 16)
    ref = _oracle_attention(q, k, v, tables, pos, g)
    assert rel_err(out.cpu().float(), ref) < 2e-2


def test_attention_verify_equals_decode_bitwise():
    """A query's output does not depend on T: the k+1-token verify pass and 1-token decodes at the
    same positions produce identical bits (the batch-invariance that keeps greedy tokens identical)."""
    case("attention invariance")
    t = 7
    ctx = [300, 511, 512, 513, 2049]
    q, k, v, tables, pos = _paged_case(len(ctx), t, 32, 8, 128, 16, ctx, 800, torch.bfloat16, 9)
    full, pool = _run_attention(q, k, v, tables, pos, torch.bfloat16, 16)
    lay = pool.layout(0)
    tab = tables.int().to(DEV)
    for i in range(t):
        one = ops.paged_attention(q[:, i: i + 1].to(DEV), lay, tab, pos[:, i: i + 1].int().to(DEV),
                                  1.0 / math.sqrt(128))
        assert torch.equal(one[:, 0], full[:, i]), i
    # a row alone gives the same bits as inside the batch
    one_row = ops.paged_attention(q[3:4].to(DEV), lay, tab[3:4], pos[3:4].int().to(DEV), 1.0 / math.sqrt(128))
    assert torch.equal(one_row[0], full[3])


@pytest.mark.parametrize("d", [128, 64])
def test_attention_prefill_equals_decode_bitwise(d):
    """A prefill-shaped call (many query tiles per row, the kernel's prefill variant) gives every token
    the bits a one-token decode at its position gives it: prompts of 300 and 37 tokens after cached
    prefixes of 0 and 500, against 337 one-token calls."""
    case("attention prefill == decode", d)
    lens, starts = [300, 37], [0, 500]
    t = max(lens)
    ctx = [st + n for st, n in zip(starts, lens)]
    q, k, v, tables, _ = _paged_case(2, t, 32, 8, d, 16, ctx, 80, torch.bfloat16, 5 + d)
    pos = torch.full((2, t), -1, dtype=torch.long)
    for i, (st, n) in enumerate(zip(starts, lens)):
        pos[i, :n] = torch.arange(st, st + n)
    full, pool = _run_attention(q, k, v, tables, pos, torch.bfloat16, 16)
    lay, tab = pool.layout(0), tables.int().to(DEV)
    for i, n in enumerate(lens):
        for j in range(n):
            one = ops.paged_attention(q[i: i + 1, j: j + 1].to(DEV), lay, tab[i: i + 1], pos[i: i + 1, j: j + 1].int().to(DEV),
                                      1.0 / math.sqrt(d))
            assert torch.equal(one[0, 0], full[i, j]), (i, j)


@pytest.mark.parametrize("d,g,bs,lens,starts,qscale", [
    (128, 4, 16, [17000], [0], 1.0),             # the prompt crosses key 16384: two chunks and the combine
    (128, 4, 32, [700, 1500], [0, 300], 1.0),    # block size 32; row 0 has 800 padding tokens
    (64, 8, 16, [513, 90], [40, 0], 1.0),
    (128, 1, 16, [260], [3], 1.0),               # one head per KV head: 9 query tiles
    (128, 2, 48, [16500], [0], 1.0),             # blocks of 48 keys: the second chunk starts mid-block
    (128, 4, 16, [1100, 333], [0, 64], 12.0),    # scores spread over ~2^30: references move often
    (64, 4, 16, [700], [5], 12.0),
])
def test_attention_prefill_kernel_equals_unit_kernel_bitwise(d, g, bs, lens, starts, qscale):
    """The prefill kernel (groups of 8 query tiles sharing each key tile through LDS) gives every token
    the bits the unit kernel gives it: the same prompts cut into windows of 32 // g tokens (one query
    tile each, so the unit kernel runs), every window a batch row on the same table row. qscale
    stretches the scores so that a tile often lifts a row's reference maximum (the rescale paths)."""
    case("attention prefill kernel == unit kernel", d, g, bs, lens, qscale)
    hkv = 2
    h = hkv * g
    ctx = [st + n for st, n in zip(starts, lens)]
    nblocks = sum(-(-c // bs) for c in ctx) + 3
    t = max(lens)
    q, k, v, tables, _ = _paged_case(len(lens), t, h, hkv, d, bs, ctx, nblocks, torch.bfloat16, 100 + d + g + bs)
    q = (q.float() * qscale).bfloat16()
    pos = torch.full((len(lens), t), -1, dtype=torch.long)
    for i, (st, n) in enumerate(zip(starts, lens)):
        pos[i, :n] = torch.arange(st, st + n)
    full, pool = _run_attention(q, k, v, tables, pos, torch.bfloat16, bs)
    full = full.cpu()
    win = 32 // g
    lay = pool.layout(0)
    for i, n in enumerate(lens):
        nw = -(-n // win)
        qw = torch.zeros(nw, win, h, d, dtype=torch.bfloat16)
        pw = torch.full((nw, win), -1, dtype=torch.long)
        qw.view(-1, h, d)[:n] = q[i, :n]
        pw.view(-1)[:n] = pos[i, :n]
        tw = tables[i: i + 1].expand(nw, -1).contiguous()
        one = ops.paged_attention(qw.to(DEV), lay, tw.int().to(DEV), pw.int().to(DEV), 1.0 / math.sqrt(d)).cpu()
        got = one.view(-1, h, d)[:n]
        bad = (got != full[i, :n]).any(-1).any(-1).nonzero()
        assert bad.numel() == 0, f"row {i}: {bad.numel()} tokens differ, first {bad[:5].flatten().tolist()}"
        assert torch.count_nonzero(full[i, n:]) == 0   # padding tokens


@pytest.mark.parametrize("d,g,bs,t,b,lo_ctx,hi_ctx,qscale", [
    (128, 4, 16, 7, 200, 8, 4200, 1.0),       # verify windows, one chunk: outputs written directly
    (128, 4, 16, 7, 200, 8, 4200, 12.0),      # scores spread over ~2^30: partial maxima far apart
    (64, 8, 32, 5, 160, 3, 4100, 1.0),        # head_dim 64, block size 32
    (128, 2, 48, 3, 140, 3, 4100, 1.0),       # blocks of 48 keys
    (128, 4, 16, 1, 80, 16300, 16500, 1.0),   # decode over two chunks: partials for the combine
])
def test_attention_split_units_equal_unit_kernel_bitwise(d, g, bs, t, b, lo_ctx, hi_ctx, qscale):
    """A call of at most 128 (item, KV head) units whose tables hold at least 3072 keys runs each unit as
    two workgroups of four waves (the second to finish folds the other's partials in); any other call
    runs one workgroup of eight waves per unit. A row's outputs do not depend on which: the rows of one
    large call, recomputed in slices small enough to split, give identical bits."""
    case("attention split units == unit kernel", d, g, bs, t, b, qscale)
    hkv = 2
    gen = torch.Generator().manual_seed(d + g + bs + t + b)
    ctx = torch.randint(lo_ctx, hi_ctx + 1, (b,), generator=gen)
    ctx[: min(b, 4)] = torch.tensor([lo_ctx, hi_ctx, t, t + 1])[: min(b, 4)].clamp(min=t)
    maxb = -(-int(ctx.max()) // bs)
    nblocks = 2 * maxb + 7   # rows share blocks: tables draw from a small pool
    tables = torch.randint(0, nblocks, (b, maxb), generator=gen)
    k = torch.randn(nblocks, hkv, bs, d, generator=gen).bfloat16()
    v = torch.randn(nblocks, hkv, bs, d, generator=gen).bfloat16()
    q = (torch.randn(b, t, hkv * g, d, generator=gen) * qscale).bfloat16()
    pos = ctx[:, None] - t + torch.arange(t)[None, :]
    pos[1, 0] = -1   # a padding query
    split = _lib.load().fs_paged_attention_split()
    nsplit = -(-maxb * bs // split)
    units = lambda rows: rows * (-(-t * g // 32)) * nsplit * hkv   # noqa: E731
    step = max(r for r in range(1, b + 1) if units(r) <= 128)
    assert units(b) > 128 and step < b and maxb * bs >= 3072
    full, pool = _run_attention(q, k, v, tables, pos, torch.bfloat16, bs)
    full = full.cpu()
    lay, tab = pool.layout(0), tables.int().to(DEV)
    for lo in range(0, b, step):
        hi = min(b, lo + step)
        part = ops.paged_attention(q[lo:hi].to(DEV), lay, tab[lo:hi], pos[lo:hi].int().to(DEV), 1.0 / math.sqrt(d))
        bad = (part.cpu() != full[lo:hi]).any(-1).nonzero()
        assert bad.numel() == 0, f"rows {lo}:{hi}: {bad.shape[0]} outputs differ, first {bad[:3].tolist()}"
    assert torch.count_nonzero(full[1, 0]) == 0
    ref = _oracle_attention(q[2:8], k, v, tables[2:8], pos[2:8], g)
    assert rel_err(full[2:8].float(), ref) < 2e-2


def test_attention_split_units_replayed_from_a_graph():
    """The split-unit kernel captured in a HIP graph: each replay, with new queries copied in and other
    attention calls run eagerly between replays, gives the eager call's bits (the arrival counters
    are left at zero by every call, so a replay finds them as a fresh call does)."""
    case("attention split units in a graph")
    hkv, g, d, bs, t, b = 2, 4, 128, 16, 5, 8
    gen = torch.Generator().manual_seed(77)
    ctx = torch.randint(3000, 4201, (b,), generator=gen)
    maxb = -(-int(ctx.max()) // bs)
    assert maxb * bs >= 3072 and b * hkv <= 128   # the split kernel's conditions
    nblocks = 2 * maxb + 7
    tables = torch.randint(0, nblocks, (b, maxb), generator=gen)
    k = torch.randn(nblocks, hkv, bs, d, generator=gen).bfloat16()
    v = torch.randn(nblocks, hkv, bs, d, generator=gen).bfloat16()
    qs = [torch.randn(b, t, hkv * g, d, generator=gen).bfloat16().to(DEV) for _ in range(3)]
    pos = (ctx[:, None] - t + torch.arange(t)[None, :]).int().to(DEV)
    _, pool = _run_attention(qs[0].cpu(), k, v, tables, pos.cpu(), torch.bfloat16, bs)
    lay, tab = pool.layout(0), tables.int().to(DEV)
    sc = 1.0 / math.sqrt(d)
    want = [ops.paged_attention(q, lay, tab, pos, sc).clone() for q in qs]
    q_in = qs[0].clone()
    out = torch.empty_like(q_in)
    ops.paged_attention(q_in, lay, tab, pos, sc, out=out)   # sizes the workspace before the capture
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        ops.paged_attention(q_in, lay, tab, pos, sc, out=out)
    for rep in range(6):
        i = rep % 3
        q_in.copy_(qs[i])
        graph.replay()
        torch.cuda.synchronize()
        assert torch.equal(out, want[i]), rep
        # eager calls between replays: a split call on other rows, and an unsplit one (a table of
        # 2400 keys)
        ops.paged_attention(qs[(i + 1) % 3][:3], lay, tab[:3], pos[:3], sc)
        short = torch.full((b, 1), 2000 + rep, dtype=torch.int32, device=DEV)
        ops.paged_attention(qs[i][:, :1].contiguous(), lay, tab[:, :150].contiguous(), short, sc)
        torch.cuda.synchronize()


@pytest.mark.parametrize("d,g,bs,t,ctx,dtype", [
    (128, 4, 16, 7, [2048, 5000, 16380, 16389, 20000], torch.bfloat16),  # verify windows; two chunks + combine
    (128, 4, 16, 1, [300, 16385, 34000], torch.bfloat16),                # decode, 2 and 3 chunks
    (64, 8, 32, 5, [700, 1500, 33], torch.bfloat16),                     # block size 32, head_dim 64
    (128, 2, 48, 3, [16500, 100], torch.bfloat16),                       # blocks of 48 keys, 2 chunks
    (128, 4, 16, 600, [600, 1300], torch.bfloat16),                      # prompts: the prefill kernel
    (64, 4, 32, 300, [300, 17000], torch.bfloat16),                      # prefill kernel, head_dim 64, 2 chunks
    (32, 4, 16, 5, [9, 40, 300], torch.float32),                         # the generic kernel
])
def test_attention_grouped_keys_equal_slot_keys_bitwise(d, g, bs, t, ctx, dtype):
    """Keys stored as 8-dim groups (key_layout="groups") change only the addresses the kernels read
    them from: every output equals the slot-major pool's bit for bit (unit, prefill and generic
    kernels), and the grouped pool holds the same keys."""
    case("attention grouped keys", d, g, bs, t, ctx, dtype)
    hkv = 2
    nblocks = sum(-(-c // bs) for c in ctx) + 5
    q, k, v, tables, pos = _paged_case(len(ctx), t, hkv * g, hkv, d, bs, ctx, nblocks, dtype, 7 * d + bs + t)
    a, _ = _run_attention(q, k, v, tables, pos, dtype, bs)
    b, pool = _run_attention(q, k, v, tables, pos, dtype, bs, key_layout="groups")
    assert torch.equal(_keys(pool).cpu(), k)
    bad = (a != b).any(-1).nonzero()
    assert bad.numel() == 0, f"{bad.shape[0]} (row, token, head) outputs differ, first {bad[:3].tolist()}"


def test_attention_padding_rows_are_zero():
    case("attention padding")
    q, k, v, tables, pos = _paged_case(3, 3, 8, 2, 128, 16, [50, 70, 30], 20, torch.bfloat16, 4)
    pos[1, 2] = -1
    pos[2, :] = -1   # a row of padding only
    out, _ = _run_attention(q, k, v, tables, pos, torch.bfloat16, 16)
    assert torch.count_nonzero(out[1, 2]) == 0
    assert torch.count_nonzero(out[2]) == 0
    assert torch.count_nonzero(out[1, :2]) > 0


LONG_CTX = [8, 8192, 16383, 16384, 16385, 16391, 33000]   # one, two and three 16384-key chunks


def test_attention_long_contexts():
    """Contexts that span several key chunks: queries past the first chunk are merged from per-chunk
    partials, the others are finished by their chunk's workgroup."""
    case("attention long", LONG_CTX)
    q, k, v, tables, pos = _paged_case(len(LONG_CTX), 7, 8, 2, 128, 16, LONG_CTX, 6700, torch.bfloat16, 12)
    out, _ = _run_attention(q, k, v, tables, pos, torch.bfloat16, 16)
    ref = _oracle_attention(q, k, v, tables, pos, 4)
    assert rel_err(out.cpu().float(), ref) < 2e-2


def test_attention_long_verify_equals_decode_bitwise():
    case("attention long invariance", LONG_CTX)
    t = 7
    q, k, v, tables, pos = _paged_case(len(LONG_CTX), t, 8, 2, 128, 16, LONG_CTX, 6700, torch.bfloat16, 13)
    full, pool = _run_attention(q, k, v, tables, pos, torch.bfloat16, 16)
    lay = pool.layout(0)
    tab = tables.int().to(DEV)
    for i in range(t):
        one = ops.paged_attention(q[:, i: i + 1].to(DEV), lay, tab, pos[:, i: i + 1].int().to(DEV),
                                  1.0 / math.sqrt(128))
        assert torch.equal(one[:, 0], full[:, i]), i


def test_attention_plan_reuse_equals_fresh_plan():
    """The layers of a step reuse the first layer's work plan (plan_key): every layer's output is
    bit-identical to a call that builds its own plan; a call with other positions under the same key,
    or the reuse entry point called after a call with other positions, builds a new plan."""
    case("attention plan reuse")
    from forgeserve_amd import PagedKVPool, ModelConfig, _lib
    h, hkv, d, bs, t = 8, 2, 128, 16, 7
    ctx = [300, 17000, 40, 2100]   # 17000 keys span two chunks: the combine path runs too
    nblocks = sum(-(-c // bs) for c in ctx) + 2
    q, k, v, tables, pos = _paged_case(len(ctx), t, h, hkv, d, bs, ctx, nblocks, torch.bfloat16, 77)
    cfg = ModelConfig(vocab_size=8, d_model=h * d, n_layers=3, n_heads=h, n_kv_heads=hkv, max_seq_len=16)
    pool = PagedKVPool(cfg, nblocks, bs, dtype=torch.bfloat16, device=DEV)
    g = torch.Generator().manual_seed(5)
    for layer in range(3):
        pool.k[layer].copy_((k.float() + layer).bfloat16().to(DEV))
        pool.v[layer].copy_(torch.randn(v.shape, generator=g).bfloat16().to(DEV))
    qs = [(q.float() * (layer + 1)).bfloat16().to(DEV) for layer in range(3)]
    tab, p32 = tables.int().to(DEV), pos.int().to(DEV)
    sc = 1.0 / math.sqrt(d)
    fresh = [ops.paged_attention(qs[layer], pool.layout(layer), tab, p32, sc) for layer in range(3)]
    key = object()
    reused = [ops.paged_attention(qs[layer], pool.layout(layer), tab, p32, sc, plan_key=key) for layer in range(3)]
    for a, b in zip(fresh, reused):
        assert torch.equal(a, b)
    # same key, other positions (one query per row at the last position): a new plan
    p1 = p32[:, -1:].contiguous()
    one = ops.paged_attention(qs[0][:, -1:].contiguous(), pool.layout(0), tab, p1, sc, plan_key=key)
    assert torch.equal(one, ops.paged_attention(qs[0][:, -1:].contiguous(), pool.layout(0), tab, p1, sc))
    # the reuse entry point right after a call with other positions builds its own plan
    p2 = (p32 - 5).contiguous()
    want = ops.paged_attention(qs[1], pool.layout(1), tab, p2, sc)
    ops.paged_attention(qs[0], pool.layout(0), tab, p32, sc)
    lib = _lib.load()
    out = torch.empty_like(want)
    nb = tab.shape[1]
    ws = ops._persistent_ws("attention", lib.fs_paged_attention_workspace_size(len(ctx), t, h, d, nb, bs), DEV)
    qq = qs[1]
    ops.check(lib.fs_paged_attention_reuse_plan(ops.ptr(qq), qq.stride(0), qq.stride(1), qq.stride(2), pool.layout(1),
                                                ops.ptr(tab), tab.stride(0), nb, ops.ptr(p2), len(ctx), t, h, sc,
                                                ops.ptr(out), out.stride(0), out.stride(1), out.stride(2), ops.ptr(ws),
                                                ws.numel(), ops.stream_ptr()), "reuse")
    assert torch.equal(out, want)


def _packed(xs, lens, cu):
    """Dense (S, T, ...) rows -> packed (sum(lens), ...) tokens."""
    return torch.cat([xs[i, :n] for i, n in enumerate(lens)], 0)


@pytest.mark.parametrize("dtype,d,bs,lens,starts", [
    (torch.bfloat16, 128, 16, [37, 1, 300, 64, 8300], [0, 5, 100, 7, 0]),   # the last one spans two key chunks
    (torch.bfloat16, 64, 16, [15, 200, 3], [0, 0, 61]),
    (torch.float32, 32, 4, [9, 600, 1, 40], [3, 0, 0, 500]),
])
def test_attention_varlen_equals_dense(dtype, d, bs, lens, starts):
    """Packed sequences (no padding rows) give every token the bits the dense (S, T) call gives it, and
    leave the rows of out past the sequences' tokens untouched."""
    case("attention varlen", dtype, d, bs, lens)
    h, hkv = 8, 2
    ctx = [st + n for st, n in zip(starts, lens)]
    nblocks = sum(-(-c // bs) for c in ctx) + 3
    q, k, v, tables, _ = _paged_case(len(lens), max(lens), h, hkv, d, bs, ctx, nblocks, dtype, d + len(lens))
    pos = torch.full((len(lens), max(lens)), -1, dtype=torch.long)
    for i, (st, n) in enumerate(zip(starts, lens)):
        pos[i, :n] = torch.arange(st, st + n)
    dense, pool = _run_attention(q, k, v, tables, pos, dtype, bs)
    cu = torch.tensor([0] + list(np.cumsum(lens)), dtype=torch.int32)
    n_tok = int(cu[-1])
    qp = torch.cat([_packed(q, lens, cu), torch.randn(3, h, d).to(dtype)], 0).to(DEV)   # 3 rows past the tokens
    out = torch.full((n_tok + 3, h, d), 7.0, dtype=dtype, device=DEV)
    ops.paged_attention_varlen(qp, pool.layout(0), tables.int().to(DEV), pos.int().to(DEV), cu.to(DEV),
                               1.0 / math.sqrt(d), out=out)
    assert torch.equal(out[:n_tok], _packed(dense, lens, cu))
    assert bool((out[n_tok:] == 7.0).all())


@pytest.mark.parametrize("d", [128, 64])
def test_prefill_attention_matches_oracle(d):
    """Prefill-shaped attention (engine.py:80-95: a prompt's tokens attend causally to themselves and to
    what the cache holds, paged.py:71-82 with T = the prompt length): packed sequences of 37, 300 and
    2048 tokens, the 300-token one after a 500-token cached prefix, bf16, 32/8 heads, against the fp32
    oracle: max-abs error over max |out| < 2e-2 and mean-abs error < 2e-3, as for decode."""
    case("prefill attention vs oracle", d)
    lens, starts = [37, 300, 2048], [0, 500, 0]
    h, hkv, bs = 32, 8, 16
    ctx = [st + n for st, n in zip(starts, lens)]
    nblocks = sum(-(-c // bs) for c in ctx) + 5
    q, k, v, tables, _ = _paged_case(len(lens), max(lens), h, hkv, d, bs, ctx, nblocks, torch.bfloat16, 70 + d)
    pos = torch.full((len(lens), max(lens)), -1, dtype=torch.long)
    for i, (st, n) in enumerate(zip(starts, lens)):
        pos[i, :n] = torch.arange(st, st + n)
    from forgeserve_amd import ModelConfig, PagedKVPool
    cfg = ModelConfig(vocab_size=8, d_model=h * d, n_layers=1, n_heads=h, n_kv_heads=hkv, max_seq_len=8)
    pool = PagedKVPool(cfg, nblocks, bs, dtype=torch.bfloat16, device=DEV)
    pool.k[0].copy_(k.to(DEV))
    pool.v[0].copy_(v.to(DEV))
    cu = torch.tensor([0] + list(np.cumsum(lens)), dtype=torch.int32)
    out = ops.paged_attention_varlen(_packed(q, lens, cu).to(DEV), pool.layout(0), tables.int().to(DEV),
                                     pos.int().to(DEV), cu.to(DEV), 1.0 / math.sqrt(d)).float().cpu()
    ref = torch.cat([_oracle_attention(q[i: i + 1, :n], k, v, tables[i: i + 1], pos[i: i + 1, :n], h // hkv)[0]
                     for i, n in enumerate(lens)], 0)
    err = (out - ref).abs()
    rel = err.max().item() / ref.abs().max().item()
    print(f"prefill d={d}: max-abs/max {rel:.3e}, mean-abs {err.mean().item():.3e}")
    assert rel < 2e-2 and err.mean().item() < 2e-3


@pytest.mark.parametrize("b,t,h,hkv,k", [(64, 1, 8, 2, 1024), (64, 7, 8, 2, 1024), (9, 3, 32, 8, 4096)])
def test_qkv_rope_gemm_equals_gemm_then_rope(b, t, h, hkv, k):
    """The QKV projection reduced inside the rotary + pool write (split-K partials added by the rotary
    kernel) stores the same keys/values and returns the same queries as the projection followed by
    fs_qkv_rope_write; a padding token (position -1) is neither rotated nor written either way. A third
    pool keeps its keys as 8-dim groups and receives the same keys."""
    case("qkv_rope_gemm", b, t, h, hkv, k)
    from forgeserve_amd import PagedKVPool, ModelConfig, _lib
    d, bs = 128, 16
    n = (h + 2 * hkv) * d
    assert _lib.load().fs_gemm_splits(n, k, _lib.BF16) > 1   # the fused path is the one under test
    cfg = ModelConfig(vocab_size=10, d_model=h * d, n_layers=1, n_heads=h, n_kv_heads=hkv, max_seq_len=256)
    cos, sin = orc.rope_tables(orc.Shape.of(cfg))
    g = torch.Generator().manual_seed(b * 10 + t)
    x = torch.randn(b * t, k, generator=g).bfloat16().to(DEV)
    w = (torch.randn(n, k, generator=g) * 0.03).bfloat16().to(DEV)
    nb = 12
    tables = torch.randperm(b * nb, generator=g).reshape(b, nb).int().to(DEV)
    pos = torch.randint(0, nb * bs - t, (b, 1), generator=g) + torch.arange(t)
    pos[0, -1] = -1                                   # a padding token
    pos = pos.int().reshape(-1).to(DEV)
    pools = [PagedKVPool(cfg, b * nb, bs, dtype=torch.bfloat16, device=DEV) for _ in range(2)]
    q_two = ops.qkv_rope_write(ops.gemm(x, w), pos, t, h, cos.to(DEV), sin.to(DEV), tables, pools[0].layout(0))
    q_one = ops.qkv_rope_gemm(x, w, pos, t, h, cos.to(DEV), sin.to(DEV), tables, pools[1].layout(0))
    assert torch.equal(q_one, q_two)
    assert torch.equal(pools[1].k_store, pools[0].k_store)
    assert torch.equal(pools[1].v_store, pools[0].v_store)
    grouped = PagedKVPool(cfg, b * nb, bs, dtype=torch.bfloat16, device=DEV, key_layout="groups")
    q_grp = ops.qkv_rope_gemm(x, w, pos, t, h, cos.to(DEV), sin.to(DEV), tables, grouped.layout(0))
    assert torch.equal(q_grp, q_two)
    assert torch.equal(_keys(grouped), pools[0].k[0]) and torch.equal(grouped.v_store, pools[0].v_store)


@pytest.mark.parametrize("dtype,d,bs", [(torch.bfloat16, 128, 16), (torch.float32, 32, 4)])
def test_qkv_rope_write_varlen_equals_dense(dtype, d, bs):
    """The packed rotary + KV write stores every token where the dense (S, T) call stores it, returns
    the same rotated queries, and neither writes nor rotates a token whose table row is out of range."""
    case("qkv_rope_write varlen", dtype, d, bs)
    from forgeserve_amd import PagedKVPool, ModelConfig
    h, hkv = 8, 2
    lens, starts = [5, 1, 30, 12], [0, 9, 3, 40]
    cfg = ModelConfig(vocab_size=10, d_model=h * d, n_layers=1, n_heads=h, n_kv_heads=hkv, max_seq_len=128)
    s = orc.Shape.of(cfg)
    cos, sin = orc.rope_tables(s)
    g = torch.Generator().manual_seed(8)
    nb = -(-max(st + n for st, n in zip(starts, lens)) // bs)
    perm = torch.randperm(len(lens) * nb, generator=g)
    tables = perm.reshape(len(lens), nb).int()
    t = max(lens)
    qkv = torch.randn(len(lens), t, (h + 2 * hkv) * d, generator=g).to(dtype)
    pos = torch.full((len(lens), t), -1, dtype=torch.int32)
    for i, (st, n) in enumerate(zip(starts, lens)):
        pos[i, :n] = torch.arange(st, st + n, dtype=torch.int32)
    pos[2, 7] = -1                   # this token gets an out-of-range table row below: it must not be written
    dense_pool = PagedKVPool(cfg, len(lens) * nb, bs, dtype=dtype, device=DEV)
    q_dense = ops.qkv_rope_write(qkv.reshape(-1, qkv.shape[-1]).to(DEV), pos.reshape(-1).to(DEV), t, h, cos.to(DEV),
                                 sin.to(DEV), tables.to(DEV), dense_pool.layout(0)).view(len(lens), t, -1)
    cu = [0] + list(np.cumsum(lens))
    rows = torch.cat([torch.full((n,), i, dtype=torch.int32) for i, n in enumerate(lens)])
    rows[cu[2] + 7] = len(lens)       # out of range
    ppos = torch.cat([torch.arange(st, st + n, dtype=torch.int32) for st, n in zip(starts, lens)])
    pool = PagedKVPool(cfg, len(lens) * nb, bs, dtype=dtype, device=DEV)
    q = ops.qkv_rope_write_varlen(_packed(qkv, lens, cu).to(DEV), ppos.to(DEV), rows.to(DEV), h, cos.to(DEV),
                                  sin.to(DEV), tables.to(DEV), pool.layout(0))
    assert torch.equal(pool.k_store, dense_pool.k_store) and torch.equal(pool.v_store, dense_pool.v_store)
    qd = _packed(q_dense, lens, cu)
    keep = torch.ones(q.shape[0], dtype=torch.bool)
    keep[cu[2] + 7] = False
    assert torch.equal(q[keep.to(DEV)], qd[keep.to(DEV)])
    assert torch.count_nonzero(q[cu[2] + 7]) == 0


def test_attention_c3_shape():
    """B=32, T=5, 32/8 heads, D=128, bf16, contexts U[512, 4096], a 12288-block pool in random order."""
    case("attention c3")
    g = torch.Generator().manual_seed(6)
    ctx = torch.randint(512, 4097, (32,), generator=g).tolist()
    q, k, v, tables, pos = _paged_case(32, 5, 32, 8, 128, 16, ctx, 12288, torch.bfloat16, 6)
    out, _ = _run_attention(q, k, v, tables, pos, torch.bfloat16, 16)
    ref = _oracle_attention(q, k, v, tables, pos, 4)
    err = (out.cpu().float() - ref).abs()
    assert err.max().item() / ref.abs().max().item() < 2e-2
    assert err.mean().item() < 2e-3


# ---- sampling / acceptance ----------------------------------------------------------------------------
def _c2_inputs(b=64, k=5, v=32000, seed=3, dtype=torch.float32):
    tgt = torch.randn(b, k + 1, v, generator=torch.Generator().manual_seed(seed)) * 2.0
    dft = tgt[:, :k] + torch.randn(b, k, v, generator=torch.Generator().manual_seed(seed + 1)) * 0.5
    return tgt.to(dtype), dft.to(dtype)


@pytest.mark.parametrize("temperature", [1.0, 0.0, 0.7])
@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16, torch.float16])
def test_spec_accept_c2_bit_exact(temperature, dtype):
    """Batch 64, k=5, V=32000: accepted lengths, replacement and bonus tokens identical to the oracle's
    verify_draft on the same injected uniforms and Exp(1) noise."""
    case("spec_accept c2", temperature, dtype)
    b, k, v = 64, 5, 32000
    tgt, dft = _c2_inputs(dtype=dtype)
    g = torch.Generator().manual_seed(5)
    xs = torch.zeros(b, k, dtype=torch.int32)
    for bi in range(b):
        for i in range(k):
            if temperature == 0:
                xs[bi, i] = int(dft[bi, i].float().argmax())
            else:
                qrow = orc.probs_from_logits(dft[bi, i].float(), temperature)
                xs[bi, i] = orc.draw(qrow, orc.exp_noise(v, g))
    u = torch.rand(b, k, generator=g)
    e = torch.empty(b, v).exponential_(generator=g)
    k_eff = torch.tensor([k if i % 7 else i % 5 for i in range(b)], dtype=torch.int32)
    seq = torch.randint(100, 1000, (b,), generator=g, dtype=torch.int32)
    temps = torch.full((b,), float(temperature))
    out, n = ops.spec_accept(tgt.to(DEV), dft.to(DEV), xs.to(DEV), k_eff.to(DEV), temps.to(DEV), u.to(DEV), e.to(DEV),
                             seq_len=(seq_dev := seq.to(DEV)))
    out, n, seq_after = out.cpu(), n.cpu(), seq_dev.cpu()
    for bi in range(b):
        ke = int(k_eff[bi])
        tl = tgt[bi, : ke + 1]
        dl = dft[bi, :ke]
        p = orc.probs_from_logits(tl, temperature) if temperature else orc.probs_from_logits(tl.float(), 0)
        q = orc.probs_from_logits(dl, temperature) if temperature else orc.probs_from_logits(dl.float(), 0)
        acc, extra = orc.verify_with_noise(p, q, xs[bi, :ke].tolist(), u[bi], e[bi])
        assert int(n[bi]) == len(acc), bi
        assert out[bi, : len(acc) + 1].tolist() == acc + [extra], bi
        assert (out[bi, len(acc) + 1:] == -1).all()
        assert int(seq_after[bi]) == int(seq[bi]) + 1 + len(acc)


@pytest.mark.parametrize("temperature", [0.0, 0.8])
def test_sample_logits(temperature):
    case("sample_logits", temperature)
    g = torch.Generator().manual_seed(8)
    x = (torch.randn(37, 5003, generator=g) * 3).bfloat16()
    e = torch.empty(37, 5003).exponential_(generator=g)
    got = ops.sample_logits(x.to(DEV), temperature, e.to(DEV) if temperature else None).cpu().tolist()
    want = [orc.draw(orc.probs_from_logits(x[r].float(), temperature), e[r]) if temperature else int(x[r].argmax())
            for r in range(37)]
    assert got == want


@pytest.mark.parametrize("temperature", [0.0, 0.7, 1.0])
@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16, torch.float16])
def test_sample_logits_whole_groups(temperature, dtype):
    """Rows whose columns fill whole 16-byte groups (V = 32000 and 20000: the loads issued together, a
    partial last chunk for 20000), against the oracle's draw on the same noise."""
    case("sample_logits whole groups", temperature, dtype)
    g = torch.Generator().manual_seed(9)
    for v in (32000, 20000):
        x = (torch.randn(23, v, generator=g) * 3).to(dtype)
        e = torch.empty(23, v).exponential_(generator=g)
        got = ops.sample_logits(x.to(DEV), temperature, e.to(DEV) if temperature else None).cpu().tolist()
        want = [orc.draw(orc.probs_from_logits(x[r].float(), temperature), e[r]) if temperature
                else int(x[r].float().argmax()) for r in range(23)]
        assert got == want, v


def test_probs_from_logits():
    case("probs_from_logits")
    x = torch.randn(5, 20000) * 4
    p = ops.probs_from_logits(x.to(DEV), 0.7).cpu()
    torch.testing.assert_close(p, orc.probs_from_logits(x, 0.7), atol=1e-7, rtol=2e-5)
    hot = ops.probs_from_logits(x.bfloat16().to(DEV), 0).cpu()
    assert torch.equal(hot, orc.probs_from_logits(x.bfloat16(), 0))


def test_verify_draft_reference_streams():
    """forgeserve_amd.verify_draft on the GPU reproduces the reference's outcomes for seeded generators."""
    case("verify_draft golden")
    from forgeserve_amd import verify_draft
    from helpers import golden_json
    for c in golden_json("verify_cases.json"):
        p = torch.tensor(c["p"], dtype=torch.float32).to(DEV)
        q = torch.tensor(c["q"], dtype=torch.float32).reshape(c["k"], c["V"]).to(DEV)
        got = verify_draft(p, q, c["xs"], torch.Generator().manual_seed(c["seed"]))
        assert got == (c["accepted"], c["extra"]), c["seed"]



def _verify_probs_case(p, q, xs, u, e):
    out, n = ops.verify_probs(p.to(DEV), q.to(DEV), torch.tensor(xs, dtype=torch.int32).to(DEV), u.to(DEV),
                              e.to(DEV))
    n = int(n.cpu())
    return out.cpu()[: n + 1].tolist(), n


def test_residual_draw_ties_and_edge_sums():
    """The residual draw's corner cases, each against the oracle's verify_draft arithmetic:
    many equal keys across a chunk boundary (the first index wins), a residual that sums to zero
    (the draw falls back to p), and a residual too small for the candidates' relative bound."""
    case("residual draw corners")
    v = 10000
    base = torch.full((v,), 1.0 / v)
    u = torch.tensor([0.99])
    ones = torch.ones(v)
    # 1) equal residuals on columns 4090..4109 (two 4096-column chunks) with equal noise
    p = base.clone().reshape(1, v).repeat(2, 1)
    q = base.clone().reshape(1, v)
    q[0, 7] = 4.0 / v   # proposal 7 has ratio 1/4: rejected by u = 0.99
    p[0, 4090:4110] += 1.0 / v
    got = _verify_probs_case(p, q, [7], u, ones)
    want = orc.verify_with_noise(p, q, [7], u, ones)
    assert got == (want[0] + [want[1]], len(want[0])) and want[1] == 4090
    # 2) Σ max(p - q, 0) = 0: w = p
    p = base.clone().reshape(1, v).repeat(2, 1)
    p[0, 7] = 0.5 / v
    e = torch.empty(v).exponential_(generator=torch.Generator().manual_seed(21))
    got = _verify_probs_case(p, q[:, :].clone().fill_(1.0 / v), [7], u, e)
    qq = torch.full((1, v), 1.0 / v)
    want = orc.verify_with_noise(p, qq, [7], u, e)
    assert got == (want[0] + [want[1]], len(want[0]))
    # 3) a residual of 1e-36 at a single column: below the bound, the draw rescans exactly
    p = base.clone().reshape(1, v).repeat(2, 1)
    q = base.clone().reshape(1, v)
    p[0, 7] = 0.5 / v
    q[0, 1234] = 0.0
    p[0, 1234] = 1e-36
    got = _verify_probs_case(p, q, [7], u, e)
    want = orc.verify_with_noise(p, q, [7], u, e)
    assert got == (want[0] + [want[1]], len(want[0])) and want[1] == 1234


def test_residual_draw_random_rows_bit_exact():
    """Random probability rows (f32 and bf16) with forced rejections at every position."""
    case("residual draw random")
    g = torch.Generator().manual_seed(22)
    for dtype in (torch.float32, torch.bfloat16):
        for trial in range(6):
            k, v = 4, 32000 + 17 * trial
            p = torch.softmax(torch.randn(k + 1, v, generator=g) * 2, -1).to(dtype)
            q = torch.softmax(torch.randn(k, v, generator=g) * 2, -1).to(dtype)
            xs = torch.randint(0, v, (k,), generator=g).tolist()
            u = torch.rand(k, generator=g) * (0.2 if trial % 2 else 1.0)
            e = torch.empty(v).exponential_(generator=g)
            got = _verify_probs_case(p, q, xs, u, e)
            want = orc.verify_with_noise(p, q, xs, u, e)
            assert got == (want[0] + [want[1]], len(want[0])), (dtype, trial)


def _records(m, s, av, ai):
    """(..., 4) int32 records of softmax statistics (max, sum, argmax value, argmax index)."""
    f = torch.stack([m.float(), s.float(), av.float()], -1).contiguous().view(torch.int32)
    return torch.cat([f, ai.to(torch.int32)[..., None]], -1).contiguous()


@pytest.mark.parametrize("m,n,k", [(64, 5003, 256), (100, 4096, 128), (448, 6000, 256), (448, 25000, 128),
                                   (64, 70003, 128)])   # 64 x 128 tiles
def test_gemm_row_stats(m, n, k):
    """The head GEMM's statistics epilogue, merged per row, against torch on the stored logits:
    max and argmax exact, the sum of exponentials within float rounding."""
    case("gemm row stats", m, n, k)
    g = torch.Generator().manual_seed(m + n)
    a = (torch.randn(m, k, generator=g) * 0.5).bfloat16().to(DEV)
    w = (torch.randn(n, k, generator=g) * 0.5).bfloat16().to(DEV)
    temps = torch.tensor([0.0 if r % 5 == 0 else 0.5 + (r % 3) * 0.25 for r in range(m)], dtype=torch.float32)
    nparts = ops.row_stats_parts(m, n, k)
    assert nparts > 0
    parts = torch.empty((m, nparts, 4), dtype=torch.int32, device=DEV)
    out = ops.gemm_row_stats(a, w, temps.to(DEV), parts)
    assert torch.equal(out, ops.gemm(a, w))            # the logits are the plain GEMM's
    rs = ops.row_stats_merge(parts, torch.empty((m, 4), dtype=torch.int32, device=DEV)).cpu()
    x = out.cpu().float()
    # y = x / T as sampling.py:13 divides (T = 0 rows: y = x, only their argmax is used)
    y = torch.where(temps[:, None] > 0, x / temps.clamp(min=1e-30)[:, None], x)
    mx = y.max(-1).values
    fl = rs[:, :3].contiguous().view(torch.float32)
    assert torch.equal(fl[:, 0], mx)
    assert torch.equal(fl[:, 2], x.max(-1).values)
    assert torch.equal(rs[:, 3], x.argmax(-1).to(torch.int32))
    want = torch.exp((y - mx[:, None]).double()).sum(-1)
    assert ((fl[:, 1].double() - want).abs() / want).max() < 2e-6


@pytest.mark.parametrize("temperature", [1.0, 0.7, 0.0])
def test_spec_accept_with_row_stats_bit_exact(temperature):
    """fs_spec_accept_stats (statistics given, as the LM head emits them) against the oracle."""
    case("spec_accept row stats", temperature)
    b, k, v = 64, 5, 32000
    tgt, dft = _c2_inputs(dtype=torch.bfloat16)
    g = torch.Generator().manual_seed(7)
    xs = torch.zeros(b, k, dtype=torch.int32)
    for bi in range(b):
        for i in range(k):
            if temperature == 0:
                xs[bi, i] = int(dft[bi, i].float().argmax())
            else:
                xs[bi, i] = orc.draw(orc.probs_from_logits(dft[bi, i].float(), temperature), orc.exp_noise(v, g))
    u = torch.rand(b, k, generator=g)
    e = torch.empty(b, v).exponential_(generator=g)
    k_eff = torch.tensor([k if i % 5 else i % 4 for i in range(b)], dtype=torch.int32)
    temps = torch.full((b,), float(temperature))
    rows = torch.cat([tgt, dft], 1).float()                       # (b, 2k+1, v)
    y = rows / temperature if temperature > 0 else rows   # sampling.py:13's logits.float() / T
    mx = y.max(-1).values
    st = _records(mx, torch.exp((y - mx[..., None]).double()).sum(-1).float(), rows.max(-1).values,
                  rows.argmax(-1))
    out, n = ops.spec_accept(tgt.to(DEV), dft.to(DEV), xs.to(DEV), k_eff.to(DEV), temps.to(DEV), u.to(DEV),
                             e.to(DEV), row_stats=st.to(DEV))
    out, n = out.cpu(), n.cpu()
    for bi in range(b):
        ke = int(k_eff[bi])
        p = orc.probs_from_logits(tgt[bi, : ke + 1].float() if temperature == 0 else tgt[bi, : ke + 1], temperature)
        q = orc.probs_from_logits(dft[bi, :ke].float() if temperature == 0 else dft[bi, :ke], temperature)
        acc, extra = orc.verify_with_noise(p, q, xs[bi, :ke].tolist(), u[bi], e[bi])
        assert int(n[bi]) == len(acc), bi
        assert out[bi, : len(acc) + 1].tolist() == acc + [extra], bi


def _dirty_accept_workspace():
    """Fill the acceptance's workspace with 0xFF bytes (NaN records, index -1): a call must not depend
    on what an earlier call left there."""
    for (name, _), w in ops._PERSISTENT.items():
        if name == "accept":
            w.fill_(255)


def test_spec_accept_many_proposals_debug_outputs():
    """K = 70 proposals, so the step tests them in two batches of 64 (f32 logits, T = 1): sequence 0
    rejects proposal 10, sequence 1 accepts the first 64 and rejects proposal 66, sequence 2 accepts all
    70 (bonus token), sequence 3 has an out-of-range proposal id at 3 (never accepted). Tokens and counts
    against the oracle; the debug p(x), q(x) hold the oracle's values for every proposal the test
    evaluated (all of the first 64 batch, the second batch only when the first was all accepted) and
    stay untouched (NaN) for the others and for the out-of-range id; the residual sum."""
    case("spec_accept K=70 debug")
    b, k, v = 4, 70, 3001
    g = torch.Generator().manual_seed(41)
    tgt = torch.randn(b, k + 1, v, generator=g)
    dft = tgt[:, :k] + 0.05 * torch.randn(b, k, v, generator=g)
    p_all = [orc.probs_from_logits(tgt[i], 1.0) for i in range(b)]
    q_all = [orc.probs_from_logits(dft[i], 1.0) for i in range(b)]
    xs = torch.tensor([[orc.draw(q_all[i][j], orc.exp_noise(v, g)) for j in range(k)] for i in range(b)],
                      dtype=torch.int32)
    u = torch.zeros(b, k)          # u = 0 accepts any proposal with p(x) > 0
    u[0, 10] = 1.0                 # u = 1 rejects whatever the ratio
    u[1, 66] = 1.0
    xs[3, 3] = v                   # out of range: never accepted
    e = torch.empty(b, v).exponential_(generator=g)
    temps = torch.ones(b)
    out, n, dbg = ops.spec_accept(tgt.to(DEV), dft.to(DEV), xs.to(DEV), None, temps.to(DEV), u.to(DEV), e.to(DEV),
                                  debug=True)
    out, n = out.cpu(), n.cpu()
    dbg = {key: val.cpu() for key, val in dbg.items()}
    want_j = [10, 66, 70, 3]
    for i in range(b):
        xo, uo = xs[i].tolist(), u[i].clone()
        if i == 3:
            xo[3], uo[3] = 0, 1.0      # the same outcome: a rejection at 3
        acc, extra = orc.verify_with_noise(p_all[i], q_all[i], xo, uo, e[i])
        assert len(acc) == want_j[i] and int(n[i]) == len(acc), i
        assert out[i, : len(acc) + 1].tolist() == acc + [extra], i
        evaluated = set(range(64)) | (set(range(64, k)) if want_j[i] >= 64 else set())
        for j in range(k):
            x = int(xs[i, j])
            if j in evaluated and x < v:
                for key, ref in (("p_x", p_all[i][j, x]), ("q_x", q_all[i][j, x])):
                    assert abs(float(dbg[key][i, j]) - float(ref)) <= 1e-5 * float(ref) + 1e-30, (i, j, key)
            else:
                assert math.isnan(float(dbg["p_x"][i, j])) and math.isnan(float(dbg["q_x"][i, j])), (i, j)
        if want_j[i] < k:
            tot = float(torch.clamp(p_all[i][want_j[i]] - q_all[i][want_j[i]], min=0).sum())
            assert abs(float(dbg["res_sum"][i]) - tot) <= 1e-5 * tot, i
        else:
            assert float(dbg["res_sum"][i]) == 0.0


def test_spec_accept_vocab_past_32_chunks():
    """A vocabulary of 140,003 columns: 35 chunks of 4096, so the draw takes its chunks in two passes of
    32, and V is not a multiple of 8, so every row ends in a partial 16-byte group (the bounds-checked
    loads). f32, bf16 and f16 logits, statistics computed or given; one sequence's residual is planted in
    the last chunk and one's in the first, against the oracle."""
    case("spec_accept V=140003")
    g = torch.Generator().manual_seed(44)
    b, k, v = 4, 3, 140003
    tgt = torch.randn(b, k + 1, v, generator=g) * 2
    dft = tgt[:, :k] + torch.randn(b, k, v, generator=g)
    xs = torch.randint(0, v, (b, k), generator=g, dtype=torch.int32)
    u = torch.rand(b, k, generator=g)
    u[0, 0] = u[1, 0] = 1.0          # sequences 0 and 1 reject their first proposal
    tgt[0, 0, v - 5] = dft[0, 0, v - 5] + 20.0   # ... with the residual's mass in the last chunk
    tgt[1, 0, 3] = dft[1, 0, 3] + 20.0
    e = torch.empty(b, v).exponential_(generator=g)
    temps = torch.ones(b)
    for dtype in (torch.float32, torch.bfloat16, torch.float16):
        t_, d_ = tgt.to(dtype), dft.to(dtype)
        for mode in ("logits", "stats"):
            kw = {}
            if mode == "stats":
                rows = torch.cat([t_, d_], 1).float()
                mx = rows.max(-1).values
                kw["row_stats"] = _records(mx, torch.exp((rows - mx[..., None]).double()).sum(-1).float(),
                                           mx, rows.argmax(-1)).to(DEV)
            out, n = ops.spec_accept(t_.to(DEV), d_.to(DEV), xs.to(DEV), None, temps.to(DEV), u.to(DEV), e.to(DEV),
                                     **kw)
            out, n = out.cpu(), n.cpu()
            for i in range(b):
                p = orc.probs_from_logits(t_[i].float(), 1.0)
                q = orc.probs_from_logits(d_[i].float(), 1.0)
                acc, extra = orc.verify_with_noise(p, q, xs[i].tolist(), u[i], e[i])
                assert int(n[i]) == len(acc) and out[i, : len(acc) + 1].tolist() == acc + [extra], (dtype, mode, i)
            assert int(out[0, 0]) >= 32 * 4096 and int(out[1, 0]) < 4096, (dtype, mode)


def test_spec_accept_repeated_calls_on_a_dirty_workspace():
    """Back-to-back calls of different shapes and modes on the one workspace (statistics pass, given
    statistics, probabilities, greedy and sampled rows), each after the workspace was filled with 0xFF
    bytes, each give the oracle's outcome."""
    case("spec_accept repeated calls")
    g = torch.Generator().manual_seed(43)
    for b, k, v, temp in ((3, 2, 700, 1.0), (9, 5, 9000, 0.0), (2, 0, 513, 0.8), (64, 6, 20000, 1.0)):
        tgt = torch.randn(b, k + 1, v, generator=g) * 2
        dft = tgt[:, :k] + torch.randn(b, k, v, generator=g)
        xs = torch.randint(0, v, (b, k), generator=g, dtype=torch.int32)
        u = torch.rand(b, k, generator=g)
        e = torch.empty(b, v).exponential_(generator=g)
        temps = torch.full((b,), temp)
        for mode in ("logits", "stats"):
            _dirty_accept_workspace()
            kw = {}
            if mode == "stats":
                rows = torch.cat([tgt, dft], 1)
                y = rows / temp if temp > 0 else rows
                mx = y.max(-1).values
                kw["row_stats"] = _records(mx, torch.exp((y - mx[..., None]).double()).sum(-1).float(),
                                           rows.max(-1).values, rows.argmax(-1)).to(DEV)
            out, n = ops.spec_accept(tgt.to(DEV), dft.to(DEV), xs.to(DEV), None, temps.to(DEV), u.to(DEV), e.to(DEV),
                                     **kw)
            out, n = out.cpu(), n.cpu()
            for i in range(b):
                p = orc.probs_from_logits(tgt[i], temp)
                q = orc.probs_from_logits(dft[i], temp)
                acc, extra = orc.verify_with_noise(p, q, xs[i].tolist(), u[i], e[i])
                assert int(n[i]) == len(acc) and out[i, : len(acc) + 1].tolist() == acc + [extra], (b, k, mode, i)
        if k:
            _dirty_accept_workspace()
            pr = torch.softmax(tgt[0], -1)
            qr = torch.softmax(dft[0], -1)
            got = _verify_probs_case(pr, qr, xs[0].tolist(), u[0], e[0])
            want = orc.verify_with_noise(pr, qr, xs[0].tolist(), u[0], e[0])
            assert got == (want[0] + [want[1]], len(want[0]))


# ---- keyed random numbers (the speculative Engine's per-request streams) --------------------------------
def test_keyed_noise_matches_the_philox_stream():
    """Uniforms bit-exact and Exp(1) variates within a few ulps of the numpy restatement of the Philox
    stream, on strided rows and several slots; columns past n are not written; a row's values depend
    only on its key (the same with other rows beside it or alone)."""
    from oracle import keyed_noise as kn
    case("keyed noise")
    keys = torch.tensor([0, 1, 12345, (1 << 62) - 1, 987654321123], dtype=torch.int64)
    n = 1001
    for kind in (ops.RNG_UNIFORM, ops.RNG_EXP):
        buf = torch.full((3, 5, 1004), -1.0, device=DEV)
        ops.keyed_noise(keys.to(DEV), 7, buf[:, :, :n], kind)
        got = buf.cpu()
        assert (got[:, :, n:] == -1).all()
        for s in range(3):
            for b, key in enumerate(keys.tolist()):
                if kind == ops.RNG_UNIFORM:
                    assert np.array_equal(got[s, b, :n].numpy(), kn.uniform(key, 7 + s, n)), (s, b)
                else:
                    want = kn.exponential(key, 7 + s, n)
                    assert (np.abs(got[s, b, :n].numpy() - want) / want).max() < 5e-7, (s, b)
        alone = torch.empty(1, 1, n, device=DEV)
        ops.keyed_noise(keys[2:3].to(DEV), 8, alone, kind)
        assert torch.equal(alone[0, 0].cpu(), got[1, 2, :n])


def test_keyed_noise_distribution_at_vocab_size():
    """One 128256-column Exp(1) row per key for 64 keys (a round's final draws at the 8B shape): the
    pooled values follow Exp(1) (Kolmogorov-Smirnov), none is 0 or infinite."""
    from scipy import stats
    case("keyed noise distribution")
    keys = torch.arange(64, dtype=torch.int64).mul_(1_000_033).add_(17)
    e = ops.keyed_noise(keys.to(DEV), 1 << 20, torch.empty(64, 128256, device=DEV), ops.RNG_EXP).cpu().numpy()
    assert (e > 0).all() and np.isfinite(e).all()
    assert stats.kstest(e.reshape(-1)[::7], "expon").statistic < 2e-3
    u = ops.keyed_noise(keys.to(DEV), 5, torch.empty(64, 4096, device=DEV), ops.RNG_UNIFORM).cpu().numpy()
    assert u.min() >= 0 and u.max() < 1 and stats.kstest(u.reshape(-1), "uniform").statistic < 3e-3
