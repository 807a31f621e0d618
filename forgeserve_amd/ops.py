"""Tensor-level wrappers of the gfx950 kernels (C ABI in include/forgeserve_amd.h).

Each function checks shapes on the host, allocates outputs and workspace with torch's caching
allocator, and launches on torch's current stream. Inputs must already be on the GPU; nothing here
computes on the CPU.
"""

from typing import Optional, Tuple

import torch

from . import _lib
from ._lib import DTYPE_CODE, KVLayout, check, ptr, require_device, stream_ptr

I32 = torch.int32

def _dt(t: torch.Tensor) -> int:
    try:
        return DTYPE_CODE[t.dtype]
    except KeyError:
        raise ValueError(f"unsupported dtype {t.dtype} (float32, bfloat16, float16)") from None


def _ws(nbytes: int, device) -> torch.Tensor:
    return torch.empty(max(int(nbytes), 256), dtype=torch.uint8, device=device)


_PERSISTENT = {}
_RETIRED = []   # outgrown scratch buffers: a captured HIP graph may still hold their addresses


def _persistent_ws(name: str, nbytes: int, device) -> torch.Tensor:
    """A per-device scratch buffer reused across calls (calls are ordered on torch's current stream,
    so consecutive users never overlap); grown when a call needs more. An outgrown buffer is kept
    alive for the life of the process, since graphs captured earlier launch kernels on it."""
    key = (name, torch.device(device))
    ws = _PERSISTENT.get(key)
    if ws is None or ws.numel() < nbytes:
        if ws is not None:
            _RETIRED.append(ws)
        ws = torch.empty(max(int(nbytes * 1.25), 1 << 20), dtype=torch.uint8, device=key[1])
        _PERSISTENT[key] = ws
    return ws


def _rows(t: torch.Tensor) -> Tuple[int, int]:
    """(rows, row stride) of a 2-D tensor whose last dim is contiguous."""
    if t.dim() != 2 or (t.stride(1) != 1 and t.shape[1] > 1):
        raise ValueError(f"expected a 2-D tensor with a contiguous last dim, got {tuple(t.shape)} {t.stride()}")
    return t.shape[0], t.stride(0)


# ------------------------------------------------------------------------------------------------
# KV pool layout
# ------------------------------------------------------------------------------------------------
def kv_layout(k: torch.Tensor, v: torch.Tensor) -> KVLayout:
    """Layout of one layer: v is a (num_blocks, n_kv_heads, block_size, head_dim) view (any strides); k
    is the same, or (num_blocks, n_kv_heads, block_size, head_dim // 8, 8) with unit stride inside a
    group for keys stored as 8-dim groups (fs_kv_layout.k_group)."""
    if k.dim() == 5 and k.shape[-1] == 8 and k.stride(-1) == 1:
        kb, kh, ks, kg, _ = k.stride()
        k_strides, k_group, kshape = (kb, kh, ks, 1), kg, (*k.shape[:3], 8 * k.shape[3])
    elif k.dim() == 4:
        k_strides, k_group, kshape = k.stride(), 0, tuple(k.shape)
    else:
        raise ValueError(f"k pool view must be 4-D or grouped 5-D (..., head_dim // 8, 8): {tuple(k.shape)}")
    if kshape != tuple(v.shape) or v.dim() != 4 or k.dtype != v.dtype:
        raise ValueError(f"k/v pool views must match: {tuple(k.shape)} vs {tuple(v.shape)}")
    nb, h, bs, d = v.shape
    return KVLayout(k.data_ptr(), v.data_ptr(), *k_strides, *v.stride(), bs, h, d, _dt(k), nb, k_group)


# ------------------------------------------------------------------------------------------------
# dense ops
# ------------------------------------------------------------------------------------------------
def gemm(a: torch.Tensor, w: torch.Tensor, out: Optional[torch.Tensor] = None,
         residual: Optional[torch.Tensor] = None) -> torch.Tensor:
    """out = a @ w.T (+ residual): nn.Linear (model.py:57-60, 88-90, 119) with the residual add fused."""
    require_device(a, w)
    m, lda = _rows(a)
    n, ldb = _rows(w)
    k = a.shape[1]
    if w.shape[1] != k or a.dtype != w.dtype:
        raise ValueError(f"gemm: {tuple(a.shape)} {a.dtype} x {tuple(w.shape)} {w.dtype}")
    if out is None:
        out = torch.empty((m, n), dtype=a.dtype, device=a.device)
    _, ldc = _rows(out)
    ldr = 0
    if residual is not None:
        _, ldr = _rows(residual)
        if residual.shape != out.shape or residual.dtype != a.dtype:
            raise ValueError("gemm: residual shape/dtype")
    lib = _lib.load()
    need = lib.fs_gemm_workspace_size(m, n, k, _dt(a))
    ws = _persistent_ws("gemm", need, a.device) if need > 0 else None
    check(lib.fs_gemm(ptr(a), lda, ptr(w), ldb, ptr(out), ldc, ptr(residual), ldr, m, n, k, _dt(a), ptr(ws),
                      ws.numel() if ws is not None else 0, stream_ptr()), "gemm")
    return out


def gemm_add_rmsnorm(a: torch.Tensor, w: torch.Tensor, residual: torch.Tensor, norm_weight: torch.Tensor,
                     eps: float, x_out: Optional[torch.Tensor] = None) -> Tuple[torch.Tensor, torch.Tensor]:
    """x = a @ w.T + residual (nn.Linear then the residual add, model.py:105-106) and y = RMSNorm(x)
    with norm_weight (model.py:29-31): returns (x, y). When the GEMM splits K into partials, they are
    added by the norm kernel itself (no separate reduction pass); otherwise (no split, or a long batch
    whose workgroups run the splits one after the other) the GEMM adds the residual and the norm runs
    on its output. The results are the same either way. x_out: an (m, n) tensor with unit column stride
    that receives x (returned as x)."""
    require_device(a, w, residual, norm_weight)
    m, lda = _rows(a)
    n, ldb = _rows(w)
    k = a.shape[1]
    lib = _lib.load()
    if (a.dtype in (torch.bfloat16,) and w.dtype == a.dtype and w.shape[1] == k and residual.shape == (m, n)
            and residual.dtype == a.dtype and n % 8 == 0 and n <= 8192 and lib.fs_gemm_splits(n, k, _dt(a)) > 1
            and not lib.fs_gemm_serial(m, n, k, _dt(a))
            and k % 64 == 0 and lda % 8 == 0 and ldb % 8 == 0 and residual.stride(1) == 1
            and residual.stride(0) % 8 == 0 and norm_weight.is_contiguous() and norm_weight.dtype == a.dtype):
        splits = lib.fs_gemm_splits(n, k, _dt(a))
        need = splits * m * n * 4
        ws = _persistent_ws("gemm", need, a.device)
        check(lib.fs_gemm_partials(ptr(a), lda, ptr(w), ldb, m, n, k, _dt(a), ptr(ws), ws.numel(), stream_ptr()),
              "gemm_partials")
        direct = (x_out is not None and x_out.shape == (m, n) and x_out.dtype == a.dtype and x_out.stride(1) == 1
                  and x_out.stride(0) % 8 == 0 and x_out.data_ptr() % 16 == 0)
        x = x_out if direct else torch.empty((m, n), dtype=a.dtype, device=a.device)
        y = torch.empty((m, n), dtype=a.dtype, device=a.device)
        check(lib.fs_splitk_add_rmsnorm(ptr(ws), splits, ptr(residual), residual.stride(0), ptr(x), x.stride(0),
                                        ptr(norm_weight), ptr(y), n, m, n, float(eps), _dt(a), stream_ptr()),
              "splitk_add_rmsnorm")
        if x_out is not None and not direct:
            x = x_out.copy_(x)
        return x, y
    x = gemm(a, w, residual=residual)
    y = add_rmsnorm(x, norm_weight, eps)
    return (x if x_out is None else x_out.copy_(x)), y


def row_stats_parts(m: int, n: int, k: int) -> int:
    """Column blocks per row of gemm_row_stats at this shape (0: the shape has no statistics epilogue)."""
    return int(_lib.load().fs_gemm_row_stats_parts(m, n, k))


def gemm_row_stats(a: torch.Tensor, w: torch.Tensor, temperature: Optional[torch.Tensor],
                   stats: torch.Tensor, out: Optional[torch.Tensor] = None) -> torch.Tensor:
    """out = a @ w.T (the LM head, model.py:137-138) and, per row and column block, the softmax
    statistics of the stored logits x at y = x / temperature[row] (a true division, sampling.py:13;
    rows at T = 0 keep only a meaningful argmax). stats: int32
    (M, nparts, 4) records (max, sum, argmax value as float bits, argmax index); rows may be strided."""
    require_device(a, w, stats)
    m, lda = _rows(a)
    n, ldb = _rows(w)
    k = a.shape[1]
    if w.shape[1] != k or a.dtype != w.dtype or a.dtype != torch.bfloat16:
        raise ValueError(f"gemm_row_stats: bf16 {tuple(a.shape)} x {tuple(w.shape)}")
    nparts = row_stats_parts(m, n, k)
    if (stats.dtype != I32 or tuple(stats.shape) != (m, nparts, 4) or stats.stride(2) != 1 or stats.stride(1) != 4
            or stats.stride(0) % 4):
        raise ValueError(f"gemm_row_stats: stats must be int32 ({m}, {nparts}, 4) with whole records per row")
    if temperature is not None and (temperature.dtype != torch.float32 or temperature.shape != (m,)):
        raise ValueError("gemm_row_stats: temperature must be float32 (M,)")
    if out is None:
        out = torch.empty((m, n), dtype=a.dtype, device=a.device)
    _, ldc = _rows(out)
    check(_lib.load().fs_gemm_row_stats(ptr(a), lda, ptr(w), ldb, ptr(out), ldc, m, n, k, ptr(temperature),
                                        ptr(stats), stats.stride(0) // 4, nparts, stream_ptr()), "gemm_row_stats")
    return out


def row_stats_merge(parts: torch.Tensor, out: torch.Tensor, group: int = 1, gstride: int = 1,
                    offset: int = 0) -> torch.Tensor:
    """Merge gemm_row_stats' (M, nparts, 4) records into one per row: row m goes to record
    (m // group) * gstride + m % group + offset of out (int32 (..., 4), contiguous)."""
    require_device(parts, out)
    m, nparts, _ = parts.shape
    if parts.dtype != I32 or out.dtype != I32 or out.shape[-1] != 4 or not out.is_contiguous():
        raise ValueError("row_stats_merge: int32 records of 4")
    if parts.stride(2) != 1 or parts.stride(1) != 4 or parts.stride(0) % 4:
        raise ValueError("row_stats_merge: parts must hold whole records per row")
    last = ((m - 1) // group) * gstride + (m - 1) % group + offset if m else 0
    if last >= out.numel() // 4:
        raise ValueError("row_stats_merge: out is too small for the row mapping")
    check(_lib.load().fs_row_stats_merge(ptr(parts), parts.stride(0) // 4, nparts, m, ptr(out), group, gstride, offset,
                                         stream_ptr()), "row_stats_merge")
    return out


def add_rmsnorm(x: torch.Tensor, weight: torch.Tensor, eps: float, delta: Optional[torch.Tensor] = None,
                x_out: Optional[torch.Tensor] = None, y: Optional[torch.Tensor] = None) -> torch.Tensor:
    """y = RMSNorm(x [+ delta]) (model.py:29-31); with delta, x + delta is also written to x_out."""
    require_device(x, weight)
    m, ldx = _rows(x)
    n = x.shape[1]
    if weight.shape != (n,) or weight.dtype != x.dtype:
        raise ValueError("add_rmsnorm: weight shape/dtype")
    ldd = ldxo = 0
    if delta is not None:
        _, ldd = _rows(delta)
        if x_out is None:
            raise ValueError("add_rmsnorm: delta needs x_out")
        _, ldxo = _rows(x_out)
    if y is None:
        y = torch.empty((m, n), dtype=x.dtype, device=x.device)
    _, ldy = _rows(y)
    check(_lib.load().fs_add_rmsnorm(ptr(x), ldx, ptr(delta), ldd, ptr(x_out), ldxo, ptr(weight), ptr(y), ldy, m, n,
                                     float(eps), _dt(x), stream_ptr()), "add_rmsnorm")
    return y


def gemm_swiglu(a: torch.Tensor, w: torch.Tensor) -> torch.Tensor:
    """silu_mul(gemm(a, w)) for w the [gate; up] weight (2F, K): h (M, F) = silu(a w_gate^T) * (a w_up^T)
    (model.py:93). One kernel when the shape allows it (bf16, no K split), else the two; the results
    are the same either way."""
    require_device(a, w)
    m, lda = _rows(a)
    n2, ldb = _rows(w)
    k = a.shape[1]
    f = n2 // 2
    lib = _lib.load()
    if (a.dtype == torch.bfloat16 and w.dtype == a.dtype and w.shape[1] == k and n2 % 4 == 0 and k % 64 == 0
            and lda % 8 == 0 and ldb % 8 == 0 and lib.fs_gemm_splits(n2, k, _dt(a)) == 1):
        h = torch.empty((m, f), dtype=a.dtype, device=a.device)
        check(lib.fs_gemm_swiglu(ptr(a), lda, ptr(w), ldb, ptr(h), f, m, f, k, _dt(a), stream_ptr()), "gemm_swiglu")
        return h
    return silu_mul(gemm(a, w))


def silu_mul(gu: torch.Tensor, out: Optional[torch.Tensor] = None) -> torch.Tensor:
    """silu(gu[:, :F]) * gu[:, F:] (model.py:93)."""
    require_device(gu)
    m, ld = _rows(gu)
    f = gu.shape[1] // 2
    if out is None:
        out = torch.empty((m, f), dtype=gu.dtype, device=gu.device)
    _, ldh = _rows(out)
    check(_lib.load().fs_silu_mul(ptr(gu), ld, ptr(out), ldh, m, f, _dt(gu), stream_ptr()), "silu_mul")
    return out


def embedding(ids: torch.Tensor, weight: torch.Tensor, out: Optional[torch.Tensor] = None) -> torch.Tensor:
    """weight[ids] for int64 ids of any shape -> (ids.numel(), d) (model.py:134-135)."""
    require_device(ids, weight)
    ids = ids.reshape(-1)
    if ids.dtype != torch.int64:
        ids = ids.long()
    ids = ids.contiguous()
    vocab, d = weight.shape
    if out is None:
        out = torch.empty((ids.numel(), d), dtype=weight.dtype, device=weight.device)
    _, ldo = _rows(out)
    check(_lib.load().fs_embedding(ptr(ids), ids.numel(), ptr(weight.contiguous()), d, vocab, ptr(out), ldo,
                                   _dt(weight), stream_ptr()), "embedding")
    return out


# ------------------------------------------------------------------------------------------------
# KV cache + attention
# ------------------------------------------------------------------------------------------------
def qkv_rope_write(qkv: torch.Tensor, positions: torch.Tensor, T: int, n_heads: int, rope_cos: torch.Tensor,
                   rope_sin: torch.Tensor, tables: torch.Tensor, layout: KVLayout,
                   slots: Optional[torch.Tensor] = None, q_out: Optional[torch.Tensor] = None) -> torch.Tensor:
    """Rotate q and k (model.py:40-45, 67) and write k, v into the pool (paged.py:74-78).

    qkv: (B*T, (n_heads + 2*n_kv_heads) * head_dim); positions/slots: int32 (B*T,);
    tables: int32 (B, max_blocks). Returns the rotated queries (B*T, n_heads * head_dim)."""
    require_device(qkv, positions, tables)
    m, ld = _rows(qkv)
    d = layout.head_dim
    if q_out is None:
        q_out = torch.empty((m, n_heads * d), dtype=qkv.dtype, device=qkv.device)
    _, ldq = _rows(q_out)
    if positions.dtype != I32 or tables.dtype != I32 or (slots is not None and slots.dtype != I32):
        raise ValueError("qkv_rope_write: positions, slots and tables must be int32")
    check(_lib.load().fs_qkv_rope_write(ptr(qkv), ld, m, T, n_heads, ptr(positions), ptr(slots), ptr(rope_cos),
                                        ptr(rope_sin), rope_cos.shape[0], ptr(tables), tables.stride(0),
                                        tables.shape[1], layout, ptr(q_out), ldq, stream_ptr()), "qkv_rope_write")
    return q_out


def qkv_rope_gemm(h: torch.Tensor, w: torch.Tensor, positions: torch.Tensor, T: int, n_heads: int,
                  rope_cos: torch.Tensor, rope_sin: torch.Tensor, tables: torch.Tensor, layout: KVLayout,
                  slots: Optional[torch.Tensor] = None) -> torch.Tensor:
    """qkv_rope_write(gemm(h, w), ...): the fused QKV projection (model.py:57-60, 64-66) followed by the
    rotary + pool write. When the projection splits K into partials, the rotary kernel adds them itself
    (no separate reduction pass); the results are the same either way."""
    require_device(h, w, positions, tables)
    m, lda = _rows(h)
    n, ldb = _rows(w)
    k = h.shape[1]
    lib = _lib.load()
    d = layout.head_dim
    if (h.dtype == torch.bfloat16 and w.dtype == h.dtype and w.shape[1] == k and layout.dtype == _dt(h)
            and k % 64 == 0 and lda % 8 == 0 and ldb % 8 == 0 and n % 8 == 0 and (d // 2) % 8 == 0
            and lib.fs_gemm_splits(n, k, _dt(h)) > 1 and not lib.fs_gemm_serial(m, n, k, _dt(h))
            and positions.dtype == I32 and tables.dtype == I32
            and (slots is None or slots.dtype == I32)):
        splits = lib.fs_gemm_splits(n, k, _dt(h))
        ws = _persistent_ws("gemm", splits * m * n * 4, h.device)
        check(lib.fs_gemm_partials(ptr(h), lda, ptr(w), ldb, m, n, k, _dt(h), ptr(ws), ws.numel(), stream_ptr()),
              "gemm_partials")
        q_out = torch.empty((m, n_heads * d), dtype=h.dtype, device=h.device)
        check(lib.fs_qkv_rope_write_partials(ptr(ws), splits, m, n, T, n_heads, ptr(positions), ptr(slots),
                                             ptr(rope_cos), ptr(rope_sin), rope_cos.shape[0], ptr(tables),
                                             tables.stride(0), tables.shape[1], layout, ptr(q_out), q_out.stride(0),
                                             stream_ptr()), "qkv_rope_write_partials")
        return q_out
    return qkv_rope_write(gemm(h, w), positions, T, n_heads, rope_cos, rope_sin, tables, layout, slots=slots)


def qkv_rope_write_varlen(qkv: torch.Tensor, positions: torch.Tensor, token_row: torch.Tensor, n_heads: int,
                          rope_cos: torch.Tensor, rope_sin: torch.Tensor, tables: torch.Tensor, layout: KVLayout,
                          q_out: Optional[torch.Tensor] = None) -> torch.Tensor:
    """qkv_rope_write for packed sequences: token m writes through table row token_row[m].

    qkv: (n_tokens, (n_heads + 2*n_kv_heads) * head_dim); positions, token_row: int32 (n_tokens,);
    tables: int32 (rows, max_blocks). Returns the rotated queries (n_tokens, n_heads * head_dim)."""
    require_device(qkv, positions, token_row, tables)
    m, ld = _rows(qkv)
    d = layout.head_dim
    if positions.dtype != I32 or token_row.dtype != I32 or tables.dtype != I32:
        raise ValueError("qkv_rope_write_varlen: positions, token_row and tables must be int32")
    if positions.numel() != m or token_row.numel() != m:
        raise ValueError("qkv_rope_write_varlen: one position and one table row per token")
    if q_out is None:
        q_out = torch.empty((m, n_heads * d), dtype=qkv.dtype, device=qkv.device)
    _, ldq = _rows(q_out)
    check(_lib.load().fs_qkv_rope_write_varlen(ptr(qkv), ld, m, n_heads, ptr(positions.contiguous()),
                                               ptr(token_row.contiguous()), tables.shape[0], ptr(rope_cos),
                                               ptr(rope_sin), rope_cos.shape[0], ptr(tables), tables.stride(0),
                                               tables.shape[1], layout, ptr(q_out), ldq, stream_ptr()),
          "qkv_rope_write_varlen")
    return q_out


def paged_kv_write(k: torch.Tensor, v: torch.Tensor, positions: torch.Tensor, tables: torch.Tensor,
                   layout: KVLayout) -> None:
    """Scatter k, v (B, n_kv_heads, T, head_dim) to the pool slots of positions (B, T) (paged.py:74-78)."""
    require_device(k, v, positions, tables)
    if k.shape != v.shape or k.stride() != v.stride() or k.stride(3) != 1:
        raise ValueError("paged_kv_write: k and v must share shape and strides, head_dim contiguous")
    b, h, t, d = k.shape
    if positions.dtype != I32 or tables.dtype != I32:
        raise ValueError("paged_kv_write: positions and tables must be int32")
    check(_lib.load().fs_paged_kv_write(ptr(k), ptr(v), k.stride(0), k.stride(1), k.stride(2), b, t,
                                        ptr(positions.contiguous()), ptr(tables), tables.stride(0), tables.shape[1],
                                        layout, stream_ptr()), "paged_kv_write")


def paged_gather(layout: KVLayout, tables: torch.Tensor, dtype, device) -> Tuple[torch.Tensor, torch.Tensor]:
    """Every block of every table row, in table order: (B, n_kv_heads, max_blocks*block_size, head_dim)."""
    b, nb = tables.shape
    shape = (b, layout.n_kv_heads, nb * layout.block_size, layout.head_dim)
    k_all = torch.empty(shape, dtype=dtype, device=device)
    v_all = torch.empty(shape, dtype=dtype, device=device)
    check(_lib.load().fs_paged_gather(layout, ptr(tables), tables.stride(0), b, nb, ptr(k_all), ptr(v_all),
                                      stream_ptr()), "paged_gather")
    return k_all, v_all


# The plan key and positions tensor of the last paged-attention call (held, so that no later object
# can share their identities).
_PLAN_KEY = [None, None]


def _reuse_plan(plan_key, positions: torch.Tensor) -> bool:
    """True when the previous paged-attention call carried the same plan key and the same positions
    tensor (the layers of one step)."""
    reuse = plan_key is not None and _PLAN_KEY[0] is plan_key and _PLAN_KEY[1] is positions
    _PLAN_KEY[0], _PLAN_KEY[1] = plan_key, positions
    return reuse


def paged_attention(q: torch.Tensor, layout: KVLayout, tables: torch.Tensor, positions: torch.Tensor,
                    scale: float, out: Optional[torch.Tensor] = None, plan_key=None) -> torch.Tensor:
    """Causal GQA attention of q (B, T, n_heads, head_dim) over the paged keys (model.py:70-76).

    positions: int32 (B, T); query (b, t) sees the keys at positions 0..positions[b, t].
    plan_key: an object that stands for these positions (the forward step): consecutive calls with the
    same key reuse the work plan of the first (the positions must not change between them)."""
    require_device(q, tables, positions)
    b, t, h, d = q.shape
    if q.stride(3) != 1:
        raise ValueError("paged_attention: head_dim must be contiguous")
    if positions.dtype != I32 or tables.dtype != I32 or positions.shape != (b, t):
        raise ValueError("paged_attention: positions (B, T) and tables must be int32")
    positions = positions.contiguous()
    if out is None:
        out = torch.empty((b, t, h, d), dtype=q.dtype, device=q.device)
    nb = tables.shape[1]
    lib = _lib.load()
    need = lib.fs_paged_attention_workspace_size(b, t, h, d, nb, layout.block_size)
    ws = _persistent_ws("attention", need, q.device)
    fn = lib.fs_paged_attention_reuse_plan if _reuse_plan(plan_key, positions) else lib.fs_paged_attention
    check(fn(ptr(q), q.stride(0), q.stride(1), q.stride(2), layout, ptr(tables), tables.stride(0), nb, ptr(positions),
             b, t, h, float(scale), ptr(out), out.stride(0), out.stride(1), out.stride(2), ptr(ws), ws.numel(),
             stream_ptr()), "paged_attention")
    return out


def paged_attention_varlen(q: torch.Tensor, layout: KVLayout, tables: torch.Tensor, positions: torch.Tensor,
                           cu_seqlens: torch.Tensor, scale: float, out: Optional[torch.Tensor] = None,
                           plan_key=None) -> torch.Tensor:
    """paged_attention over packed sequences: q (n_tokens, n_heads, head_dim); sequence s owns tokens
    cu_seqlens[s] .. cu_seqlens[s+1]-1 (int32 (S+1,), on the device; the caller guarantees the bounds:
    cu_seqlens[S] <= n_tokens and no sequence longer than T); positions int32 (S, T), -1 past a
    sequence's tokens; tables int32 (S, max_blocks). Returns out (n_tokens, n_heads, head_dim).
    plan_key: as for paged_attention."""
    require_device(q, tables, positions, cu_seqlens)
    n, h, d = q.shape
    if q.stride(2) != 1:
        raise ValueError("paged_attention_varlen: head_dim must be contiguous")
    s, t = positions.shape
    if (positions.dtype != I32 or tables.dtype != I32 or cu_seqlens.dtype != I32 or cu_seqlens.numel() != s + 1
            or tables.shape[0] != s):
        raise ValueError("paged_attention_varlen: positions (S, T), tables (S, .) and cu_seqlens (S+1,) int32")
    positions = positions.contiguous()
    if out is None:
        out = torch.empty((n, h, d), dtype=q.dtype, device=q.device)
    nb = tables.shape[1]
    lib = _lib.load()
    ws = _persistent_ws("attention", lib.fs_paged_attention_workspace_size(s, t, h, d, nb, layout.block_size), q.device)
    fn = (lib.fs_paged_attention_varlen_reuse_plan if _reuse_plan(plan_key, positions)
          else lib.fs_paged_attention_varlen)
    check(fn(ptr(q), q.stride(0), q.stride(1), layout, ptr(tables), tables.stride(0), nb, ptr(positions),
             ptr(cu_seqlens.contiguous()), s, t, h, float(scale), ptr(out), out.stride(0), out.stride(1), ptr(ws),
             ws.numel(), stream_ptr()), "paged_attention_varlen")
    return out


# ------------------------------------------------------------------------------------------------
# sampling / acceptance
# ------------------------------------------------------------------------------------------------
def probs_from_logits(logits: torch.Tensor, temperature: float) -> torch.Tensor:
    """softmax(f32(logits) / T), or the one-hot of the argmax in the logits dtype at T == 0 (sampling.py:9-13)."""
    require_device(logits)
    shape = logits.shape
    x = logits.reshape(-1, shape[-1])
    if x.stride(1) != 1:
        x = x.contiguous()
    r, ld = x.shape[0], x.stride(0)
    v = shape[-1]
    out_dtype = torch.float32 if temperature > 0 else logits.dtype
    out = torch.empty((r, v), dtype=out_dtype, device=logits.device)
    lib = _lib.load()
    ws = _ws(lib.fs_sampling_workspace_size(r, v), logits.device)
    check(lib.fs_probs_from_logits(ptr(x), ld, r, v, float(temperature), _dt(x), ptr(out), v, DTYPE_CODE[out_dtype],
                                   ptr(ws), ws.numel(), stream_ptr()), "probs_from_logits")
    return out.reshape(shape)


def sample_logits(logits: torch.Tensor, temperature, noise: Optional[torch.Tensor] = None,
                  out32: Optional[torch.Tensor] = None, out64: Optional[torch.Tensor] = None) -> torch.Tensor:
    """Token ids (int64, logits.shape[:-1]) for logits (..., V) (sampling.py:16-21).

    temperature: a float for every row, or a float32 device tensor with one value per row.
    noise: float32 Exp(1) noise with the logits' shape (the categorical draw is argmax(p / noise));
    None makes every row greedy. out32: optional int32 view that also receives the tokens; out64: an
    optional contiguous int64 tensor of one element per row that receives them as the result does (and
    is returned, reshaped)."""
    require_device(logits)
    shape = logits.shape
    x = logits.reshape(-1, shape[-1])
    if x.stride(1) != 1:
        x = x.contiguous()
    r, ld = x.shape[0], x.stride(0)
    v = shape[-1]
    if out64 is not None and (out64.dtype != torch.int64 or out64.numel() != r or not out64.is_contiguous()):
        raise ValueError("sample_logits: out64 must be a contiguous int64 tensor of one element per row")
    tok = out64.view(-1) if out64 is not None else torch.empty((r,), dtype=torch.int64, device=logits.device)
    t_ptr, t_all = 0, 0.0
    if isinstance(temperature, torch.Tensor):
        require_device(temperature)
        temperature = temperature.to(torch.float32).reshape(-1).contiguous()
        if temperature.numel() != r:
            raise ValueError("sample_logits: one temperature per row")
        t_ptr = ptr(temperature)
    else:
        t_all = float(temperature)
        if t_all < 0:
            raise ValueError("temperature must be >= 0")
    e_ptr, lde = 0, 0
    if noise is not None:
        require_device(noise)
        noise = noise.reshape(-1, v)
        if noise.dtype != torch.float32 or noise.shape[0] != r or noise.stride(1) != 1:
            raise ValueError("sample_logits: noise must be float32 with the logits' shape")
        e_ptr, lde = ptr(noise), noise.stride(0)
    o32, ld32 = 0, 0
    if out32 is not None:
        o32, ld32 = ptr(out32), out32.stride(0) if out32.dim() else 1
    lib = _lib.load()
    ws = _ws(lib.fs_sampling_workspace_size(r, v), logits.device)
    check(lib.fs_sample_logits(ptr(x), ld, r, v, t_ptr, t_all, e_ptr, lde, _dt(x), ptr(tok), o32, ld32, ptr(ws),
                               ws.numel(), stream_ptr()), "sample_logits")
    return tok.reshape(shape[:-1])


def spec_accept(tgt: torch.Tensor, dft: torch.Tensor, draft_tokens: torch.Tensor, k_eff: Optional[torch.Tensor],
                temperature: torch.Tensor, u: torch.Tensor, noise: torch.Tensor,
                seq_len: Optional[torch.Tensor] = None, out_tokens: Optional[torch.Tensor] = None,
                n_accepted: Optional[torch.Tensor] = None,
                row_stats: Optional[torch.Tensor] = None, debug: bool = False):
    """Batched verify_draft from logits (speculative.py:20-33, sampling.py:9-13).

    tgt (B, K+1, V), dft (B, K, V) logits; draft_tokens int32 (B, K); k_eff int32 (B,) or None (= K);
    temperature float32 (B,); u float32 (B, K) uniforms; noise float32 (B, V) Exp(1);
    seq_len int32 (B,) cached lengths, advanced in place by 1 + n_accepted;
    row_stats: int32 (B, 2K+1, 4) softmax statistics of the rows (row_stats_merge of the LM heads'
    gemm_row_stats at the temperatures), which skips the statistics pass.
    Returns out_tokens int32 (B, K+1) (accepted, extra, then -1) and n_accepted int32 (B,); with debug,
    also {"p_x", "q_x": float32 (B, K), p_i(x_i) and q_i(x_i) of the proposals i < k_eff (NaN past it),
    "res_sum": float32 (B,), the residual sum at the first rejection (0: none)}."""
    require_device(tgt, dft, draft_tokens, temperature, u, noise)
    b, k1, v = tgt.shape
    k = k1 - 1
    if dft.shape != (b, k, v) or dft.dtype != tgt.dtype:
        raise ValueError(f"spec_accept: draft logits {tuple(dft.shape)} vs target {tuple(tgt.shape)}")
    if tgt.stride(2) != 1 or dft.stride(2) != 1:
        raise ValueError("spec_accept: vocab dim must be contiguous")
    for name, t, dt, shp in (("draft_tokens", draft_tokens, I32, (b, k)), ("temperature", temperature,
                             torch.float32, (b,)), ("u", u, torch.float32, (b, k)), ("noise", noise, torch.float32,
                             (b, v))):
        if t.dtype != dt or tuple(t.shape) != shp or not t.is_contiguous():
            raise ValueError(f"spec_accept: {name} must be contiguous {dt} {shp}")
    if k_eff is not None and (k_eff.dtype != I32 or k_eff.shape != (b,)):
        raise ValueError("spec_accept: k_eff must be int32 (B,)")
    if out_tokens is None:
        out_tokens = torch.empty((b, k + 1), dtype=I32, device=tgt.device)
    if n_accepted is None:
        n_accepted = torch.empty((b,), dtype=I32, device=tgt.device)
    lib = _lib.load()
    ws = _persistent_ws("accept", lib.fs_spec_accept_workspace_size(b, k, v), tgt.device)
    dbg = None
    if debug:
        dbg = {"p_x": torch.full((b, k), float("nan"), dtype=torch.float32, device=tgt.device),
               "q_x": torch.full((b, k), float("nan"), dtype=torch.float32, device=tgt.device),
               "res_sum": torch.zeros((b,), dtype=torch.float32, device=tgt.device)}
    px, qx, rs = (ptr(dbg["p_x"]), ptr(dbg["q_x"]), ptr(dbg["res_sum"])) if dbg else (0, 0, 0)
    if row_stats is not None:
        if row_stats.dtype != I32 or tuple(row_stats.shape) != (b, 2 * k + 1, 4) or not row_stats.is_contiguous():
            raise ValueError(f"spec_accept: row_stats must be contiguous int32 ({b}, {2 * k + 1}, 4)")
        require_device(row_stats)
        check(lib.fs_spec_accept_stats(ptr(tgt), tgt.stride(0), tgt.stride(1), ptr(dft), dft.stride(0),
                                       dft.stride(1) if k else 0, b, k, v, _dt(tgt), ptr(draft_tokens), ptr(k_eff),
                                       ptr(temperature), ptr(u), ptr(noise), noise.stride(0), ptr(row_stats),
                                       ptr(out_tokens), ptr(n_accepted), ptr(seq_len), px, qx, rs, ptr(ws),
                                       ws.numel(), stream_ptr()), "spec_accept")
    else:
        check(lib.fs_spec_accept(ptr(tgt), tgt.stride(0), tgt.stride(1), ptr(dft), dft.stride(0),
                                 dft.stride(1) if k else 0, b, k, v, _dt(tgt), ptr(draft_tokens), ptr(k_eff),
                                 ptr(temperature), ptr(u), ptr(noise), noise.stride(0), ptr(out_tokens),
                                 ptr(n_accepted), ptr(seq_len), px, qx, rs, ptr(ws), ws.numel(), stream_ptr()),
              "spec_accept")
    return (out_tokens, n_accepted, dbg) if debug else (out_tokens, n_accepted)


def verify_probs(p: torch.Tensor, q: torch.Tensor, draft_tokens: torch.Tensor, u: torch.Tensor,
                 noise: torch.Tensor) -> Tuple[torch.Tensor, torch.Tensor]:
    """verify_draft on probability rows p (K+1, V), q (K, V) (speculative.py:20-33)."""
    require_device(p, q, draft_tokens, u, noise)
    k1, v = p.shape
    k = k1 - 1
    if q.shape != (k, v) or q.dtype != p.dtype or p.stride(1) != 1 or (k and q.stride(1) != 1):
        raise ValueError("verify_probs: p (K+1, V) and q (K, V) of one dtype, contiguous rows")
    if draft_tokens.dtype != I32 or draft_tokens.numel() != k or u.numel() != k or noise.numel() != v:
        raise ValueError("verify_probs: draft_tokens int32 (K,), u (K,), noise (V,)")
    out = torch.empty((k + 1,), dtype=I32, device=p.device)
    n = torch.empty((1,), dtype=I32, device=p.device)
    lib = _lib.load()
    ws = _persistent_ws("accept", lib.fs_spec_accept_workspace_size(1, k, v), p.device)
    check(lib.fs_verify_probs(ptr(p), p.stride(0), ptr(q), q.stride(0) if k else 0, k, v, _dt(p),
                              ptr(draft_tokens.contiguous()), ptr(u.contiguous()), ptr(noise.contiguous()), ptr(out),
                              ptr(n), ptr(ws), ws.numel(), stream_ptr()), "verify_probs")
    return out, n


def spec_advance(res: torch.Tensor, b: int, k: int, first: int, n: torch.Tensor, budget: torch.Tensor,
                 eos: torch.Tensor, done: torch.Tensor, ids: torch.Tensor, last: torch.Tensor, keff: torch.Tensor,
                 pos0: torch.Tensor, posd: torch.Tensor, posv: torch.Tensor) -> None:
    """The next round's inputs from this round's acceptance, in place on the device (the bookkeeping
    of speculative.py:71-85 for b rows): res (b, k+2) int32 from the acceptance; n, budget, eos, done
    int32 (b,); ids int64 (b, 2); last int64 (b,); keff int32 (b,); pos0 int32 (b, 2); posd int32
    (k - first, b); posv int32 (b, k+1)."""
    require_device(res, n, budget, eos, done, ids, last, keff, pos0, posv)
    i32 = (res, n, budget, eos, done, keff, pos0, posd, posv)
    if any(t.dtype != I32 or not t.is_contiguous() for t in i32) or ids.dtype != torch.int64 or last.dtype != torch.int64:
        raise ValueError("spec_advance: int32 rows and positions, int64 ids, contiguous")
    shapes_ok = (res.shape[0] >= b and res.shape[1] >= k + 2 and n.numel() >= b and ids.shape == (b, 2)
                 and posv.shape == (b, k + 1) and pos0.shape == (b, 2) and (k <= first or posd.shape == (k - first, b)))
    if not shapes_ok:
        raise ValueError("spec_advance: shapes")
    check(_lib.load().fs_spec_advance(ptr(res), res.stride(0), b, k, first, ptr(n), ptr(budget), ptr(eos), ptr(done),
                                      ptr(ids), ptr(last), ptr(keff), ptr(pos0), ptr(posd), ptr(posv), stream_ptr()),
          "spec_advance")


RNG_UNIFORM, RNG_EXP = 0, 1


def keyed_noise(keys: torch.Tensor, slot0: int, out: torch.Tensor, kind: int) -> torch.Tensor:
    """Counter-based draws keyed per row: out (n_slots, B, n) or (B, n) float32 (last dim contiguous)
    receives, for slot s and row b, the variates of (keys[b], slot0 + s, column j): uniforms in
    [0, 1) (kind RNG_UNIFORM) or Exp(1) (RNG_EXP). keys: int64 (B,) on the device."""
    require_device(keys, out)
    if keys.dtype != torch.int64 or keys.dim() != 1 or not keys.is_contiguous():
        raise ValueError("keyed_noise: keys must be a contiguous int64 (B,) tensor")
    o = out if out.dim() == 3 else out.unsqueeze(0)
    s, b, n = o.shape
    if o.dtype != torch.float32 or (n > 1 and o.stride(2) != 1) or b != keys.numel():
        raise ValueError("keyed_noise: out must be float32 (n_slots, B, n) with B = len(keys), last dim contiguous")
    check(_lib.load().fs_keyed_noise(ptr(keys), b, slot0, s, n, kind, ptr(o), o.stride(1), o.stride(0), stream_ptr()),
          "keyed_noise")
    return out
