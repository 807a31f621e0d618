// Paged KV cache kernels: fused rotary + KV write, plain KV write, and the compatibility gather.
//
// Reference: paged.py:71-82 (PagedLayerView.update) and model.py:40-45 (apply_rope).
// Pool layout is described by fs_kv_layout; one (block, kv-head) tile of keys is block_size*head_dim
// contiguous elements (slot-major, or as 8-dim groups of every slot), and values are stored dim-major
// so the attention kernel reads 16 keys of one dim as one contiguous run.
#include "common.h"

namespace {

// Rotary half-split rotation of one pair (x[i], x[i + D/2]) at table row `pos`, in dtype DT:
//   out[i]       = x1*c - x2*s,   out[i + D/2] = x2*c + x1*s        (model.py:44-45)
// with c, s rounded to DT first (model.py:42-43) and every product and sum rounded to DT.
template <int DT>
FS_DEVICE void rope_pair(float x1, float x2, float c, float s, float& o1, float& o2) {
  typedef Elem<DT> E;
  c = E::round(c);
  s = E::round(s);
  float a = E::round(x1 * c), b = E::round(x2 * s);
  float d = E::round(x2 * c), e = E::round(x1 * s);
  o1 = E::round(a - b);
  o2 = E::round(d + e);
}

FS_DEVICE bool slot_of(int pos, const int32_t* table, int64_t table_stride, int b, int max_blocks,
                       const fs_kv_layout& kv, int64_t& blk, int& slot) {
  if (pos < 0) return false;
  int bi = pos / kv.block_size;
  if (bi >= max_blocks) return false;
  blk = table[(int64_t)b * table_stride + bi];
  if (blk < 0 || blk >= kv.num_blocks) return false;
  slot = pos - bi * kv.block_size;
  return true;
}

typedef __attribute__((__vector_size__(4 * sizeof(uint32_t)))) uint32_t u32x4_t;

template <int DT>
FS_DEVICE void unpack8(const u32x4_t& w, float (&v)[8]) {
#pragma unroll
  for (int j = 0; j < 4; ++j) {
    v[2 * j] = Elem<DT>::to_f32((uint16_t)(w[j] & 0xffffu));
    v[2 * j + 1] = Elem<DT>::to_f32((uint16_t)(w[j] >> 16));
  }
}

template <int DT>
FS_DEVICE u32x4_t pack8(const float (&v)[8]) {
  u32x4_t w;
#pragma unroll
  for (int j = 0; j < 4; ++j)
    w[j] = (uint32_t)Elem<DT>::store_bits(v[2 * j]) | ((uint32_t)Elem<DT>::store_bits(v[2 * j + 1]) << 16);
  return w;
}

// The same as qkv_rope_write_kernel for 16-bit dtypes whose rows split into 16-byte groups (D/2 % 8 == 0,
// aligned rows, each 8-dim group of a key contiguous): a thread rotates 8 pairs at once (two 16-byte loads of the halves,
// 16-byte loads of cos/sin, 16-byte stores of q and k); values keep the dim-major element stores.
// Eight consecutive qkv elements as floats: the 16-bit row itself, or (PART) the split-K partials of
// the QKV projection [splits][rows][cols] added in increasing split order and rounded to DT, exactly the
// values the GEMM's own reduction would have stored.
struct QkvPart {
  const float* part;   // null: read the 16-bit qkv rows
  int32_t splits;
  int64_t stride;      // elements between consecutive splits (rows * cols)
};

// PART: 0 reads the 16-bit row; > 0 adds that many partials, all loaded before the first add; < 0
// adds pp.splits partials one at a time.
template <int DT, int PART>
FS_DEVICE void load8(const uint16_t* qkv, const QkvPart& pp, int64_t e, float (&v)[8]) {
  if (PART == 0) {
    unpack8<DT>(*reinterpret_cast<const u32x4_t*>(qkv + e), v);
    return;
  }
  float4_t a, b;
  if (PART > 0) {
    constexpr int NS = PART > 0 ? PART : 1;
    float4_t qa[NS], qb[NS];
#pragma unroll
    for (int sp = 0; sp < NS; ++sp) {
      qa[sp] = *reinterpret_cast<const float4_t*>(pp.part + sp * pp.stride + e);
      qb[sp] = *reinterpret_cast<const float4_t*>(pp.part + sp * pp.stride + e + 4);
    }
    a = qa[0];
    b = qb[0];
#pragma unroll
    for (int sp = 1; sp < NS; ++sp)
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        a[j] += qa[sp][j];
        b[j] += qb[sp][j];
      }
  } else {
    a = *reinterpret_cast<const float4_t*>(pp.part + e);
    b = *reinterpret_cast<const float4_t*>(pp.part + e + 4);
    for (int sp = 1; sp < pp.splits; ++sp) {
      const float4_t a2 = *reinterpret_cast<const float4_t*>(pp.part + sp * pp.stride + e);
      const float4_t b2 = *reinterpret_cast<const float4_t*>(pp.part + sp * pp.stride + e + 4);
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        a[j] += a2[j];
        b[j] += b2[j];
      }
    }
  }
#pragma unroll
  for (int j = 0; j < 4; ++j) {
    v[j] = Elem<DT>::round(a[j]);
    v[j + 4] = Elem<DT>::round(b[j]);
  }
}

// Verify windows: T consecutive tokens of a table row (rows back to back, T <= VWIN_MAX_T) sit in
// consecutive pool slots, so a dim's values of the window are one short run of the dim-major value
// tile. Their values are written by the grid's last row of workgroups through LDS, lanes taking
// consecutive tokens of one dim; written per token, every lane of a store would hit its own 32-byte
// run (the 8B verify shape, 448 tokens from two K splits: 12.8 -> 10.6 us per call).
// A window workgroup stages the values of all its heads (at most ceil(n_kv_heads / T) of them) at once.
constexpr int VWIN_MAX_T = 16;
constexpr int VWIN_LDS = 8192;   // 16-bit elements
__host__ __device__ inline bool value_window(int T, const int32_t* token_row, int n_kv_heads, int head_dim) {
  return T > 1 && T <= VWIN_MAX_T && token_row == nullptr && (n_kv_heads + T) * head_dim <= VWIN_LDS;
}

// Grid (token, group block): each thread takes one 8-pair rotation group of a q or k head, or one
// 8-element group of the values (grid.y blocks of blockDim.x groups cover both), so a token's work is
// spread over several workgroups and every thread issues its loads at once. For a verify window
// (value_window) the per-token blocks take only the rotation groups, and workgroup (token m, last
// grid row) writes the values of KV heads m % T, m % T + T, ... for every token of m's row.
template <int DT, int PART = 0>
__global__ void __launch_bounds__(128) qkv_rope_write_vec_kernel(
    const uint16_t* __restrict__ qkv, QkvPart pp, int64_t qkv_stride, int32_t T, int32_t H,
    const int32_t* __restrict__ positions,
    const int32_t* __restrict__ slots, const int32_t* __restrict__ token_row, int32_t n_rows,
    const float* __restrict__ rope_cos, const float* __restrict__ rope_sin,
    int32_t rope_len, const int32_t* __restrict__ table, int64_t table_stride, int32_t max_blocks, fs_kv_layout kv,
    uint16_t* __restrict__ q_out, int64_t q_stride) {
  const int64_t m = blockIdx.x;
  const int D = kv.head_dim, half = D / 2, Hkv = kv.n_kv_heads;
  const int ng = half / 8;
  const int n_groups = (H + Hkv) * ng, nv = Hkv * D / 8;
  const bool vwin = value_window(T, token_row, Hkv, D);
  if (vwin && blockIdx.y == gridDim.y - 1) {
    __shared__ uint16_t vt[VWIN_LDS];   // the window's values of the workgroup's heads, [head][dim][token]
    __shared__ int64_t sblk[VWIN_MAX_T];
    __shared__ int sslot[VWIN_MAX_T], sok[VWIN_MAX_T];
    const int b = (int)(m / T), t0 = (int)(m - (int64_t)b * T);
    const int64_t mrow = (int64_t)b * T;
    if ((int)threadIdx.x < T) {   // each token's pool slot, found as the per-token path finds it
      const int64_t mt = mrow + threadIdx.x;
      const int pos = positions[mt];
      int64_t blk = 0;
      int slot = 0;
      const int wpos = slots ? slots[mt] : pos;
      const bool ok = pos >= 0 && pos < rope_len && slot_of(wpos, table, table_stride, b, max_blocks, kv, blk, slot);
      sblk[threadIdx.x] = blk;
      sslot[threadIdx.x] = slot;
      sok[threadIdx.x] = ok ? 1 : 0;
    }
    uint16_t* vp = reinterpret_cast<uint16_t*>(kv.v);
    const int gpt = D / 8, nh = t0 < Hkv ? (Hkv - t0 + T - 1) / T : 0;   // heads t0, t0 + T, ...
    for (int i = threadIdx.x; i < T * gpt; i += blockDim.x) {   // token i / gpt, dims 8 (i % gpt) ..
      const int t = i / gpt, c = i - t * gpt;
      const int64_t e0 = (mrow + t) * qkv_stride + (int64_t)(H + Hkv + t0) * D + 8 * c;
      for (int h0 = 0; h0 < nh; h0 += 2) {   // two heads' loads in flight together
        u32x4_t w[2];
#pragma unroll
        for (int u = 0; u < 2; ++u) {
          const int64_t e = e0 + (int64_t)min(h0 + u, nh - 1) * T * D;
          if (PART != 0) {
            float x[8];
            load8<DT, PART>(qkv, pp, e, x);
            w[u] = pack8<DT>(x);
          } else {
            w[u] = *reinterpret_cast<const u32x4_t*>(qkv + e);
          }
        }
#pragma unroll
        for (int u = 0; u < 2; ++u) {
          if (h0 + u >= nh) break;
          uint16_t* row = vt + ((h0 + u) * D + 8 * c) * T + t;
#pragma unroll
          for (int j = 0; j < 4; ++j) {
            row[(2 * j) * T] = (uint16_t)(w[u][j] & 0xffffu);
            row[(2 * j + 1) * T] = (uint16_t)(w[u][j] >> 16);
          }
        }
      }
    }
    __syncthreads();
    // thread k stores token k % T of dims k / T, k / T + dstep, ...: a store's lanes run along the
    // tokens of one dim, then to the next dim
    const int tq = (int)threadIdx.x % T, dq = (int)threadIdx.x / T, dstep = (int)blockDim.x / T;
    if (dq < dstep && sok[tq]) {
      uint16_t* vq = vp + sblk[tq] * kv.v_block + (int64_t)t0 * kv.v_head + (int64_t)sslot[tq] * kv.v_slot;
      for (int hi = 0; hi < nh; ++hi) {
        uint16_t* vh = vq + (int64_t)hi * T * kv.v_head;
        const uint16_t* src = vt + hi * D * T + tq;
        for (int d = dq; d < D; d += dstep) vh[(int64_t)d * kv.v_dim] = src[d * T];
      }
    }
    return;
  }
  const int64_t row0 = m * qkv_stride;   // the token's first element (of qkv, or of each partial)
  const int gi = blockIdx.y * blockDim.x + threadIdx.x;
  // The thread's inputs are loaded first: they depend on nothing the position decides, so they are in
  // flight while the position, the rotary row and the pool slot are looked up.
  const bool rot_thread = gi < n_groups, val_thread = !vwin && !rot_thread && gi < n_groups + nv;
  const int head = rot_thread ? gi / ng : 0, p0 = rot_thread ? 8 * (gi - head * ng) : 0;
  const int e0 = val_thread ? 8 * (gi - n_groups) : 0;   // value group: element e0 of the kv heads' values
  float x1[8], x2[8];
  u32x4_t w = {0u, 0u, 0u, 0u};
  if (rot_thread) {
    load8<DT, PART>(qkv, pp, row0 + (int64_t)head * D + p0, x1);
    load8<DT, PART>(qkv, pp, row0 + (int64_t)head * D + p0 + half, x2);
  } else if (val_thread) {
    const int64_t ve = row0 + (int64_t)(H + Hkv) * D + e0;
    if (PART != 0) {
      load8<DT, PART>(qkv, pp, ve, x1);
      w = pack8<DT>(x1);
    } else {
      w = *reinterpret_cast<const u32x4_t*>(qkv + ve);
    }
  }
  int b = token_row ? token_row[m] : (int)(m / T);   // the token's table row
  const bool row_ok = token_row == nullptr || (b >= 0 && b < n_rows);
  b = row_ok ? b : 0;
  const int pos = row_ok ? positions[m] : -1;
  const bool rot_ok = pos >= 0 && pos < rope_len;
  // the rotary row is loaded before the slot lookup: both depend only on the position
  const int64_t cs = rot_ok ? (int64_t)pos * half : 0;
  float4_t c0 = {}, c1 = {}, s0 = {}, s1 = {};
  if (rot_thread) {
    c0 = *reinterpret_cast<const float4_t*>(rope_cos + cs + p0);
    c1 = *reinterpret_cast<const float4_t*>(rope_cos + cs + p0 + 4);
    s0 = *reinterpret_cast<const float4_t*>(rope_sin + cs + p0);
    s1 = *reinterpret_cast<const float4_t*>(rope_sin + cs + p0 + 4);
  }
  int64_t blk = 0;
  int slot = 0;
  const int wpos = slots ? slots[m] : pos;
  const bool write_ok = rot_ok && slot_of(wpos, table, table_stride, b, max_blocks, kv, blk, slot);
  uint16_t* kp = reinterpret_cast<uint16_t*>(kv.k);
  uint16_t* vp = reinterpret_cast<uint16_t*>(kv.v);
  if (rot_thread) {
    float c[8], sn[8], o1[8], o2[8];
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      c[j] = c0[j]; c[j + 4] = c1[j];
      sn[j] = s0[j]; sn[j + 4] = s1[j];
    }
#pragma unroll
    for (int j = 0; j < 8; ++j) {
      o1[j] = o2[j] = 0.f;
      if (rot_ok) rope_pair<DT>(x1[j], x2[j], c[j], sn[j], o1[j], o2[j]);
    }
    if (head < H) {
      uint16_t* qo = q_out + m * q_stride + (int64_t)head * D + p0;
      *reinterpret_cast<u32x4_t*>(qo) = pack8<DT>(o1);
      *reinterpret_cast<u32x4_t*>(qo + half) = pack8<DT>(o2);
    } else if (write_ok) {
      const int64_t kgs = key_group_stride(kv);
      uint16_t* ko = kp + blk * kv.k_block + (int64_t)(head - H) * kv.k_head + slot * kv.k_slot;
      *reinterpret_cast<u32x4_t*>(ko + (p0 >> 3) * kgs) = pack8<DT>(o1);
      *reinterpret_cast<u32x4_t*>(ko + ((p0 + half) >> 3) * kgs) = pack8<DT>(o2);
    }
  }
  if (write_ok && val_thread) {
    const int h = e0 / D, d0 = e0 - h * D;
    uint16_t* vo = vp + blk * kv.v_block + h * kv.v_head + slot * kv.v_slot + d0 * kv.v_dim;
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      vo[(2 * j) * kv.v_dim] = (uint16_t)(w[j] & 0xffffu);
      vo[(2 * j + 1) * kv.v_dim] = (uint16_t)(w[j] >> 16);
    }
  }
}

// One workgroup per token. Threads cover (q heads + kv heads) * D/2 rotation pairs, then the values.
template <int DT>
__global__ void __launch_bounds__(256) qkv_rope_write_kernel(
    const typename Elem<DT>::T* __restrict__ qkv, int64_t qkv_stride, int32_t T, int32_t H,
    const int32_t* __restrict__ positions, const int32_t* __restrict__ slots, const int32_t* __restrict__ token_row,
    int32_t n_rows, const float* __restrict__ rope_cos, const float* __restrict__ rope_sin, int32_t rope_len,
    const int32_t* __restrict__ table,
    int64_t table_stride, int32_t max_blocks, fs_kv_layout kv, typename Elem<DT>::T* __restrict__ q_out,
    int64_t q_stride) {
  typedef Elem<DT> E;
  typedef typename E::T T_;
  const int64_t m = blockIdx.x;
  int b = token_row ? token_row[m] : (int)(m / T);   // the token's table row
  const bool row_ok = token_row == nullptr || (b >= 0 && b < n_rows);
  b = row_ok ? b : 0;
  const int D = kv.head_dim, half = D / 2, Hkv = kv.n_kv_heads;
  const int pos = row_ok ? positions[m] : -1;
  const bool rot_ok = pos >= 0 && pos < rope_len;
  int64_t blk = 0;
  int slot = 0;
  const int wpos = slots ? slots[m] : pos;
  const bool write_ok = rot_ok && slot_of(wpos, table, table_stride, b, max_blocks, kv, blk, slot);
  const T_* row = qkv + m * qkv_stride;
  T_* kp = reinterpret_cast<T_*>(kv.k);
  T_* vp = reinterpret_cast<T_*>(kv.v);

  const int n_pairs = (H + Hkv) * half;
  for (int i = threadIdx.x; i < n_pairs; i += blockDim.x) {
    const int head = i / half, p = i - head * half;
    const float x1 = E::load(row, (int64_t)head * D + p);
    const float x2 = E::load(row, (int64_t)head * D + p + half);
    float o1 = 0.f, o2 = 0.f;
    if (rot_ok) rope_pair<DT>(x1, x2, rope_cos[(int64_t)pos * half + p], rope_sin[(int64_t)pos * half + p], o1, o2);
    if (head < H) {
      T_* qo = q_out + m * q_stride + (int64_t)head * D;
      E::store(qo, p, o1);
      E::store(qo, p + half, o2);
    } else if (write_ok) {
      const int h = head - H;
      const int64_t base = blk * kv.k_block + h * kv.k_head + slot * kv.k_slot;
      E::store(kp, base + key_dim_off(kv, p), o1);
      E::store(kp, base + key_dim_off(kv, p + half), o2);
    }
  }
  if (write_ok) {
    const int n_v = Hkv * D;
    const T_* vrow = row + (int64_t)(H + Hkv) * D;
    for (int i = threadIdx.x; i < n_v; i += blockDim.x) {
      const int h = i / D, d = i - h * D;
      vp[blk * kv.v_block + h * kv.v_head + slot * kv.v_slot + d * kv.v_dim] = vrow[i];
    }
  }
}

// One workgroup per (b, t): scatter k_new[b, :, t, :] and v_new[b, :, t, :].
template <int DT>
__global__ void __launch_bounds__(256) kv_write_kernel(const typename Elem<DT>::T* __restrict__ k_new,
                                                       const typename Elem<DT>::T* __restrict__ v_new,
                                                       int64_t s_b, int64_t s_h, int64_t s_t, int32_t T,
                                                       const int32_t* __restrict__ positions,
                                                       const int32_t* __restrict__ table, int64_t table_stride,
                                                       int32_t max_blocks, fs_kv_layout kv) {
  typedef typename Elem<DT>::T T_;
  const int bt = blockIdx.x;
  const int b = bt / T, t = bt - b * T;
  int64_t blk = 0;
  int slot = 0;
  if (!slot_of(positions[bt], table, table_stride, b, max_blocks, kv, blk, slot)) return;
  const int D = kv.head_dim, n = kv.n_kv_heads * D;
  T_* kp = reinterpret_cast<T_*>(kv.k);
  T_* vp = reinterpret_cast<T_*>(kv.v);
  for (int i = threadIdx.x; i < n; i += blockDim.x) {
    const int h = i / D, d = i - h * D;
    const int64_t src = (int64_t)b * s_b + (int64_t)h * s_h + (int64_t)t * s_t + d;
    kp[blk * kv.k_block + h * kv.k_head + slot * kv.k_slot + key_dim_off(kv, d)] = k_new[src];
    vp[blk * kv.v_block + h * kv.v_head + slot * kv.v_slot + d * kv.v_dim] = v_new[src];
  }
}

// out[b, h, j, d] for j < max_blocks*block_size; invalid block ids read as zeros.
template <int DT>
__global__ void __launch_bounds__(256) gather_kernel(fs_kv_layout kv, const int32_t* __restrict__ table,
                                                     int64_t table_stride, int32_t max_blocks,
                                                     typename Elem<DT>::T* __restrict__ k_out,
                                                     typename Elem<DT>::T* __restrict__ v_out, int64_t total) {
  typedef typename Elem<DT>::T T_;
  const T_* kp = reinterpret_cast<const T_*>(kv.k);
  const T_* vp = reinterpret_cast<const T_*>(kv.v);
  const int D = kv.head_dim, BS = kv.block_size, Hkv = kv.n_kv_heads;
  const int64_t S = (int64_t)max_blocks * BS;
  for (int64_t i = blockIdx.x * (int64_t)blockDim.x + threadIdx.x; i < total; i += (int64_t)gridDim.x * blockDim.x) {
    const int d = (int)(i % D);
    int64_t r = i / D;
    const int64_t j = r % S;
    r /= S;
    const int h = (int)(r % Hkv);
    const int b = (int)(r / Hkv);
    const int64_t blk = table[(int64_t)b * table_stride + j / BS];
    const int slot = (int)(j % BS);
    T_ kv_k = T_(0), kv_v = T_(0);
    if (blk >= 0 && blk < kv.num_blocks) {
      kv_k = kp[blk * kv.k_block + h * kv.k_head + slot * kv.k_slot + key_dim_off(kv, d)];
      kv_v = vp[blk * kv.v_block + h * kv.v_head + slot * kv.v_slot + d * kv.v_dim];
    }
    k_out[i] = kv_k;
    v_out[i] = kv_v;
  }
}

int check_layout(const fs_kv_layout* kv) {
  FS_CHECK_ARG(kv != nullptr && kv->k != nullptr && kv->v != nullptr, "kv layout: null pool");
  FS_CHECK_ARG(kv->dtype == FS_F32 || kv->dtype == FS_BF16 || kv->dtype == FS_F16, "kv layout: bad dtype %d",
               kv->dtype);
  FS_CHECK_ARG(kv->block_size > 0 && kv->n_kv_heads > 0 && kv->head_dim > 0 && kv->head_dim % 2 == 0,
               "kv layout: block_size %d, n_kv_heads %d, head_dim %d", kv->block_size, kv->n_kv_heads,
               kv->head_dim);
  FS_CHECK_ARG(kv->num_blocks > 0, "kv layout: num_blocks %lld", (long long)kv->num_blocks);
  FS_CHECK_ARG(kv->k_group == 0 || (kv->k_group > 0 && kv->k_dim == 1 && kv->head_dim % 8 == 0),
               "kv layout: grouped keys need k_group > 0, k_dim == 1 and head_dim %% 8 == 0 (k_group %lld)",
               (long long)kv->k_group);
  return 0;
}

}  // namespace

namespace {
int qkv_rope_write(const void* qkv, int64_t qkv_stride, int64_t n_tokens, int32_t T, int32_t n_heads,
                   const int32_t* positions, const int32_t* slots, const int32_t* token_row, int32_t n_rows,
                   const float* rope_cos,
                   const float* rope_sin, int32_t rope_len, const int32_t* block_tables, int64_t table_stride,
                   int32_t max_blocks, const fs_kv_layout* kv, void* q_out, int64_t q_stride, void* stream,
                   QkvPart pp = QkvPart{nullptr, 0, 0}) {
  if (int e = check_layout(kv)) return e;
  FS_CHECK_ARG((qkv || pp.part) && positions && rope_cos && rope_sin && block_tables && q_out,
               "qkv_rope_write: null pointer");
  FS_CHECK_ARG(T > 0 && n_tokens >= 0 && n_tokens % T == 0, "qkv_rope_write: n_tokens %lld not a multiple of T %d",
               (long long)n_tokens, T);
  FS_CHECK_ARG(n_heads > 0 && n_heads % kv->n_kv_heads == 0, "qkv_rope_write: n_heads %d vs n_kv_heads %d", n_heads,
               kv->n_kv_heads);
  FS_CHECK_ARG(max_blocks > 0 && table_stride >= max_blocks, "qkv_rope_write: table %d/%lld", max_blocks,
               (long long)table_stride);
  FS_CHECK_ARG(qkv_stride >= (int64_t)(n_heads + 2 * kv->n_kv_heads) * kv->head_dim, "qkv_rope_write: qkv stride");
  if (n_tokens == 0) return 0;
  hipStream_t s = fs::as_stream(stream);
  dim3 grid((unsigned)n_tokens);
  auto al16 = [](const void* p) { return (reinterpret_cast<uintptr_t>(p) & 15) == 0; };
  const bool vec = kv->dtype != FS_F32 && (kv->head_dim / 2) % 8 == 0 && kv->head_dim % 2 == 0 &&
                   qkv_stride % 8 == 0 && q_stride % 8 == 0 && kv->k_dim == 1 && kv->k_slot % 8 == 0 &&
                   kv->k_group % 8 == 0 &&
                   kv->k_head % 8 == 0 && kv->k_block % 8 == 0 && al16(pp.part ? (const void*)pp.part : qkv) &&
                   al16(q_out) && al16(kv->k) && al16(rope_cos) && al16(rope_sin);
  // the vectorised kernel: one thread per 8-element group (q/k rotation groups, then value groups)
  // (a verify window: the rotation groups' blocks, then one row of value workgroups)
  const int rot_groups = (n_heads + kv->n_kv_heads) * (kv->head_dim / 16);
  const int vec_groups = rot_groups + kv->n_kv_heads * kv->head_dim / 8;
  const dim3 vgrid((unsigned)n_tokens, value_window(T, token_row, kv->n_kv_heads, kv->head_dim)
                                           ? (unsigned)((rot_groups + 127) / 128 + 1)
                                           : (unsigned)((vec_groups + 127) / 128));
  if (pp.part) {   // the partials are read by the vectorised kernel only
    FS_CHECK_ARG(vec && pp.splits >= 1 && pp.stride >= n_tokens * qkv_stride,
                 "qkv_rope_write_partials: needs 16-bit data, head_dim/2 %% 8 == 0, 16-byte aligned rows");
#define FS_VEC(DT, P)                                                                                              \
  qkv_rope_write_vec_kernel<DT, P><<<vgrid, 128, 0, s>>>(nullptr, pp, qkv_stride, T, n_heads, positions, slots,      \
                                                         token_row, n_rows, rope_cos, rope_sin, rope_len,            \
                                                         block_tables, table_stride, max_blocks, *kv,                \
                                                         (uint16_t*)q_out, q_stride)
#define FS_VEC_DT(DT)                                                                                              \
  switch (pp.splits) {                                                                                         \
    case 2: FS_VEC(DT, 2); break;                                                                              \
    case 4: FS_VEC(DT, 4); break;                                                                              \
    case 8: FS_VEC(DT, 8); break;                                                                              \
    default: FS_VEC(DT, -1); break;                                                                            \
  }
    if (kv->dtype == FS_BF16) FS_VEC_DT(FS_BF16)
    else FS_VEC_DT(FS_F16)
#undef FS_VEC_DT
#undef FS_VEC
    return fs::launch_status("qkv_rope_write_partials");
  }
  if (vec) {
#define FS_VEC(DT)                                                                                                 \
  qkv_rope_write_vec_kernel<DT><<<vgrid, 128, 0, s>>>((const uint16_t*)qkv, pp, qkv_stride, T, n_heads, positions, \
                                                     slots, token_row, n_rows, rope_cos, rope_sin, rope_len,         \
                                                     block_tables, table_stride, max_blocks, *kv, (uint16_t*)q_out,  \
                                                     q_stride)
    if (kv->dtype == FS_BF16) FS_VEC(FS_BF16);
    else FS_VEC(FS_F16);
#undef FS_VEC
    return fs::launch_status("qkv_rope_write");
  }
#define FS_LAUNCH(DT)                                                                                        \
  qkv_rope_write_kernel<DT><<<grid, 256, 0, s>>>(                                                          \
      (const typename Elem<DT>::T*)qkv, qkv_stride, T, n_heads, positions, slots, token_row, n_rows, rope_cos,    \
      rope_sin, rope_len, \
      block_tables, table_stride, max_blocks, *kv, (typename Elem<DT>::T*)q_out, q_stride)
  switch (kv->dtype) {
    case FS_F32: FS_LAUNCH(FS_F32); break;
    case FS_BF16: FS_LAUNCH(FS_BF16); break;
    default: FS_LAUNCH(FS_F16); break;
  }
#undef FS_LAUNCH
  return fs::launch_status("qkv_rope_write");
}
}  // namespace

extern "C" int fs_qkv_rope_write(const void* qkv, int64_t qkv_stride, int64_t n_tokens, int32_t T, int32_t n_heads,
                                 const int32_t* positions, const int32_t* slots, const float* rope_cos,
                                 const float* rope_sin, int32_t rope_len, const int32_t* block_tables,
                                 int64_t table_stride, int32_t max_blocks, const fs_kv_layout* kv, void* q_out,
                                 int64_t q_stride, void* stream) {
  return qkv_rope_write(qkv, qkv_stride, n_tokens, T, n_heads, positions, slots, nullptr, 0, rope_cos, rope_sin,
                        rope_len, block_tables, table_stride, max_blocks, kv, q_out, q_stride, stream);
}

extern "C" int fs_qkv_rope_write_partials(const float* parts, int32_t splits, int64_t n_tokens, int64_t n_cols,
                                          int32_t T, int32_t n_heads, const int32_t* positions, const int32_t* slots,
                                          const float* rope_cos, const float* rope_sin, int32_t rope_len,
                                          const int32_t* block_tables, int64_t table_stride, int32_t max_blocks,
                                          const fs_kv_layout* kv, void* q_out, int64_t q_stride, void* stream) {
  FS_CHECK_ARG(parts && splits >= 1 && n_cols > 0, "qkv_rope_write_partials: parts / splits %d", splits);
  return qkv_rope_write(nullptr, n_cols, n_tokens, T, n_heads, positions, slots, nullptr, 0, rope_cos, rope_sin,
                        rope_len, block_tables, table_stride, max_blocks, kv, q_out, q_stride, stream,
                        QkvPart{parts, splits, n_tokens * n_cols});
}

extern "C" int fs_qkv_rope_write_varlen(const void* qkv, int64_t qkv_stride, int64_t n_tokens, int32_t n_heads,
                                        const int32_t* positions, const int32_t* token_row, int32_t n_rows,
                                        const float* rope_cos, const float* rope_sin, int32_t rope_len,
                                        const int32_t* block_tables, int64_t table_stride, int32_t max_blocks,
                                        const fs_kv_layout* kv, void* q_out, int64_t q_stride, void* stream) {
  FS_CHECK_ARG(token_row && n_rows > 0, "qkv_rope_write_varlen: token_row / n_rows %d", n_rows);
  return qkv_rope_write(qkv, qkv_stride, n_tokens, 1, n_heads, positions, nullptr, token_row, n_rows, rope_cos,
                        rope_sin,
                        rope_len, block_tables, table_stride, max_blocks, kv, q_out, q_stride, stream);
}

extern "C" int fs_paged_kv_write(const void* k_new, const void* v_new, int64_t s_b, int64_t s_h, int64_t s_t,
                                 int32_t B, int32_t T, const int32_t* positions, const int32_t* block_tables,
                                 int64_t table_stride, int32_t max_blocks, const fs_kv_layout* kv, void* stream) {
  if (int e = check_layout(kv)) return e;
  FS_CHECK_ARG(k_new && v_new && positions && block_tables, "paged_kv_write: null pointer");
  FS_CHECK_ARG(B >= 0 && T >= 0, "paged_kv_write: B %d T %d", B, T);
  FS_CHECK_ARG(max_blocks > 0 && table_stride >= max_blocks, "paged_kv_write: table %d/%lld", max_blocks,
               (long long)table_stride);
  if (B == 0 || T == 0) return 0;
  hipStream_t s = fs::as_stream(stream);
  dim3 grid((unsigned)(B * T));
#define FS_LAUNCH(DT)                                                                                            \
  kv_write_kernel<DT><<<grid, 256, 0, s>>>((const typename Elem<DT>::T*)k_new, (const typename Elem<DT>::T*)v_new, \
                                           s_b, s_h, s_t, T, positions, block_tables, table_stride, max_blocks, *kv)
  switch (kv->dtype) {
    case FS_F32: FS_LAUNCH(FS_F32); break;
    case FS_BF16: FS_LAUNCH(FS_BF16); break;
    default: FS_LAUNCH(FS_F16); break;
  }
#undef FS_LAUNCH
  return fs::launch_status("paged_kv_write");
}

extern "C" int fs_paged_gather(const fs_kv_layout* kv, const int32_t* block_tables, int64_t table_stride, int32_t B,
                               int32_t max_blocks, void* k_out, void* v_out, void* stream) {
  if (int e = check_layout(kv)) return e;
  FS_CHECK_ARG(block_tables && k_out && v_out, "paged_gather: null pointer");
  FS_CHECK_ARG(B >= 0 && max_blocks >= 0 && table_stride >= max_blocks, "paged_gather: B %d max_blocks %d", B,
               max_blocks);
  const int64_t total = (int64_t)B * kv->n_kv_heads * max_blocks * kv->block_size * kv->head_dim;
  if (total == 0) return 0;
  hipStream_t s = fs::as_stream(stream);
  int64_t blocks = (total + 255) / 256;
  if (blocks > 65536) blocks = 65536;
  dim3 grid((unsigned)blocks);
#define FS_LAUNCH(DT)                                                                                 \
  gather_kernel<DT><<<grid, 256, 0, s>>>(*kv, block_tables, table_stride, max_blocks,               \
                                         (typename Elem<DT>::T*)k_out, (typename Elem<DT>::T*)v_out, total)
  switch (kv->dtype) {
    case FS_F32: FS_LAUNCH(FS_F32); break;
    case FS_BF16: FS_LAUNCH(FS_BF16); break;
    default: FS_LAUNCH(FS_F16); break;
  }
#undef FS_LAUNCH
  return fs::launch_status("paged_gather");
}
