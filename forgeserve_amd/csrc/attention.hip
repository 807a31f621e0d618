// Paged causal GQA attention for the verify pass (T = k+1 queries per row), 1-token decode and
// prefill, reading keys/values straight from the block pool.
//
// Reference: paged.py:80-81 (gather every table block) + model.py:70-76 (repeat_interleave GQA,
// key_pos <= query_pos mask, scaled_dot_product_attention with scale 1/sqrt(D)).
//
// Work split (both kernels): the keys of a row are cut into fixed chunks of `split` absolute positions
// (512 for the generic kernel, FS_ATTN_SPLIT (default 16384) for the MFMA kernels; fixed for the life
// of the process); chunk s covers keys
// [s*split, (s+1)*split). Each workgroup produces the softmax partial
// (running max m, sum l, unnormalised output acc) of its chunk, and attn_combine merges the chunks of
// a query in increasing chunk order. A query at position p only ever reads the chunks that hold
// keys <= p, and inside a chunk keys above p contribute exact zeros, so the output of a query does
// not depend on T, on the other rows of the batch, or on how far the other queries of its row reach:
// the verify pass and a 1-token decode at the same position give bit-identical outputs.
//
// Fast path (bf16, head_dim 64/128, block_size % 16 == 0, fs_kv_layout with slot-major keys and
// dim-major values): one wavefront per (chunk, batch row, kv head, 32-row query tile). The query
// tile is the (token, group-head) pairs of one KV head: rows = T * (n_heads / n_kv_heads).
//   S^T[key, row] = K . Q^T    v_mfma_f32_16x16x32_bf16, A = 16 keys x 32 dims straight from HBM
//   O^T[dim, row] += V^T . P^T v_mfma_f32_16x16x16_bf16, A = 16 dims x 4 keys of the dim-major tile
// With the transposed products every lane owns whole query rows (row = lane % 16), so the softmax
// statistics, the P operand and the O rescale stay in the lane's own registers.
#include <math.h>
#include <stdlib.h>

#include "common.h"

namespace {

constexpr int QTILE = 32;            // query rows per MFMA wave
constexpr int PLAN_THREADS = 256;
constexpr int SPLIT_UNITS_MAX = 128;  // calls with at most this many units (half the CUs) split each in two,
constexpr int SPLIT_MIN_KEYS = 3072;  // when their tables can hold this many keys (shorter units do not repay
                                      // the exchange)
// workspace: item count (bytes 0..255), the split units' arrival counters (one unsigned each), then
// the item list, the chunk partials and the split units' published partials
constexpr int64_t WS_COUNTERS = 256;
constexpr int64_t WS_HEADER = WS_COUNTERS + 4 * SPLIT_UNITS_MAX;
constexpr float LOG2E = 1.4426950408889634f;

struct AttnParams {
  const void* q;
  int64_t q_sb, q_st, q_sh;
  fs_kv_layout kv;
  const int32_t* table;
  int64_t table_stride;
  int32_t max_blocks;
  const int32_t* pos;
  int32_t B, T, H, G;                // G = n_heads / n_kv_heads
  float scale_log2;                  // scale * log2(e): scores are kept in the log2 domain
  float* ws_acc;                     // [B*T*H][nsplit][D]
  float* ws_ml;                      // [B*T*H][nsplit][2]
  int32_t nsplit;
  int32_t split;                     // keys per chunk: a multiple of 16
  struct AttnItem* items;            // MFMA path: the work list written by attn_plan_kernel
  int32_t* n_items;                  // its length
  // MFMA path: a query that sees one chunk only (position < split, or nsplit == 1) has its output
  // written by that chunk's workgroup, and attn_combine leaves it alone
  int32_t direct;
  void* out;
  int64_t o_sb, o_st, o_sh;
  // packed (varlen) rows: when set, row b's token t is token row_start[b] + t of q and out (strides
  // q_st/q_sh, o_st/o_sh; q_sb and o_sb unused), and only tokens t < row_start[b+1] - row_start[b]
  // exist: the others (positions -1) are neither read nor written
  const int32_t* row_start;
  // query tiles per plan item: 1 for the unit kernel, PF_WAVES for the prefill kernel (item.z is then
  // the index of a group of zgroup consecutive tiles, item.qmax the group's furthest query)
  int32_t zgroup;
  // split units (attn_unit_half_kernel): one arrival counter per unit (zero between launches) and
  // SPLIT_SLOTS published partials per unit
  unsigned* split_cnt;
  float* split_ws;
};

// Reductions over the four 16-lane groups of a wave (lanes l, l^16, l^32, l^48) with the gfx950
// row swaps: permlane16_swap of (x, x) yields {rows 0,0,2,2 ; rows 1,1,3,3} of x, permlane32_swap
// yields {lanes 0-31 twice ; lanes 32-63 twice}. Both steps are symmetric, so every lane ends with
// the same value, and the sum adds (g0 + g1) + (g2 + g3) in every lane.
// 2^x with the bare v_exp_f32 (no denormal-result scaling): the same value as exp2f wherever the
// result is a normal float.
FS_DEVICE float fast_exp2(float x) { return __builtin_amdgcn_exp2f(x); }

// The maxima over the lanes l, l ^ 16, l ^ 32, l ^ 48 of x0 and of x1, in three swaps:
// permlane16_swap of (x0, x1) yields {x0 rows 0,1 ; x1 rows 0,1 ; x0 rows 2,3 ; x1 rows 2,3} as pairs,
// so one maximum leaves x0's groups 0/1 and 2/3 in rows 0 and 2 and x1's in rows 1 and 3;
// permlane32_swap and a maximum complete both (x0's in rows 0 and 2, x1's in rows 1 and 3), and a last
// permlane16_swap hands every lane both. Every lane gets max(max(g0, g1), max(g2, g3)). IEEE maximum
// (v_maximum3_f32, one instruction) rather than fmaxf, which needs its permuted operands canonicalised
// first; the two agree on every non-NaN input (the scores are finite or -inf) up to the sign of a
// zero maximum, which no result depends on.
FS_DEVICE void max_across_groups2(float x0, float x1, float& m0, float& m1) {
  auto a = __builtin_amdgcn_permlane16_swap(__float_as_uint(x0), __float_as_uint(x1), false, false);
  const float y = __builtin_elementwise_maximum(__uint_as_float(a[0]), __uint_as_float(a[1]));
  auto b = __builtin_amdgcn_permlane32_swap(__float_as_uint(y), __float_as_uint(y), false, false);
  const float z = __builtin_elementwise_maximum(__uint_as_float(b[0]), __uint_as_float(b[1]));
  auto c = __builtin_amdgcn_permlane16_swap(__float_as_uint(z), __float_as_uint(z), false, false);
  m0 = __uint_as_float(c[0]);
  m1 = __uint_as_float(c[1]);
}

FS_DEVICE float sum_across_groups(float x) {
  auto a = __builtin_amdgcn_permlane16_swap(__float_as_uint(x), __float_as_uint(x), false, false);
  x = __uint_as_float(a[0]) + __uint_as_float(a[1]);
  auto b = __builtin_amdgcn_permlane32_swap(__float_as_uint(x), __float_as_uint(x), false, false);
  return __uint_as_float(b[0]) + __uint_as_float(b[1]);
}

// Four floats to bf16 (round to nearest even) with gfx950's packed conversion, as MFMA operand bits.
FS_DEVICE short4_t bf16_rne4(const float (&v)[4]) {
  typedef __attribute__((__vector_size__(2 * sizeof(float)))) float f32x2;
  typedef __attribute__((__vector_size__(2 * sizeof(__bf16)))) __bf16 bf16x2;
  const bf16x2 a = __builtin_convertvector((f32x2){v[0], v[1]}, bf16x2);
  const bf16x2 b = __builtin_convertvector((f32x2){v[2], v[3]}, bf16x2);
  const uint32_t ua = __builtin_bit_cast(uint32_t, a), ub = __builtin_bit_cast(uint32_t, b);
  return short4_t{(short)(ua & 0xffff), (short)(ua >> 16), (short)(ub & 0xffff), (short)(ub >> 16)};
}

FS_DEVICE int64_t row_index(const AttnParams& P, int b, int t, int h) { return ((int64_t)b * P.T + t) * P.H + h; }

FS_DEVICE bool token_exists(const AttnParams& P, int b, int t) {
  return P.row_start == nullptr || t < P.row_start[b + 1] - P.row_start[b];
}
FS_DEVICE int64_t q_offset(const AttnParams& P, int b, int t) {
  return P.row_start ? (int64_t)(P.row_start[b] + t) * P.q_st : (int64_t)b * P.q_sb + (int64_t)t * P.q_st;
}
FS_DEVICE int64_t o_offset(const AttnParams& P, int b, int t, int64_t o_sb, int64_t o_st) {
  return P.row_start ? (int64_t)(P.row_start[b] + t) * o_st : (int64_t)b * o_sb + (int64_t)t * o_st;
}

// ------------------------------------------------------------------------------------------------
// work plan: the (query tile, chunk) items that hold visible keys
// ------------------------------------------------------------------------------------------------
struct AttnItem {
  int32_t b, z, s, qmax;   // batch row, query tile, chunk, furthest query position of the tile
};

// furthest query position of query rows [row0, row0 + n) of batch row b (-1 if none)
FS_DEVICE int rows_qmax(const AttnParams& P, int b, int row0, int n) {
  n = min(n, P.T * P.G - row0);
  if (n <= 0) return -1;
  const int t0 = row0 / P.G, t1 = (row0 + n - 1) / P.G;
  const int* posb = P.pos + (int64_t)b * P.T;
  int q = -1;
  for (int t = t0; t <= t1; ++t) q = max(q, posb[t]);
  return q;
}
FS_DEVICE int tile_qmax(const AttnParams& P, int b, int z) { return rows_qmax(P, b, z * QTILE, QTILE); }

// Chunks a query tile reads. With direct outputs a tile of padding queries still gets chunk 0, whose
// workgroup writes their zero outputs.
FS_DEVICE int tile_chunks(const AttnParams& P, int qmax) {
  return qmax < 0 ? (P.direct ? 1 : 0) : min(qmax / P.split + 1, P.nsplit);
}

constexpr int UNIT_WAVES = 8;                  // waves per unit workgroup
constexpr int HALF_WAVES = UNIT_WAVES / 2;      // waves per workgroup of a split unit
constexpr int SPLIT_SLOTS = 5;                  // published partials per split unit
// floats of one published partial: m and l of the 32 rows, then acc as the LDS holds it (2 * D/16
// (half, dim tile) pairs, 64 lanes, 4 values)
constexpr int64_t split_slot_floats(int D) { return 2 * QTILE + (int64_t)QTILE * D; }
constexpr int MAX_SPLIT = 2 * 64 * 16 * UNIT_WAVES;   // keys per chunk, at most: a wave's tiles fit two
                                                       // table entries per lane

// One workgroup lists every item: first the chunks that lie wholly below their tile's furthest
// query (the full chunks), tile by tile, then the last chunk of each tile, longest first. Workgroups
// start in list order, so the short last chunks even out the finish (longest-first list scheduling).
// Inclusive scan of one int per thread over the workgroup: lane scans inside each wave, then the
// wave totals (two barriers). `tot` receives the workgroup's total.
FS_DEVICE int block_scan(int x, int* sh, int& tot) {
  const int lane = threadIdx.x & 63, wv = threadIdx.x >> 6;
#pragma unroll
  for (int off = 1; off < 64; off <<= 1) {
    const int y = __shfl_up(x, off, 64);
    if (lane >= off) x += y;
  }
  if (lane == 63) sh[wv] = x;
  __syncthreads();
  int before = 0;
  tot = 0;
#pragma unroll
  for (int k = 0; k < PLAN_THREADS / 64; ++k) {
    const int t = sh[k];
    if (k < wv) before += t;
    tot += t;
  }
  __syncthreads();
  return x + before;
}

__global__ void __launch_bounds__(PLAN_THREADS) attn_plan_kernel(AttnParams P) {
  // the split units' arrival counters start at zero (each unit's second half leaves its counter zero,
  // so calls that reuse this plan find them so too)
  for (int i = threadIdx.x; i < SPLIT_UNITS_MAX; i += PLAN_THREADS) st_ag(P.split_cnt + i, 0u);
  __shared__ int sh[PLAN_THREADS / 64];
  __shared__ int cursor[MAX_SPLIT / 16 + 1];   // last chunks by length in 16-key tiles
  const int tid = threadIdx.x;
  const int qtiles = (P.T * P.G + QTILE - 1) / QTILE;
  const int U = P.B * qtiles;
  if (qtiles > 1) {
    // A prefill (several query tiles per row): the tiles (or groups of zgroup tiles) of one row are
    // listed together, longest first, so the workgroups running at any time on an XCD (one KV head
    // each) read one row's keys and values and share them in that XCD's L2; across rows the reads
    // would not fit it. The order decides only which workgroup runs an item, never what it computes.
    const int qg = (qtiles + P.zgroup - 1) / P.zgroup;
    const int UG = P.B * qg;
    int base = 0;
    for (int u0 = 0; u0 < UG; u0 += PLAN_THREADS) {
      const int u = u0 + tid;
      int qm = -1, nch = 0, b = 0, z = 0;
      if (u < UG) {
        b = u / qg;
        z = qg - 1 - (u - b * qg);
        qm = rows_qmax(P, b, z * P.zgroup * QTILE, P.zgroup * QTILE);
        nch = tile_chunks(P, qm);
      }
      int n_round;
      const int e0 = base + block_scan(nch, sh, n_round) - nch;
      for (int c = 0; c < nch; ++c) P.items[e0 + c] = AttnItem{b, z, c, qm};
      base += n_round;
    }
    if (tid == 0) P.n_items[0] = base;
    return;
  }
  const int nlen = P.split / 16;   // a last chunk holds 1..nlen tiles (an empty one counts as 1)
  for (int i = tid; i <= nlen; i += PLAN_THREADS) cursor[i] = 0;
  // the thread's first tile (u = tid) stays in registers; tiles past the first PLAN_THREADS are
  // recomputed when needed
  int qm0 = -1, nch0 = 0;
  if (tid < U) {
    qm0 = tile_qmax(P, tid / qtiles, tid % qtiles);
    nch0 = tile_chunks(P, qm0);
  }
  auto tile = [&](int u, int& qm, int& nch) {
    if (u == tid) {
      qm = qm0;
      nch = nch0;
    } else {
      qm = tile_qmax(P, u / qtiles, u % qtiles);
      nch = tile_chunks(P, qm);
    }
  };
  auto last_tiles = [&](int qm, int nch) { return max(min((qm + 1 - (nch - 1) * P.split + 15) >> 4, nlen), 1); };
  __syncthreads();
  int nf = 0;
  for (int u = tid; u < U; u += PLAN_THREADS) {   // full chunks, and a histogram of the last chunks' lengths
    int qm, nch;
    tile(u, qm, nch);
    nf += max(nch - 1, 0);
    if (nch > 0) atomicAdd(&cursor[last_tiles(qm, nch)], 1);
  }
  int n_full;
  block_scan(nf, sh, n_full);
  {   // exclusive scan from the longest length down: cursor[len] = first slot of that length
    constexpr int PER = (MAX_SPLIT / 16 + PLAN_THREADS - 1) / PLAN_THREADS;
    int c[PER], loc = 0;
#pragma unroll
    for (int k = 0; k < PER; ++k) {   // thread tid owns lengths nlen - PER*tid - k
      const int len = nlen - PER * tid - k;
      c[k] = len >= 1 ? cursor[len] : 0;
      loc += c[k];
    }
    int n_last;
    int run = n_full + block_scan(loc, sh, n_last) - loc;
#pragma unroll
    for (int k = 0; k < PER; ++k) {
      const int len = nlen - PER * tid - k;
      if (len >= 1) cursor[len] = run;
      run += c[k];
    }
    if (tid == 0) P.n_items[0] = n_full + n_last;
    __syncthreads();
  }
  int base_full = 0;
  for (int u0 = 0; u0 < U; u0 += PLAN_THREADS) {
    const int u = u0 + tid;
    int qm = -1, nch = 0;
    if (u < U) tile(u, qm, nch);
    const int b = u / qtiles, z = u - b * qtiles;
    const int f = max(nch - 1, 0);
    int n_round;
    const int ef = base_full + block_scan(f, sh, n_round) - f;
    for (int c = 0; c < f; ++c) P.items[ef + c] = AttnItem{b, z, c, qm};
    // the slot order inside one length is whatever the atomics give: it only changes which
    // workgroup runs an item, never what the item computes
    if (nch > 0) P.items[atomicAdd(&cursor[last_tiles(qm, nch)], 1)] = AttnItem{b, z, nch - 1, qm};
    base_full += n_round;
  }
}

// ------------------------------------------------------------------------------------------------
// MFMA kernel (bf16)
// ------------------------------------------------------------------------------------------------
// ------------------------------------------------------------------------------------------------
// unit kernel: one workgroup of UNIT_WAVES waves per (plan item, KV head)
// ------------------------------------------------------------------------------------------------
// The item's keys [kbeg, kend) are cut into 16-key tiles; wave w takes tiles w, w + UNIT_WAVES, ...
// in increasing order and keeps its own softmax partial, and the waves' partials are merged through
// LDS in wave order. Which tiles a wave sees, and in what order, depends only on absolute key
// positions, and a tile wholly above a query's position leaves that query's partial exactly as it
// was; a query's result therefore does not depend on the other queries of its tile.

// One 16-key tile into a wave's online-softmax partial of up to 32 query rows (two 16-row halves; the
// second only when `two`). kf holds the tile's keys as A operands of S^T = K.Q^T, vf its values as A
// operands of O^T += V^T.P^T (zeroed in place where a key must not reach the product: an unmapped
// block, or a key past qmax, the furthest query of the 32 rows, which may never have been written).
// j0 is the tile's first key, rpos the positions of the lane's two rows (-1: no query), rmin the
// smallest position over all 32 rows (-1 if any row is missing). A key above a row's position gets
// score -inf.
//
// The partial is (m, l, acc) with p = 2^(s - m): m is a reference maximum that moves only when a
// tile's maximum exceeds it by more than 8 (then to that maximum, and acc and l are rescaled), so
// p <= 2^8 and the rescale is rare once a row has seen a few tiles. A tile wholly above a row leaves
// that row's partial exactly as it was (m unchanged, alpha = 1, p = 0). A tile whose keys every row
// sees takes a path without the per-key masks; its arithmetic is the same. LAZY skips the rescale
// when no row of the wave moved (multiplying by alpha = 1 is exact, so the bits do not change). Every
// kernel that builds a partial calls this function, so a row's partial does not depend on which
// kernel ran it.
// Smallest position over the rows r < nrows of a wave's 32-row tile (-1 if nrows <= 0); the rows of
// lane l16 are l16 and 16 + l16, whose positions are rpos[0] and rpos[1].
FS_DEVICE int rows_min_pos(const int (&rpos)[2], int nrows) {
  if (nrows <= 0) return -1;
  const int l16 = threadIdx.x & 15;
  int v = min(l16 < nrows ? rpos[0] : 0x7fffffff, 16 + l16 < nrows ? rpos[1] : 0x7fffffff);
#pragma unroll
  for (int o = 1; o < 16; o <<= 1) v = min(v, __shfl_xor(v, o, 64));
  return __builtin_amdgcn_readfirstlane(v);
}

constexpr float REF_SLACK = 8.f;   // log2 units a tile's maximum may exceed the reference by

// The softmax step of one tile for the lane's two rows: scores in log2 units (a key the row may not
// see gets -inf; FULL: every row sees every key), the tile's row maxima, the references (a row's m
// moves to the tile's maximum when that exceeds m by more than REF_SLACK), p = 2^(s - m) as bf16
// MFMA operands, and l <- l * alpha + (the lane's sum of p), alpha = 2^(m_old - m_new) for a row
// that moved, else 1. Returns whether any row of the wave moved; alpha is for the caller's rescale
// of acc. LAZY: when no row moved, l <- l + sum, which is l * 1 + sum bit for bit.
template <bool FULL, bool LAZY>
FS_DEVICE bool tile_probs(const float4_t (&sc)[2], int j0, bool tile_valid, const int (&rpos)[2], float scale_log2,
                          float (&m_run)[2], float (&l_run)[2], float (&alpha)[2], short4_t (&pf)[2]) {
  const int g = (threadIdx.x & 63) >> 4;
  float sv[2][4], x[2];
#pragma unroll
  for (int nt = 0; nt < 2; ++nt) {
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      const float v = sc[nt][e] * scale_log2;
      sv[nt][e] = (FULL || (tile_valid && j0 + 4 * g + e <= rpos[nt])) ? v : -INFINITY;
    }
    x[nt] = __builtin_elementwise_maximum(__builtin_elementwise_maximum(sv[nt][0], sv[nt][1]),
                                          __builtin_elementwise_maximum(sv[nt][2], sv[nt][3]));
  }
  // A row's tile maximum exceeds m + REF_SLACK exactly when one of its four lane groups' maxima does.
  // LAZY: when no lane's does, no row moves (m_new = m, alpha = 1), and the reduction across the lane
  // groups is skipped: the same values as the path below.
  if (LAZY && !__any(x[0] > m_run[0] + REF_SLACK || x[1] > m_run[1] + REF_SLACK)) {
#pragma unroll
    for (int nt = 0; nt < 2; ++nt) {
      float pv[4];
#pragma unroll
      for (int e = 0; e < 4; ++e)
        pv[e] = (FULL || sv[nt][e] != -INFINITY) ? fast_exp2(sv[nt][e] - m_run[nt]) : 0.f;
      pf[nt] = bf16_rne4(pv);
      alpha[nt] = 1.f;
      l_run[nt] = l_run[nt] + ((pv[0] + pv[1]) + (pv[2] + pv[3]));
    }
    return false;
  }
  float tmax[2];
  max_across_groups2(x[0], x[1], tmax[0], tmax[1]);
  bool mv[2];
  float m_new[2], psum[2];
#pragma unroll
  for (int nt = 0; nt < 2; ++nt) {
    // (-inf > x is false: a row that sees nothing here keeps its reference)
    mv[nt] = tmax[nt] > m_run[nt] + REF_SLACK;
    m_new[nt] = mv[nt] ? tmax[nt] : m_run[nt];
    float pv[4];
#pragma unroll
    for (int e = 0; e < 4; ++e)
      pv[e] = (FULL || sv[nt][e] != -INFINITY) ? fast_exp2(sv[nt][e] - m_new[nt]) : 0.f;
    pf[nt] = bf16_rne4(pv);
    psum[nt] = (pv[0] + pv[1]) + (pv[2] + pv[3]);
  }
  const bool moved = __any(mv[0] || mv[1]);
  if (!LAZY || moved) {
#pragma unroll
    for (int nt = 0; nt < 2; ++nt) {
      alpha[nt] = mv[nt] ? fast_exp2(m_run[nt] - m_new[nt]) : 1.f;
      l_run[nt] = l_run[nt] * alpha[nt] + psum[nt];
    }
  } else {
#pragma unroll
    for (int nt = 0; nt < 2; ++nt) {
      alpha[nt] = 1.f;
      l_run[nt] = l_run[nt] + psum[nt];
    }
  }
#pragma unroll
  for (int nt = 0; nt < 2; ++nt) m_run[nt] = m_new[nt];
  return moved;
}

template <int D, bool LAZY, bool BOTH = false>
FS_DEVICE void attn_tile(const bf16x8_t (&kf)[D / 32], short4_t (&vf)[D / 16], int j0, bool tile_valid, int qmax,
                         const int (&rpos)[2], int rmin, bool two, const bf16x8_t (&qf)[2][D / 32],
                         float scale_log2, float4_t (&acc)[D / 16][2], float (&m_run)[2], float (&l_run)[2]) {
  constexpr int KS = D / 32;
  constexpr int MT = D / 16;
  const int g = (threadIdx.x & 63) >> 4;
  const bool full = tile_valid && j0 + 15 <= rmin;   // wave-uniform
  if (!full && (!tile_valid || j0 + 15 > qmax)) {
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      if (!tile_valid || j0 + 4 * g + e > qmax) {
#pragma unroll
        for (int mt = 0; mt < MT; ++mt) vf[mt][e] = 0;
      }
    }
  }
  // BOTH: the second half's products are formed whatever `two` says (rows past the tile's end hold
  // values that are never written out), so the two halves' MFMA chains interleave without a branch
  float4_t sc[2];
  if (BOTH) {
    sc[0] = float4_t{0.f, 0.f, 0.f, 0.f};
    sc[1] = float4_t{0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int ks = 0; ks < KS; ++ks) {
      sc[0] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(kf[ks], qf[0][ks], sc[0], 0, 0, 0);
      sc[1] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(kf[ks], qf[1][ks], sc[1], 0, 0, 0);
    }
  } else {
#pragma unroll
    for (int nt = 0; nt < 2; ++nt) {
      sc[nt] = float4_t{0.f, 0.f, 0.f, 0.f};
      if (nt == 0 || two) {
#pragma unroll
        for (int ks = 0; ks < KS; ++ks)
          sc[nt] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(kf[ks], qf[nt][ks], sc[nt], 0, 0, 0);
      }
    }
  }
  short4_t pf[2];
  float alpha[2];
  const bool moved = full ? tile_probs<true, LAZY>(sc, j0, tile_valid, rpos, scale_log2, m_run, l_run, alpha, pf)
                          : tile_probs<false, LAZY>(sc, j0, tile_valid, rpos, scale_log2, m_run, l_run, alpha, pf);
  // LAZY: only when a row moved (alpha = 1 for every row that did not, so skipping it is exact)
  if (!LAZY || moved) {
#pragma unroll
    for (int mt = 0; mt < MT; ++mt)
#pragma unroll
      for (int nt = 0; nt < 2; ++nt) {
        acc[mt][nt][0] *= alpha[nt];
        acc[mt][nt][1] *= alpha[nt];
        acc[mt][nt][2] *= alpha[nt];
        acc[mt][nt][3] *= alpha[nt];
      }
  }
#pragma unroll
  for (int mt = 0; mt < MT; ++mt) {
    acc[mt][0] = __builtin_amdgcn_mfma_f32_16x16x16bf16_1k(vf[mt], pf[0], acc[mt][0], 0, 0, 0);
    if (BOTH || two) acc[mt][1] = __builtin_amdgcn_mfma_f32_16x16x16bf16_1k(vf[mt], pf[1], acc[mt][1], 0, 0, 0);
  }
}

// A chunk's result for one query row is its 8 partials (tiles t with t % 8 == v, v = 0..7) folded in
// increasing v: (M, L, O) <- (max(M, m), L*2^(M-M') + l*2^(m-M'), O*2^(M-M') + a*2^(m-M')). An empty
// partial (m = -inf: no visible key) leaves the state as it is; the first non-empty one gets weight 1
// and the empty state weight 2^-inf = 0. fold_weights returns false for an empty partial.
FS_DEVICE bool fold_weights(float M, float m, float& Mn, float& cM, float& cm) {
  if (m == -INFINITY) return false;
  Mn = fmaxf(M, m);
  cM = fast_exp2(M - Mn);
  cm = fast_exp2(m - Mn);
  return true;
}
FS_DEVICE float fold_value(float x, float cM, float y, float cm) { return x * cM + y * cm; }

template <int D, int BSZ>
__device__ __attribute__((always_inline)) inline void attn_wave_tiles(const AttnParams& P, int b, int kbeg, int kend,
                                                                      int qmax, int row0, int nrows,
                                                                      const int (&rpos)[2], int hkv, int w,
                                                                      float4_t (*red_acc)[64], float* red_m,
                                                                      float* red_l) {
  constexpr int KS = D / 32;   // k-steps of the QK^T product
  constexpr int MT = D / 16;   // 16-dim tiles of the PV product
  const int lane = threadIdx.x & 63;
  const int l16 = lane & 15, g = lane >> 4;
  const int ntiles = (kend - kbeg + 15) >> 4;
  const int nt_w = ntiles > w ? (ntiles - w + UNIT_WAVES - 1) / UNIT_WAVES : 0;   // <= 128 tiles
  const bool two = nrows > 16;
  const int BS = BSZ ? BSZ : P.kv.block_size;
  const int64_t v_dim = BSZ ? BSZ : P.kv.v_dim;   // == block_size (dim-major values)

  // lane i: raw table entries of the blocks holding this wave's tiles i and 64 + i (-1 past the table)
  int my_phys[2] = {-1, -1};
#pragma unroll
  for (int h = 0; h < 2; ++h) {
    const int i = 64 * h + lane;
    if (i < nt_w) {
      const int blk = (kbeg + 16 * (w + UNIT_WAVES * i)) / BS;
      if (blk < P.max_blocks) my_phys[h] = P.table[(int64_t)b * P.table_stride + blk];
    }
  }

  typedef uint16_t u16;
  const u16* kpool = reinterpret_cast<const u16*>(P.kv.k);
  const u16* vpool = reinterpret_cast<const u16*>(P.kv.v);
  const int64_t k_head_off = (int64_t)hkv * P.kv.k_head;
  const int64_t v_head_off = (int64_t)hkv * P.kv.v_head;
  // key (slot, dims 8c .. 8c+7) at slot * k_slot + c * kgs: slot-major (k_slot = D, kgs = 8) or grouped
  // (k_slot = 8, kgs = 8 * block_size: one load of a tile's 32 dims is a contiguous 1 KB)
  const int64_t k_slot = P.kv.k_slot, kgs = key_group_stride(P.kv);

  // Three tile buffers in registers: while tile i is consumed, tiles i+1 and i+2 are in flight.
  // Every load is unconditional (a prefetch past the end re-reads the last tile, an unmapped block
  // reads block 0 and is masked in consume) so that each wait before a consume counts exactly the
  // loads issued after that tile, on every path through the loop.
  bf16x8_t kb0[KS], kb1[KS], kb2[KS];
  short4_t vb0[MT], vb1[MT], vb2[MT];

  auto key0 = [&](int i) { return kbeg + 16 * (w + UNIT_WAVES * i); };
  auto block_of = [&](int i) {   // physical block of the wave's i-th tile, -1 when unmapped (i uniform)
    const int v = __builtin_amdgcn_readlane(i < 64 ? my_phys[0] : my_phys[1], i & 63);
    return (v >= 0 && v < P.kv.num_blocks) ? v : -1;
  };

  // the lane's element offsets inside a tile, fixed for the launch; a tile adds its wave-uniform base
  const int64_t k_lane = (int64_t)l16 * k_slot + g * kgs;
  const int64_t v_lane = (int64_t)l16 * v_dim + 4 * g;
  auto load_tile = [&](int i, bf16x8_t (&kd)[KS], short4_t (&vd)[MT]) {
    const int ic = max(min(i, nt_w - 1), 0);   // a wave without tiles reads block 0 and consumes nothing
    const int j0 = key0(ic);
    const int phys = block_of(ic);
    const int64_t pb = phys >= 0 ? phys : 0;
    const int slot0 = j0 - (j0 / BS) * BS;
    const u16* kt_ = kpool + (pb * P.kv.k_block + k_head_off + (int64_t)slot0 * k_slot) + k_lane;
#pragma unroll
    for (int ks = 0; ks < KS; ++ks)   // read once per launch: nontemporal
      kd[ks] = __builtin_nontemporal_load(reinterpret_cast<const bf16x8_t*>(kt_ + 4 * ks * kgs));
    const u16* vt_ = vpool + (pb * P.kv.v_block + v_head_off + slot0) + v_lane;
#pragma unroll
    for (int mt = 0; mt < MT; ++mt)
      vd[mt] = __builtin_nontemporal_load(reinterpret_cast<const short4_t*>(vt_ + (int64_t)(16 * mt) * v_dim));
  };

  load_tile(0, kb0, vb0);
  load_tile(1, kb1, vb1);

  // Q fragments (B operand of S^T): Q[row][32*ks + 8*g .. +8]
  const u16* qbase = reinterpret_cast<const u16*>(P.q);
  bf16x8_t qf[2][KS];
#pragma unroll
  for (int nt = 0; nt < 2; ++nt) {
    const int r = row0 + 16 * nt + l16;
    const bool in_tile = (16 * nt + l16) < nrows;
    const bool ok = in_tile && token_exists(P, b, r / P.G);
    const int t = ok ? r / P.G : 0;
    const int h = hkv * P.G + (ok ? r - (r / P.G) * P.G : 0);
    const u16* qr = qbase + q_offset(P, b, t) + (int64_t)h * P.q_sh;
#pragma unroll
    for (int ks = 0; ks < KS; ++ks) {
      if (ok)
        qf[nt][ks] = *reinterpret_cast<const bf16x8_t*>(qr + 32 * ks + 8 * g);
      else
        qf[nt][ks] = bf16x8_t{};
    }
  }

  float4_t acc[MT][2];
#pragma unroll
  for (int mt = 0; mt < MT; ++mt) {
    acc[mt][0] = float4_t{0.f, 0.f, 0.f, 0.f};
    acc[mt][1] = float4_t{0.f, 0.f, 0.f, 0.f};
  }
  float m_run[2] = {-INFINITY, -INFINITY};
  float l_run[2] = {0.f, 0.f};

  const int rmin = rows_min_pos(rpos, nrows);
  auto consume = [&](int i, const bf16x8_t (&kf)[KS], short4_t (&vf)[MT]) {
    attn_tile<D, true>(kf, vf, key0(i), block_of(i) >= 0, qmax, rpos, rmin, two, qf, P.scale_log2, acc, m_run,
                        l_run);
  };

  for (int i = 0; i < nt_w; i += 3) {
    load_tile(i + 2, kb2, vb2);
    consume(i, kb0, vb0);
    if (i + 1 >= nt_w) break;
    load_tile(i + 3, kb0, vb0);
    consume(i + 1, kb1, vb1);
    if (i + 2 >= nt_w) break;
    load_tile(i + 4, kb1, vb1);
    consume(i + 2, kb2, vb2);
  }
  // this wave's partial to LDS: acc by (query half, dim tile, lane), m and l by query row
#pragma unroll
  for (int nt = 0; nt < 2; ++nt) {
#pragma unroll
    for (int mt = 0; mt < MT; ++mt) red_acc[nt * MT + mt][lane] = acc[mt][nt];
    const float lsum = sum_across_groups(l_run[nt]);
    if (g == 0) {
      red_m[16 * nt + l16] = m_run[nt];
      red_l[16 * nt + l16] = lsum;
    }
  }
}

// Row `rr` of the query rows (token rr / G, head hkv*G + rr % G), dims 16*mt + 4g .. +4, from its
// folded chunk-s state (M, L, O): a query that sees one chunk only is finished here (a padding query,
// position < 0, gets zeros from chunk 0); any other query gets this chunk's partial for attn_combine
// if the chunk holds keys it sees.
template <int D>
FS_DEVICE void attn_emit(const AttnParams& P, int b, int s, int kbeg, int hkv, int rr, int rp, int mt, float M,
                         float L, const float4_t& o) {
  const int lane = threadIdx.x & 63, g = lane >> 4;
  const bool direct = P.direct && (rp < P.split || P.nsplit == 1);
  if (direct ? s != 0 : rp < kbeg) return;
  const int t = rr / P.G, h = hkv * P.G + (rr - t * P.G);
  if (direct) {   // the same normalisation as attn_combine's
    if (!token_exists(P, b, t)) return;
    const float f[4] = {L > 0.f ? o[0] / L : 0.f, L > 0.f ? o[1] / L : 0.f, L > 0.f ? o[2] / L : 0.f,
                        L > 0.f ? o[3] / L : 0.f};
    uint16_t* orow = reinterpret_cast<uint16_t*>(P.out) + o_offset(P, b, t, P.o_sb, P.o_st) + (int64_t)h * P.o_sh;
    *reinterpret_cast<short4_t*>(orow + 16 * mt + 4 * g) = bf16_rne4(f);
    return;
  }
  const int64_t R = row_index(P, b, t, h);
  *reinterpret_cast<float4_t*>(P.ws_acc + (R * P.nsplit + s) * D + 16 * mt + 4 * g) = o;
  if (mt == 0 && g == 0) {
    float* pm = P.ws_ml + (R * P.nsplit + s) * 2;
    pm[0] = M;
    pm[1] = L;
  }
}

template <int D, int BSZ>
__global__ void __launch_bounds__(64 * UNIT_WAVES) __attribute__((amdgpu_waves_per_eu(2)))
attn_unit_kernel(AttnParams P) {
  constexpr int MT = D / 16;
  __shared__ float4_t red_acc[UNIT_WAVES][2 * MT][64];
  __shared__ float red_m[UNIT_WAVES][QTILE], red_l[UNIT_WAVES][QTILE];
  const int nkv = P.kv.n_kv_heads;
  const int64_t e_idx = blockIdx.x / nkv;
  const int hkv = (int)(blockIdx.x - e_idx * nkv);
  if (e_idx >= P.n_items[0]) return;   // uniform over the workgroup
  typedef __attribute__((address_space(4))) const AttnItem ConstItem;   // read-only: scalar loads
  ConstItem* ep = (ConstItem*)(uintptr_t)(P.items + e_idx);
  const int b = ep->b, z = ep->z, s = ep->s, qmax = ep->qmax;
  const int lane = threadIdx.x & 63, l16 = lane & 15;
  const int w = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);   // wave-uniform, in a scalar register
  const int row0 = z * QTILE;
  const int nrows = min(QTILE, P.T * P.G - row0);
  const int* posb = P.pos + (int64_t)b * P.T;
  int rpos[2];
#pragma unroll
  for (int nt = 0; nt < 2; ++nt) {
    const int r = 16 * nt + l16;
    rpos[nt] = (r < nrows) ? posb[(row0 + r) / P.G] : -1;
  }
  const int kbeg = s * P.split;
  const int kend = min(kbeg + P.split, qmax + 1);

  attn_wave_tiles<D, BSZ>(P, b, kbeg, kend, qmax, row0, nrows, rpos, hkv, w, red_acc[w], red_m[w], red_l[w]);
  __syncthreads();

  // fold the waves' partials in wave order; wave w takes the (query half, 16-dim tile) pairs w,
  // w + UNIT_WAVES, ...
  for (int gi = w; gi < 2 * MT; gi += UNIT_WAVES) {
    const int nt = gi / MT, mt = gi - nt * MT;
    const int r = 16 * nt + l16;
    if (r >= nrows) continue;
    float M = -INFINITY, L = 0.f;
    float4_t o = float4_t{0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int v = 0; v < UNIT_WAVES; ++v) {
      float Mn, cM, cm;
      if (!fold_weights(M, red_m[v][r], Mn, cM, cm)) continue;
      L = fold_value(L, cM, red_l[v][r], cm);
      const float4_t a = red_acc[v][gi][lane];
#pragma unroll
      for (int c = 0; c < 4; ++c) o[c] = fold_value(o[c], cM, a[c], cm);
      M = Mn;
    }
    attn_emit<D>(P, b, s, kbeg, hkv, row0 + r, rpos[nt], mt, M, L, o);
  }
}

// Device-coherent accesses to a split unit's published partials: buffer loads and stores with the sc1
// cache policy (coherent at device scope, the encoding agent-scope atomics get), four floats at a time
// where the data allows. Being plain accesses, the compiler issues a wave's loads together; the
// barrier and the arrival count order them against the other half's stores.
constexpr int CPOL_SC1 = 16;
typedef unsigned u32x4 __attribute__((ext_vector_type(4)));
FS_DEVICE __amdgpu_buffer_rsrc_t slot_rsrc(float* base, int bytes) {
  return __builtin_amdgcn_make_buffer_rsrc(base, (short)0, bytes, 0x00020000);
}
FS_DEVICE void st4_dev(__amdgpu_buffer_rsrc_t r, int off, float4_t v) {
  __builtin_amdgcn_raw_buffer_store_b128(__builtin_bit_cast(u32x4, v), r, off, 0, CPOL_SC1);
}
FS_DEVICE void st1_dev(__amdgpu_buffer_rsrc_t r, int off, float v) {
  __builtin_amdgcn_raw_buffer_store_b32(__builtin_bit_cast(unsigned, v), r, off, 0, CPOL_SC1);
}
FS_DEVICE float4_t ld4_dev(__amdgpu_buffer_rsrc_t r, int off) {
  return __builtin_bit_cast(float4_t, __builtin_amdgcn_raw_buffer_load_b128(r, off, 0, CPOL_SC1));
}
FS_DEVICE float ld1_dev(__amdgpu_buffer_rsrc_t r, int off) {
  return __builtin_bit_cast(float, __builtin_amdgcn_raw_buffer_load_b32(r, off, 0, CPOL_SC1));
}

// A unit split in two: workgroup 2u + h (HALF_WAVES waves) builds classes HALF_WAVES*h + w of unit u,
// each with the unit kernel's attn_wave_tiles, so that a call with few units keeps twice as many CUs
// streaming. A row's result is the unit kernel's fold over classes 0..7 in increasing order: half 0
// folds classes 0..3 and publishes that prefix (M, L, O), half 1 publishes its four class partials,
// and the half that arrives second continues the fold through classes 4..7 and emits the rows. The
// arrival is counted (an agent-scope atomic), never awaited; the published values cross XCDs through
// device-coherent accesses.
template <int D, int BSZ>
__global__ void __launch_bounds__(64 * HALF_WAVES) __attribute__((amdgpu_waves_per_eu(2)))
attn_unit_half_kernel(AttnParams P) {
  constexpr int MT = D / 16, NG = 2 * MT / HALF_WAVES;
  constexpr int64_t SLOT = split_slot_floats(D);
  __shared__ float4_t red_acc[HALF_WAVES][2 * MT][64];
  __shared__ float red_m[HALF_WAVES][QTILE], red_l[HALF_WAVES][QTILE];
  __shared__ int sh_last;
  const int nkv = P.kv.n_kv_heads;
  const int64_t unit = blockIdx.x >> 1;
  const int h = blockIdx.x & 1;
  const int64_t e_idx = unit / nkv;
  const int hkv = (int)(unit - e_idx * nkv);
  if (e_idx >= P.n_items[0]) return;   // uniform over the workgroup (and over both halves)
  typedef __attribute__((address_space(4))) const AttnItem ConstItem;
  ConstItem* ep = (ConstItem*)(uintptr_t)(P.items + e_idx);
  const int b = ep->b, z = ep->z, s = ep->s, qmax = ep->qmax;
  const int lane = threadIdx.x & 63, l16 = lane & 15, g = lane >> 4;
  const int w = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int row0 = z * QTILE;
  const int nrows = min(QTILE, P.T * P.G - row0);
  const int* posb = P.pos + (int64_t)b * P.T;
  int rpos[2];
#pragma unroll
  for (int nt = 0; nt < 2; ++nt) {
    const int r = 16 * nt + l16;
    rpos[nt] = (r < nrows) ? posb[(row0 + r) / P.G] : -1;
  }
  const int kbeg = s * P.split;
  const int kend = min(kbeg + P.split, qmax + 1);

  attn_wave_tiles<D, BSZ>(P, b, kbeg, kend, qmax, row0, nrows, rpos, hkv, HALF_WAVES * h + w, red_acc[w], red_m[w],
                          red_l[w]);
  __syncthreads();

  // this unit's published partials, SLOT floats each: slot 0 half 0's prefix, slots 1..4 classes 4..7
  const __amdgpu_buffer_rsrc_t scr =
      slot_rsrc(P.split_ws + unit * SPLIT_SLOTS * SLOT, (int)(SPLIT_SLOTS * SLOT * sizeof(float)));
  auto m_at = [&](int slot, int r) { return (int)((slot * SLOT + r) * sizeof(float)); };
  auto l_at = [&](int slot, int r) { return (int)((slot * SLOT + QTILE + r) * sizeof(float)); };
  auto acc_at = [&](int slot, int gi) { return (int)((slot * SLOT + 2 * QTILE + (gi * 64 + lane) * 4) * sizeof(float)); };
  float Mp[NG], Lp[NG];
  float4_t op[NG];
  if (h == 0) {   // classes 0..3 folded as the unit kernel folds them, then published
#pragma unroll
    for (int j = 0; j < NG; ++j) {
      const int gi = w + HALF_WAVES * j, nt = gi / MT, mt = gi - nt * MT;
      const int r = 16 * nt + l16;
      float M = -INFINITY, L = 0.f;
      float4_t o = float4_t{0.f, 0.f, 0.f, 0.f};
#pragma unroll
      for (int v = 0; v < HALF_WAVES; ++v) {
        float Mn, cM, cm;
        if (!fold_weights(M, red_m[v][r], Mn, cM, cm)) continue;
        L = fold_value(L, cM, red_l[v][r], cm);
        const float4_t a = red_acc[v][gi][lane];
#pragma unroll
        for (int c = 0; c < 4; ++c) o[c] = fold_value(o[c], cM, a[c], cm);
        M = Mn;
      }
      Mp[j] = M;
      Lp[j] = L;
      op[j] = o;
      st4_dev(scr, acc_at(0, gi), o);
      if (mt == 0 && g == 0) {
        st1_dev(scr, m_at(0, r), M);
        st1_dev(scr, l_at(0, r), L);
      }
    }
  } else {   // this wave's class partial, as the unit kernel's LDS holds it
#pragma unroll
    for (int gi = 0; gi < 2 * MT; ++gi) st4_dev(scr, acc_at(1 + w, gi), red_acc[w][gi][lane]);
    if (lane < QTILE) {
      st1_dev(scr, m_at(1 + w, lane), red_m[w][lane]);
      st1_dev(scr, l_at(1 + w, lane), red_l[w][lane]);
    }
  }
  stores_done();
  __syncthreads();   // every wave's published values have completed
  if (threadIdx.x == 0) sh_last = count_in(P.split_cnt + unit, 2u);
  __syncthreads();
  if (!sh_last) return;

  // the unit's second arrival: the fold continues through classes 4..7, then the rows are emitted
  if (h == 0) {
    float4_t a[NG][HALF_WAVES];   // every published value this wave needs, loaded at once
    float m[NG][HALF_WAVES], l[NG][HALF_WAVES];
#pragma unroll
    for (int j = 0; j < NG; ++j) {
      const int gi = w + HALF_WAVES * j, r = 16 * (gi / MT) + l16;
#pragma unroll
      for (int v = 0; v < HALF_WAVES; ++v) {
        a[j][v] = ld4_dev(scr, acc_at(1 + v, gi));
        m[j][v] = ld1_dev(scr, m_at(1 + v, r));
        l[j][v] = ld1_dev(scr, l_at(1 + v, r));
      }
    }
#pragma unroll
    for (int j = 0; j < NG; ++j) {
      const int gi = w + HALF_WAVES * j, nt = gi / MT, mt = gi - nt * MT;
      const int r = 16 * nt + l16;
      float M = Mp[j], L = Lp[j];
      float4_t o = op[j];
#pragma unroll
      for (int v = 0; v < HALF_WAVES; ++v) {
        float Mn, cM, cm;
        if (!fold_weights(M, m[j][v], Mn, cM, cm)) continue;
        L = fold_value(L, cM, l[j][v], cm);
#pragma unroll
        for (int c = 0; c < 4; ++c) o[c] = fold_value(o[c], cM, a[j][v][c], cm);
        M = Mn;
      }
      if (r < nrows) attn_emit<D>(P, b, s, kbeg, hkv, row0 + r, rpos[nt], mt, M, L, o);
    }
  } else {
#pragma unroll
    for (int j = 0; j < NG; ++j) {
      const int gi = w + HALF_WAVES * j, r = 16 * (gi / MT) + l16;
      Mp[j] = ld1_dev(scr, m_at(0, r));
      Lp[j] = ld1_dev(scr, l_at(0, r));
      op[j] = ld4_dev(scr, acc_at(0, gi));
    }
#pragma unroll
    for (int j = 0; j < NG; ++j) {
      const int gi = w + HALF_WAVES * j, nt = gi / MT, mt = gi - nt * MT;
      const int r = 16 * nt + l16;
      float M = Mp[j], L = Lp[j];
      float4_t o = op[j];
#pragma unroll
      for (int v = 0; v < HALF_WAVES; ++v) {
        float Mn, cM, cm;
        if (!fold_weights(M, red_m[v][r], Mn, cM, cm)) continue;
        L = fold_value(L, cM, red_l[v][r], cm);
        const float4_t av = red_acc[v][gi][lane];
#pragma unroll
        for (int c = 0; c < 4; ++c) o[c] = fold_value(o[c], cM, av[c], cm);
        M = Mn;
      }
      if (r < nrows) attn_emit<D>(P, b, s, kbeg, hkv, row0 + r, rpos[nt], mt, M, L, o);
    }
  }
}

// ------------------------------------------------------------------------------------------------
// prefill kernel: one workgroup of PF_WAVES waves per (plan item of PF_WAVES query tiles, KV head)
// ------------------------------------------------------------------------------------------------
// A prompt's queries are many 32-row tiles per row. Here the PF_WAVES tiles of an item (256 query rows:
// wave w owns tile PF_WAVES * item.z + w) share every key and value tile through an LDS ring that
// direct global->LDS copies fill, so a key tile is read from memory once per 256 query rows instead of
// once per 32. Each wave computes, for its own rows, exactly what the unit kernel computes for them:
// the partial of tiles v, v + 8, v + 16, ... (v = 0..7, increasing), with attn_tile, folded in
// increasing v with fold_weights/fold_value. The ring therefore carries the chunk's tiles in that
// order (all tiles t % 8 == 0, then t % 8 == 1, ...), and a wave skips the tiles wholly above its
// furthest query (no-ops for every row of the wave). Output bits equal the unit kernel's.
constexpr int PF_WAVES = 8;      // query tiles (waves) per workgroup
constexpr int PF_TILES = 4;      // 16-key tiles per ring stage
constexpr int PF_NS = 4;         // ring stages (two in flight behind the one awaited)
constexpr int PF_MIN_QTILES = 5; // a call with at least this many query tiles per row takes this kernel

#pragma clang diagnostic push
#pragma clang diagnostic ignored "-Winline-asm"
// One 16-byte copy per lane straight into LDS from sbase + voff (a wave-uniform base in SGPRs and a
// 32-bit unsigned per-lane byte offset; lane l lands at lds + 16 * l, the same base for the whole
// wave). The copy is counted by vmcnt like any vector load; the waits below are explicit.
FS_DEVICE void pf_dma16(const void* sbase, uint32_t voff, uint32_t lds) {
  const uint32_t l = __builtin_amdgcn_readfirstlane(lds);
  asm volatile("s_mov_b32 m0, %2\n\tglobal_load_lds_dwordx4 %0, %1" ::"v"(voff), "s"(sbase), "s"(l) : "memory", "m0");
}
#pragma clang diagnostic pop
template <int N>
FS_DEVICE void pf_wait_vm() {
  asm volatile("s_waitcnt vmcnt(%0)" ::"n"(N) : "memory");
}

// The chunk's tiles in the ring's order: class v = t % 8 in increasing v, increasing t inside a class.
// The tile after t (of a chunk of n tiles) is t + 8, or the next class's first tile (t % 8) + 1.
FS_DEVICE int pf_next_tile(int t, int n) {
  t += 8;
  return t < n ? t : (t & 7) + 1;
}
// The tile at ring position j (0 <= j < n): class v holds the n_v = ceil((n - v) / 8) tiles v, v + 8, ...
FS_DEVICE int pf_ring_tile(int j, int n) {
  int first = 0, t = 0;
#pragma unroll
  for (int v = 0; v < 8; ++v) {
    const int nv = n > v ? ((n - 1 - v) >> 3) + 1 : 0;
    if (j >= first && j < first + nv) t = v + 8 * (j - first);
    first += nv;
  }
  return t;
}

template <int D, int BSZ>
__global__ void __launch_bounds__(64 * PF_WAVES) __attribute__((amdgpu_waves_per_eu(2)))
attn_prefill_kernel(AttnParams P) {
  constexpr int KS = D / 32, MT = D / 16;
  constexpr int TK = 16 * D * 2;                    // bytes of a tile's keys (and of its values)
  constexpr int TB = 2 * TK;                        // a tile in LDS: keys, then values
  constexpr int CPT = TB / 1024;                    // 1 KB copies per tile
  constexpr int CPW = PF_TILES * CPT / PF_WAVES;    // copies per wave per stage
  constexpr int CPR = D / 8;                        // 16-byte chunks per key row
  constexpr int STAGE = PF_TILES * TB;
  static_assert(PF_WAVES % CPT == 0 && CPW >= 1, "every wave copies the same part of its tiles");
  static_assert(PF_NS == 4, "the waits below cover two stages in flight behind the awaited one");
  __shared__ __attribute__((aligned(1024))) char ring[PF_NS * STAGE];
  __shared__ int tbl[MAX_SPLIT / 16 + 1];           // the chunk's physical blocks (-1: unmapped)

  const int nkv = P.kv.n_kv_heads;
  const int64_t e_idx = blockIdx.x / nkv;
  const int hkv = (int)(blockIdx.x - e_idx * nkv);
  if (e_idx >= P.n_items[0]) return;   // uniform over the workgroup
  typedef __attribute__((address_space(4))) const AttnItem ConstItem;
  ConstItem* ep = (ConstItem*)(uintptr_t)(P.items + e_idx);
  const int b = ep->b, zb = ep->z, s = ep->s, qmax_item = ep->qmax;
  const int tid = threadIdx.x, lane = tid & 63, l16 = lane & 15, g = lane >> 4;
  const int w = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int BS = BSZ ? BSZ : P.kv.block_size;
  const int64_t v_dim = BSZ ? BSZ : P.kv.v_dim;   // == block_size (dim-major values)
  const int kbeg = s * P.split;
  const int kend = min(kbeg + P.split, qmax_item + 1);
  const int ntiles = max((kend - kbeg + 15) >> 4, 0);
  const int nst = (ntiles + PF_TILES - 1) / PF_TILES;

  // this wave's query tile: the unit kernel's tile z, with its rows, positions and furthest query
  const int z = zb * PF_WAVES + w;
  const int row0 = z * QTILE;
  const int nrows = min(QTILE, P.T * P.G - row0);   // <= 0: a wave past the last tile (copies only)
  const bool two = nrows > 16;
  const int* posb = P.pos + (int64_t)b * P.T;
  int rpos[2];
#pragma unroll
  for (int nt = 0; nt < 2; ++nt) {
    const int r = 16 * nt + l16;
    rpos[nt] = (r < nrows) ? posb[(row0 + r) / P.G] : -1;
  }
  const int qmax = nrows > 0 ? tile_qmax(P, b, z) : -1;
  const int rmin = rows_min_pos(rpos, nrows);
  const int ntiles_w = nrows > 0 ? min(max((min(kbeg + P.split, qmax + 1) - kbeg + 15) >> 4, 0), ntiles) : 0;

  typedef uint16_t u16;
  const u16* qbase = reinterpret_cast<const u16*>(P.q);
  bf16x8_t qf[2][KS];
#pragma unroll
  for (int nt = 0; nt < 2; ++nt) {
    const int r = row0 + 16 * nt + l16;
    const bool in_tile = nrows > 0 && (16 * nt + l16) < nrows;
    const bool ok = in_tile && token_exists(P, b, r / P.G);
    const int t = ok ? r / P.G : 0;
    const int h = hkv * P.G + (ok ? r - (r / P.G) * P.G : 0);
    const u16* qr = qbase + q_offset(P, b, t) + (int64_t)h * P.q_sh;
#pragma unroll
    for (int ks = 0; ks < KS; ++ks) qf[nt][ks] = ok ? *reinterpret_cast<const bf16x8_t*>(qr + 32 * ks + 8 * g) : bf16x8_t{};
  }

  // the chunk's table entries
  const int blk0 = kbeg / BS;
  const int nblk = ntiles > 0 ? (kbeg + 16 * ntiles - 1) / BS - blk0 + 1 : 0;
  int unmapped = 0;
  for (int i = tid; i < nblk; i += 64 * PF_WAVES) {
    const int blk = blk0 + i;
    int v = blk < P.max_blocks ? P.table[(int64_t)b * P.table_stride + blk] : -1;
    v = (v >= 0 && v < P.kv.num_blocks) ? v : -1;
    unmapped |= v < 0;
    tbl[i] = v;
  }
  // every load above has landed (the copies below are counted by the explicit waits only)
  __builtin_amdgcn_s_waitcnt(0);
  const bool all_mapped = !__syncthreads_or(unmapped);   // (the common case: no lookups per tile)

  // This wave copies part p = w % CPT of every tile it copies (keys for p < CPT/2, else values).
  // LDS layouts (16-byte slots; 16 consecutive slots are read without bank conflicts):
  //  * slot-major keys: row r's 16-byte chunk c at slot r * CPR + (c ^ f(r)), f(r) = r & 15 for 16
  //    chunks per row, (r >> 1) & 7 for 8, so the 16 rows of an MFMA operand read 16 different slots
  //    mod 16; grouped keys: chunk c of row r at slot 16 * c + r, the pool's own order (each copy is
  //    then one contiguous 1 KB of the pool, and an operand's 16 rows are 16 consecutive slots);
  //  * values: dim d's keys 8h .. 8h+7 at slot 2d + (h ^ ((d >> 3) & 1)), so dims d and d + 8 of an
  //    operand read different slots mod 16.
  const int p = w % CPT;
  const bool kpart = p < CPT / 2;
  const bool kgrp = P.kv.k_group != 0;
  const int64_t kgs = key_group_stride(P.kv);
  int64_t src_off;
  {
    const int P16 = (kpart ? p : p - CPT / 2) * 64 + lane;
    if (kpart && kgrp) {
      src_off = (int64_t)(P16 & 15) * 8 + (int64_t)(P16 >> 4) * kgs;
    } else if (kpart) {
      const int row = P16 / CPR, f = CPR == 16 ? (row & 15) : ((row >> 1) & 7);
      const int c = (P16 % CPR) ^ f;
      src_off = (int64_t)row * D + 8 * c;
    } else {
      const int d = P16 >> 1, h = (P16 & 1) ^ ((d >> 3) & 1);
      src_off = (int64_t)d * v_dim + 8 * h;
    }
  }
  // copies read pool_h + (a tile's offset) + coff: the head's base is wave-uniform, the lane's part of
  // a tile lies inside one block (a few KB), so it fits the 32-bit offset of the scalar-base form
  const char* pool_h = reinterpret_cast<const char*>(kpart ? P.kv.k : P.kv.v) +
                       2 * (int64_t)hkv * (kpart ? P.kv.k_head : P.kv.v_head);
  const uint32_t coff = (uint32_t)(2 * src_off);
  const int64_t blk_stride = kpart ? P.kv.k_block : P.kv.v_block;
  const int64_t slot_mul = kpart ? P.kv.k_slot : 1;
  const uint32_t ring0 = (uint32_t)(uintptr_t)ring;
  // this lane's operand reads inside a tile (bytes)
  const int fk = CPR == 16 ? (l16 & 15) : ((l16 >> 1) & 7);
  int koff[KS];
#pragma unroll
  for (int ks = 0; ks < KS; ++ks) koff[ks] = (kgrp ? (4 * ks + g) * 16 + l16 : l16 * CPR + ((4 * ks + g) ^ fk)) * 16;
  const int voff = TK + (2 * l16 + ((g >> 1) ^ ((l16 >> 3) & 1))) * 16 + 8 * (g & 1);

  // Copies walk the ring positions PF_TILES at a time; a position past the last tile copies the last
  // tile again. Lane j holds the byte offset of the tile at ring position 64 * win + j (relative to
  // pool_h), refreshed when a stage enters the next 64 positions, so a copy reads its tile's offset
  // with two lane reads instead of walking the order and the table per copy.
  static_assert(64 % PF_TILES == 0, "a stage's positions lie in one 64-position window");
  uint32_t woff_lo = 0, woff_hi = 0;
  auto refresh = [&](int win) {
    const int t = pf_ring_tile(min(64 * win + lane, ntiles - 1), ntiles);
    const int key0 = kbeg + 16 * t;
    const int bi = key0 / BS;
    const int ph = tbl[bi - blk0];
    const int64_t pb = ph >= 0 ? ph : 0;         // unmapped: block 0, masked in attn_tile
    const uint64_t o = (uint64_t)(2 * (pb * blk_stride + (int64_t)(key0 - bi * BS) * slot_mul));
    woff_lo = (uint32_t)o;
    woff_hi = (uint32_t)(o >> 32);
  };
  auto issue = [&](int k) {
    if ((k & (64 / PF_TILES - 1)) == 0) refresh(k / (64 / PF_TILES));
    const uint32_t base = ring0 + (uint32_t)((k % PF_NS) * STAGE) + (uint32_t)(p * 1024);
#pragma unroll
    for (int i = 0; i < CPW; ++i) {
      const int u = (w + PF_WAVES * i) / CPT;   // the stage's tile this copy fills
      const int j = (PF_TILES * k + u) & 63;
      const uint64_t o = ((uint64_t)(uint32_t)__builtin_amdgcn_readlane((int)woff_hi, j) << 32) |
                         (uint32_t)__builtin_amdgcn_readlane((int)woff_lo, j);
      pf_dma16(pool_h + o, coff, base + (uint32_t)(u * TB));
    }
  };
  auto wait_stages = [&](int later) {
    if (later >= 2) pf_wait_vm<2 * CPW>();
    else if (later == 1) pf_wait_vm<CPW>();
    else pf_wait_vm<0>();
  };

  float4_t acc[MT][2], O[MT][2];
#pragma unroll
  for (int mt = 0; mt < MT; ++mt)
#pragma unroll
    for (int nt = 0; nt < 2; ++nt) {
      acc[mt][nt] = float4_t{0.f, 0.f, 0.f, 0.f};
      O[mt][nt] = float4_t{0.f, 0.f, 0.f, 0.f};
    }
  float m_run[2] = {-INFINITY, -INFINITY}, l_run[2] = {0.f, 0.f};
  float Ms[2] = {-INFINITY, -INFINITY}, Ls[2] = {0.f, 0.f};
  // the finished partial of class v into the row state, then an empty partial for the next class
  auto fold = [&]() {
#pragma unroll
    for (int nt = 0; nt < 2; ++nt) {
      const float l = sum_across_groups(l_run[nt]);
      float Mn, cM, cm;
      if (fold_weights(Ms[nt], m_run[nt], Mn, cM, cm)) {
        Ls[nt] = fold_value(Ls[nt], cM, l, cm);
#pragma unroll
        for (int mt = 0; mt < MT; ++mt)
#pragma unroll
          for (int c = 0; c < 4; ++c) O[mt][nt][c] = fold_value(O[mt][nt][c], cM, acc[mt][nt][c], cm);
        Ms[nt] = Mn;
      }
      m_run[nt] = -INFINITY;
      l_run[nt] = 0.f;
#pragma unroll
      for (int mt = 0; mt < MT; ++mt) acc[mt][nt] = float4_t{0.f, 0.f, 0.f, 0.f};
    }
  };

#pragma unroll
  for (int k = 0; k < PF_NS - 1; ++k)
    if (k < nst) issue(k);
  int rt = 0;   // the tile consumed next
  int cur_v = 0;
  for (int k = 0; k < nst; ++k) {
    wait_stages(min(PF_NS - 2, nst - 1 - k));
    __syncthreads();   // stage k has landed for every wave; stage k-1 is no longer being read
    if (k + PF_NS - 1 < nst) issue(k + PF_NS - 1);
    // the stage's operand addresses, once per stage: each tile's reads add only its constant offset
    const uint32_t st_lds = ring0 + (uint32_t)((k % PF_NS) * STAGE);
    uint32_t kad[KS];
#pragma unroll
    for (int ks = 0; ks < KS; ++ks) kad[ks] = st_lds + (uint32_t)koff[ks];
    const uint32_t vad = st_lds + (uint32_t)voff;
#pragma unroll
    for (int u = 0; u < PF_TILES; ++u) {
      if (k * PF_TILES + u >= ntiles) break;
      const int t = rt;
      rt = pf_next_tile(rt, ntiles);
      if (nrows <= 0) continue;
      if ((t & 7) != cur_v) {   // a new class: fold the last one into the row state
        fold();
        cur_v = t & 7;
      }
      if (t >= ntiles_w) continue;   // wholly above every query of the wave
      typedef __attribute__((address_space(3))) const bf16x8_t LdsK;
      typedef __attribute__((address_space(3))) const short4_t LdsV;
      bf16x8_t kf[KS];
      short4_t vf[MT];
#pragma unroll
      for (int ks = 0; ks < KS; ++ks) kf[ks] = *(LdsK*)(uintptr_t)(kad[ks] + (uint32_t)(u * TB));
#pragma unroll
      for (int mt = 0; mt < MT; ++mt) vf[mt] = *(LdsV*)(uintptr_t)(vad + (uint32_t)(u * TB + mt * 16 * 32));
      const int key0 = kbeg + 16 * t;
      const bool tv = all_mapped || tbl[key0 / BS - blk0] >= 0;
      attn_tile<D, true, true>(kf, vf, key0, tv, qmax, rpos, rmin, two, qf, P.scale_log2, acc, m_run, l_run);
    }
  }
  if (nrows <= 0) return;
  fold();
#pragma unroll
  for (int nt = 0; nt < 2; ++nt) {
    const int r = 16 * nt + l16;
    if (r >= nrows) continue;
#pragma unroll
    for (int mt = 0; mt < MT; ++mt) attn_emit<D>(P, b, s, kbeg, hkv, row0 + r, rpos[nt], mt, Ms[nt], Ls[nt], O[mt][nt]);
  }
}

// ------------------------------------------------------------------------------------------------
// generic kernel (any dtype, head_dim <= 256, any strides and block size)
// ------------------------------------------------------------------------------------------------
template <int DT>
__global__ void __launch_bounds__(64) attn_generic_kernel(AttnParams P) {
  typedef Elem<DT> E;
  typedef typename E::T T_;
  __shared__ float qs[256];
  __shared__ float ps[64];
  const int lane = threadIdx.x;
  const int s = blockIdx.y;
  const int64_t R = blockIdx.x;  // (b, t, h)
  const int h = (int)(R % P.H);
  const int bt = (int)(R / P.H);
  const int b = bt / P.T, t = bt - b * P.T;
  const int pos = P.pos[bt];
  const int kbeg = s * P.split;
  if (pos < kbeg) return;
  const int kend = min(kbeg + P.split, pos + 1);
  const int D = P.kv.head_dim, BS = P.kv.block_size;
  const int hkv = h / P.G;
  const T_* qrow = reinterpret_cast<const T_*>(P.q) + q_offset(P, b, t) + (int64_t)h * P.q_sh;
  for (int d = lane; d < D; d += 64) qs[d] = E::load(qrow, d);
  __syncthreads();
  const T_* kp = reinterpret_cast<const T_*>(P.kv.k);
  const T_* vp = reinterpret_cast<const T_*>(P.kv.v);
  const int32_t* trow = P.table + (int64_t)b * P.table_stride;

  float m_run = -INFINITY, l_run = 0.f;
  float acc[4] = {0.f, 0.f, 0.f, 0.f};
  for (int j0 = kbeg; j0 < kend; j0 += 64) {
    const int j = j0 + lane;
    float sv = -INFINITY;
    if (j < kend) {
      const int bi = j / BS;
      const int64_t blk = (bi < P.max_blocks) ? trow[bi] : -1;
      if (blk >= 0 && blk < P.kv.num_blocks) {
        const T_* kr = kp + blk * P.kv.k_block + hkv * P.kv.k_head + (int64_t)(j - bi * BS) * P.kv.k_slot;
        float dot = 0.f;
        for (int d = 0; d < D; ++d) dot = fmaf(qs[d], E::load(kr, key_dim_off(P.kv, d)), dot);
        sv = dot * P.scale_log2;
      }
    }
    const float m_new = fmaxf(m_run, wave_max(sv));
    const float alpha = (m_new == -INFINITY) ? 1.f : exp2f(m_run - m_new);
    const float p = (sv == -INFINITY) ? 0.f : exp2f(sv - m_new);
    l_run = l_run * alpha + wave_sum(p);
    m_run = m_new;
    __syncthreads();
    ps[lane] = p;
    __syncthreads();
    const int nj = min(64, kend - j0);
#pragma unroll
    for (int c = 0; c < 4; ++c) {
      const int d = lane + 64 * c;
      if (d >= D) break;
      float a = acc[c] * alpha;
      for (int jj = 0; jj < nj; ++jj) {
        const float pj = ps[jj];
        if (pj == 0.f) continue;  // masked, invalid-block or underflowed key: adds an exact zero
        const int jk = j0 + jj;
        const int bi = jk / BS;
        const int64_t blk = trow[bi];
        const T_* vr = vp + blk * P.kv.v_block + hkv * P.kv.v_head + (int64_t)(jk - bi * BS) * P.kv.v_slot;
        a = fmaf(pj, E::load(vr, (int64_t)d * P.kv.v_dim), a);
      }
      acc[c] = a;
    }
  }
  float* pa = P.ws_acc + (R * P.nsplit + s) * D;
  for (int c = 0; c < 4; ++c) {
    const int d = lane + 64 * c;
    if (d < D) pa[d] = acc[c];
  }
  if (lane == 0) {
    float* pm = P.ws_ml + (R * P.nsplit + s) * 2;
    pm[0] = m_run;
    pm[1] = l_run;
  }
}

// ------------------------------------------------------------------------------------------------
// combine: out[b,t,h,:] = sum_s 2^(m_s - M) acc_s / sum_s 2^(m_s - M) l_s, chunks in increasing order
// ------------------------------------------------------------------------------------------------
constexpr int COMBINE_ROWS = 4;   // rows (waves) per combine workgroup

template <int DT>
__global__ void __launch_bounds__(64 * COMBINE_ROWS) attn_combine_kernel(AttnParams P, void* out, int64_t o_sb,
                                                                         int64_t o_st, int64_t o_sh) {
  typedef Elem<DT> E;
  typedef typename E::T T_;
  const int lane = threadIdx.x & 63;
  const int64_t R = (int64_t)blockIdx.x * COMBINE_ROWS + (threadIdx.x >> 6);
  if (R >= (int64_t)P.B * P.T * P.H) return;
  const int h = (int)(R % P.H);
  const int bt = (int)(R / P.H);
  const int b = bt / P.T, t = bt - b * P.T;
  const int pos = P.pos[bt];
  if (P.direct && (pos < P.split || P.nsplit == 1)) return;   // written by its chunk's workgroup
  if (!token_exists(P, b, t)) return;
  const int D = P.kv.head_dim;
  T_* orow = reinterpret_cast<T_*>(out) + o_offset(P, b, t, o_sb, o_st) + (int64_t)h * o_sh;
  if (pos < 0) {
    for (int d = lane; d < D; d += 64) E::store(orow, d, 0.f);
    return;
  }
  const int ns = min(pos / P.split + 1, P.nsplit);  // keys past the table were never visible
  const float* ml = P.ws_ml + R * P.nsplit * 2;
  const float* pa = P.ws_acc + R * P.nsplit * D;
  float M = -INFINITY;
  for (int s = lane; s < ns; s += 64) M = fmaxf(M, ml[2 * s]);
  M = wave_max(M);
  // Chunk s's weight and weighted sum live in lane s % 64; the partial rows are loaded eight chunks
  // at a time and summed in increasing chunk order.
  float L = 0.f;
  float acc[4] = {0.f, 0.f, 0.f, 0.f};
  for (int s0 = 0; s0 < ns; s0 += 64) {
    float w = 0.f, lw = 0.f;
    if (s0 + lane < ns) {
      const float ms = ml[2 * (s0 + lane)];
      w = (ms == -INFINITY) ? 0.f : exp2f(ms - M);
      lw = w * ml[2 * (s0 + lane) + 1];
    }
    const int n = min(64, ns - s0);
    for (int j = 0; j < n; j += 8) {
      float v[8][4];
#pragma unroll
      for (int jj = 0; jj < 8; ++jj)
#pragma unroll
        for (int c = 0; c < 4; ++c) {
          const int d = lane + 64 * c;
          v[jj][c] = (j + jj < n && d < D) ? pa[(int64_t)(s0 + j + jj) * D + d] : 0.f;
        }
#pragma unroll
      for (int jj = 0; jj < 8; ++jj) {
        if (j + jj < n) {
          const float wj = __builtin_amdgcn_readlane(__float_as_int(w), j + jj);
          L += __int_as_float(__builtin_amdgcn_readlane(__float_as_int(lw), j + jj));
#pragma unroll
          for (int c = 0; c < 4; ++c) acc[c] += __int_as_float(wj) * v[jj][c];
        }
      }
    }
  }
#pragma unroll
  for (int c = 0; c < 4; ++c) {
    const int d = lane + 64 * c;
    if (d < D) E::store(orow, d, L > 0.f ? acc[c] / L : 0.f);
  }
}

bool mfma_eligible(const fs_kv_layout& kv, const void* q, int64_t q_sb, int64_t q_st, int64_t q_sh) {
  if (kv.dtype != FS_BF16) return false;
  if (kv.head_dim != 64 && kv.head_dim != 128) return false;
  if (kv.block_size % 16 != 0) return false;  // a 16-key tile never straddles two blocks
  if (kv.k_dim != 1 || kv.v_slot != 1 || kv.v_dim != kv.block_size) return false;
  const bool slot_major = kv.k_group == 0 && kv.k_slot == kv.head_dim;
  const bool grouped = kv.k_group == 8 * (int64_t)kv.block_size && kv.k_slot == 8;
  if (!slot_major && !grouped) return false;
  if (kv.k_block % 8 || kv.k_head % 8 || kv.v_block % 8 || kv.v_head % 8) return false;
  if ((reinterpret_cast<uintptr_t>(kv.k) | reinterpret_cast<uintptr_t>(kv.v) | reinterpret_cast<uintptr_t>(q)) & 15)
    return false;
  if (q_sb % 8 || q_st % 8 || q_sh % 8) return false;
  return true;
}

// Keys per chunk. The generic kernel uses 512. The MFMA path uses FS_ATTN_SPLIT (default 16384 =
// MAX_SPLIT; a multiple of 64 in [256, MAX_SPLIT]), read once: it must stay fixed for the life of the
// process, since the chunk boundaries decide the rounding of every output. A large chunk keeps batched
// rows of up to 16K keys in one workgroup per KV head (no partials, no combine); few rows of much
// longer contexts spread over more workgroups with a smaller one.
constexpr int GENERIC_SPLIT = 512;

int attn_split() {
  static const int split = [] {
    const char* e = getenv("FS_ATTN_SPLIT");
    int v = e ? atoi(e) : MAX_SPLIT;
    if (v < 256 || v > MAX_SPLIT || v % 64) v = MAX_SPLIT;
    return v;
  }();
  return split;
}

int64_t nsplit_for(int32_t max_blocks, int32_t block_size, int split) {
  const int64_t S = (int64_t)max_blocks * block_size;
  return (S + split - 1) / split;
}

// Upper bound of the plan's length: every (row, query tile, chunk), at the smallest chunk size.
int64_t max_items(int32_t B, int32_t T, int32_t n_heads, int32_t max_blocks, int32_t block_size, int split) {
  const int64_t qtiles = ((int64_t)T * n_heads + QTILE - 1) / QTILE;   // n_heads bounds the group size
  return (int64_t)B * qtiles * nsplit_for(max_blocks, block_size, split);
}

int min_split() { return attn_split() < GENERIC_SPLIT ? attn_split() : GENERIC_SPLIT; }

// Bytes of the split units' published partials for calls of at most `units` units (KV heads never
// outnumber query heads, so items x n_heads bounds the units).
int64_t split_bytes(int64_t units, int32_t head_dim) {
  return (units < SPLIT_UNITS_MAX ? units : (int64_t)SPLIT_UNITS_MAX) * SPLIT_SLOTS * split_slot_floats(head_dim) *
         (int64_t)sizeof(float);
}

}  // namespace

extern "C" int32_t fs_paged_attention_split(void) { return attn_split(); }

extern "C" int64_t fs_paged_attention_workspace_size(int32_t B, int32_t T, int32_t n_heads, int32_t head_dim,
                                                     int32_t max_blocks, int32_t block_size) {
  if (B <= 0 || T <= 0 || n_heads <= 0 || head_dim <= 0 || max_blocks <= 0 || block_size <= 0) return 0;
  const int64_t rows = (int64_t)B * T * n_heads;
  const int64_t ns = nsplit_for(max_blocks, block_size, min_split());
  const int64_t items = max_items(B, T, n_heads, max_blocks, block_size, min_split());
  const int64_t list = (items * (int64_t)sizeof(AttnItem) + 255) / 256 * 256;
  const int64_t partials = (rows * ns * (head_dim + 2) * (int64_t)sizeof(float) + 255) / 256 * 256;
  return WS_HEADER + list + partials + split_bytes(items * n_heads, head_dim) + 256;
}

namespace {
// What the work plan of a call depends on besides the contents of its positions: a call that asks to
// reuse the plan already in its workspace skips the plan kernel only when all of these match the call
// that wrote it (on this host thread); the caller vouches that the positions hold the same values.
struct PlanKey {
  const void* ws = nullptr;
  const int32_t* pos = nullptr;
  const int32_t* row_start = nullptr;
  hipStream_t stream = nullptr;
  int32_t B = 0, T = 0, G = 0, split = 0, nsplit = 0, zgroup = 0;
  bool direct = false;
  bool operator==(const PlanKey& o) const {
    return ws == o.ws && pos == o.pos && row_start == o.row_start && stream == o.stream && B == o.B && T == o.T &&
           G == o.G && split == o.split && nsplit == o.nsplit && direct == o.direct && zgroup == o.zgroup;
  }
};
thread_local PlanKey last_plan;

int paged_attention(const void* q, int64_t q_sb, int64_t q_st, int64_t q_sh, const fs_kv_layout* kv,
                    const int32_t* block_tables, int64_t table_stride, int32_t max_blocks, const int32_t* positions,
                    const int32_t* row_start, int32_t B, int32_t T, int32_t n_heads, float scale, void* out,
                    int64_t o_sb, int64_t o_st, int64_t o_sh, void* workspace, int64_t workspace_bytes,
                    void* stream, bool reuse_plan) {
  FS_CHECK_ARG(kv != nullptr && kv->k && kv->v, "paged_attention: null pool");
  FS_CHECK_ARG(q && block_tables && positions && out && workspace, "paged_attention: null pointer");
  FS_CHECK_ARG(B > 0 && T > 0, "paged_attention: B %d T %d", B, T);
  FS_CHECK_ARG(kv->n_kv_heads > 0 && n_heads > 0 && n_heads % kv->n_kv_heads == 0,
               "paged_attention: n_heads %d, n_kv_heads %d", n_heads, kv->n_kv_heads);
  FS_CHECK_ARG(kv->head_dim > 0 && kv->head_dim <= 256, "paged_attention: head_dim %d (max 256)", kv->head_dim);
  FS_CHECK_ARG(kv->block_size > 0 && max_blocks > 0 && table_stride >= max_blocks,
               "paged_attention: block_size %d max_blocks %d", kv->block_size, max_blocks);
  FS_CHECK_ARG(kv->num_blocks > 0, "paged_attention: num_blocks");
  FS_CHECK_ARG(kv->dtype == FS_F32 || kv->dtype == FS_BF16 || kv->dtype == FS_F16, "paged_attention: dtype %d",
               kv->dtype);
  FS_CHECK_ARG(kv->k_group == 0 || (kv->k_group > 0 && kv->k_dim == 1 && kv->head_dim % 8 == 0),
               "paged_attention: grouped keys need k_group > 0, k_dim == 1 and head_dim %% 8 == 0");
  const int64_t need = fs_paged_attention_workspace_size(B, T, n_heads, kv->head_dim, max_blocks, kv->block_size);
  FS_CHECK_ARG(workspace_bytes >= need, "paged_attention: workspace %lld < %lld bytes", (long long)workspace_bytes,
               (long long)need);
  FS_CHECK_ARG((reinterpret_cast<uintptr_t>(workspace) & 255) == 0, "paged_attention: workspace not 256-aligned");

  AttnParams P;
  P.q = q;
  P.q_sb = q_sb;
  P.q_st = q_st;
  P.q_sh = q_sh;
  P.kv = *kv;
  P.table = block_tables;
  P.table_stride = table_stride;
  P.max_blocks = max_blocks;
  P.pos = positions;
  P.B = B;
  P.T = T;
  P.H = n_heads;
  P.G = n_heads / kv->n_kv_heads;
  P.scale_log2 = scale * LOG2E;
  const bool mfma = mfma_eligible(*kv, q, q_sb, q_st, q_sh);
  P.split = mfma ? attn_split() : GENERIC_SPLIT;
  P.nsplit = (int32_t)nsplit_for(max_blocks, kv->block_size, P.split);
  const int64_t rows = (int64_t)B * T * n_heads;
  char* ws = reinterpret_cast<char*>(workspace);
  const int64_t items = max_items(B, T, n_heads, max_blocks, kv->block_size, min_split());
  const int64_t list = (items * (int64_t)sizeof(AttnItem) + 255) / 256 * 256;
  const int64_t ns_ws = nsplit_for(max_blocks, kv->block_size, min_split());   // >= P.nsplit
  const int64_t partials = (rows * ns_ws * (kv->head_dim + 2) * (int64_t)sizeof(float) + 255) / 256 * 256;
  P.n_items = reinterpret_cast<int32_t*>(ws);
  P.split_cnt = reinterpret_cast<unsigned*>(ws + WS_COUNTERS);
  P.items = reinterpret_cast<AttnItem*>(ws + WS_HEADER);
  P.ws_acc = reinterpret_cast<float*>(ws + WS_HEADER + list);
  P.ws_ml = P.ws_acc + rows * P.nsplit * kv->head_dim;
  P.split_ws = reinterpret_cast<float*>(ws + WS_HEADER + list + partials);
  // direct outputs are stored 4 bf16 at a time
  P.direct = mfma && (reinterpret_cast<uintptr_t>(out) & 7) == 0 && o_sb % 4 == 0 && o_st % 4 == 0 && o_sh % 4 == 0;
  P.out = out;
  P.o_sb = o_sb;
  P.o_st = o_st;
  P.o_sh = o_sh;
  P.row_start = row_start;
  const int64_t qtiles = ((int64_t)T * P.G + QTILE - 1) / QTILE;
  // many query tiles per row (a prompt): groups of PF_WAVES tiles share their key/value reads
  const bool prefill = mfma && qtiles >= PF_MIN_QTILES;
  P.zgroup = prefill ? PF_WAVES : 1;

  hipStream_t st = fs::as_stream(stream);
  if (mfma) {
    const bool bs16 = kv->block_size == 16;
    // one workgroup per (plan item, KV head); items past the plan's length exit at once
    const int64_t units = (int64_t)B * ((qtiles + P.zgroup - 1) / P.zgroup) * P.nsplit * kv->n_kv_heads;
    FS_CHECK_ARG(units < 0x7fffffff, "paged_attention: %lld work units", (long long)units);
    PlanKey key;
    key.ws = workspace;
    key.pos = positions;
    key.row_start = row_start;
    key.stream = st;
    key.B = B;
    key.T = T;
    key.G = P.G;
    key.split = P.split;
    key.nsplit = P.nsplit;
    key.direct = P.direct;
    key.zgroup = P.zgroup;
    if (!(reuse_plan && last_plan == key)) attn_plan_kernel<<<1, PLAN_THREADS, 0, st>>>(P);
    last_plan = key;
    const unsigned grid = (unsigned)units;
    if (prefill) {
      const unsigned threads = 64 * PF_WAVES;
      if (kv->head_dim == 128) {
        if (bs16) attn_prefill_kernel<128, 16><<<grid, threads, 0, st>>>(P);
        else attn_prefill_kernel<128, 0><<<grid, threads, 0, st>>>(P);
      } else {
        if (bs16) attn_prefill_kernel<64, 16><<<grid, threads, 0, st>>>(P);
        else attn_prefill_kernel<64, 0><<<grid, threads, 0, st>>>(P);
      }
    } else if (units <= SPLIT_UNITS_MAX && (int64_t)max_blocks * kv->block_size >= SPLIT_MIN_KEYS) {
      // few, possibly long units: two workgroups each, to keep more CUs reading
      const unsigned threads = 64 * HALF_WAVES;
      if (kv->head_dim == 128) {
        if (bs16) attn_unit_half_kernel<128, 16><<<2 * grid, threads, 0, st>>>(P);
        else attn_unit_half_kernel<128, 0><<<2 * grid, threads, 0, st>>>(P);
      } else {
        if (bs16) attn_unit_half_kernel<64, 16><<<2 * grid, threads, 0, st>>>(P);
        else attn_unit_half_kernel<64, 0><<<2 * grid, threads, 0, st>>>(P);
      }
    } else {
      const unsigned threads = 64 * UNIT_WAVES;
      if (kv->head_dim == 128) {
        if (bs16) attn_unit_kernel<128, 16><<<grid, threads, 0, st>>>(P);
        else attn_unit_kernel<128, 0><<<grid, threads, 0, st>>>(P);
      } else {
        if (bs16) attn_unit_kernel<64, 16><<<grid, threads, 0, st>>>(P);
        else attn_unit_kernel<64, 0><<<grid, threads, 0, st>>>(P);
      }
    }
  } else {
    last_plan = PlanKey{};   // no plan on this path
    dim3 grid((unsigned)rows, (unsigned)P.nsplit);
    switch (kv->dtype) {
      case FS_F32: attn_generic_kernel<FS_F32><<<grid, 64, 0, st>>>(P); break;
      case FS_BF16: attn_generic_kernel<FS_BF16><<<grid, 64, 0, st>>>(P); break;
      default: attn_generic_kernel<FS_F16><<<grid, 64, 0, st>>>(P); break;
    }
  }
  if (int e = fs::launch_status("paged_attention")) return e;
  if (P.direct && P.nsplit == 1) return 0;   // every query sees one chunk: all outputs are written
  dim3 cgrid((unsigned)((rows + COMBINE_ROWS - 1) / COMBINE_ROWS));
  switch (kv->dtype) {
    case FS_F32: attn_combine_kernel<FS_F32><<<cgrid, 64 * COMBINE_ROWS, 0, st>>>(P, out, o_sb, o_st, o_sh); break;
    case FS_BF16: attn_combine_kernel<FS_BF16><<<cgrid, 64 * COMBINE_ROWS, 0, st>>>(P, out, o_sb, o_st, o_sh); break;
    default: attn_combine_kernel<FS_F16><<<cgrid, 64 * COMBINE_ROWS, 0, st>>>(P, out, o_sb, o_st, o_sh); break;
  }
  return fs::launch_status("paged_attention_combine");
}
}  // namespace

extern "C" int fs_paged_attention(const void* q, int64_t q_sb, int64_t q_st, int64_t q_sh, const fs_kv_layout* kv,
                                  const int32_t* block_tables, int64_t table_stride, int32_t max_blocks,
                                  const int32_t* positions, int32_t B, int32_t T, int32_t n_heads, float scale,
                                  void* out, int64_t o_sb, int64_t o_st, int64_t o_sh, void* workspace,
                                  int64_t workspace_bytes, void* stream) {
  return paged_attention(q, q_sb, q_st, q_sh, kv, block_tables, table_stride, max_blocks, positions, nullptr, B, T,
                         n_heads, scale, out, o_sb, o_st, o_sh, workspace, workspace_bytes, stream, false);
}

extern "C" int fs_paged_attention_reuse_plan(const void* q, int64_t q_sb, int64_t q_st, int64_t q_sh,
                                             const fs_kv_layout* kv, const int32_t* block_tables,
                                             int64_t table_stride, int32_t max_blocks, const int32_t* positions,
                                             int32_t B, int32_t T, int32_t n_heads, float scale, void* out,
                                             int64_t o_sb, int64_t o_st, int64_t o_sh, void* workspace,
                                             int64_t workspace_bytes, void* stream) {
  return paged_attention(q, q_sb, q_st, q_sh, kv, block_tables, table_stride, max_blocks, positions, nullptr, B, T,
                         n_heads, scale, out, o_sb, o_st, o_sh, workspace, workspace_bytes, stream, true);
}

extern "C" int fs_paged_attention_varlen(const void* q, int64_t q_st, int64_t q_sh, const fs_kv_layout* kv,
                                         const int32_t* block_tables, int64_t table_stride, int32_t max_blocks,
                                         const int32_t* positions, const int32_t* cu_seqlens, int32_t S,
                                         int32_t T, int32_t n_heads, float scale, void* out, int64_t o_st,
                                         int64_t o_sh, void* workspace, int64_t workspace_bytes, void* stream) {
  FS_CHECK_ARG(cu_seqlens, "paged_attention_varlen: null cu_seqlens");
  return paged_attention(q, 0, q_st, q_sh, kv, block_tables, table_stride, max_blocks, positions, cu_seqlens, S, T,
                         n_heads, scale, out, 0, o_st, o_sh, workspace, workspace_bytes, stream, false);
}

extern "C" int fs_paged_attention_varlen_reuse_plan(const void* q, int64_t q_st, int64_t q_sh,
                                                    const fs_kv_layout* kv, const int32_t* block_tables,
                                                    int64_t table_stride, int32_t max_blocks,
                                                    const int32_t* positions, const int32_t* cu_seqlens, int32_t S,
                                                    int32_t T, int32_t n_heads, float scale, void* out,
                                                    int64_t o_st, int64_t o_sh, void* workspace,
                                                    int64_t workspace_bytes, void* stream) {
  FS_CHECK_ARG(cu_seqlens, "paged_attention_varlen: null cu_seqlens");
  return paged_attention(q, 0, q_st, q_sh, kv, block_tables, table_stride, max_blocks, positions, cu_seqlens, S, T,
                         n_heads, scale, out, 0, o_st, o_sh, workspace, workspace_bytes, stream, true);
}
