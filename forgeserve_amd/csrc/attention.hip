// Paged causal GQA attention for the verify pass (T = k+1 queries per row), 1-token decode and
// prefill, reading keys/values straight from the block pool.
//
// Reference: paged.py:80-81 (gather every table block) + model.py:70-76 (repeat_interleave GQA,
// key_pos <= query_pos mask, scaled_dot_product_attention with scale 1/sqrt(D)).
//
// Work split (both kernels): the keys of a row are cut into fixed chunks of `split` absolute positions
// (512 unless FS_ATTN_SPLIT says otherwise; fixed for the life of the process); chunk s covers keys
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

#include <mutex>

#include "common.h"

namespace {

constexpr int QTILE = 32;            // query rows per MFMA wave
constexpr int MAX_HEADS_PER_WG = 8;  // waves (KV heads) per MFMA workgroup, at most
constexpr int PLAN_THREADS = 256;
constexpr int64_t WS_HEADER = 256;    // workspace: item count, then the item list, then the partials
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
  int32_t split;                     // keys per chunk: a multiple of 16, at most 512
  struct AttnItem* items;            // MFMA path: the work list written by attn_plan_kernel
  int32_t* n_items;                  // its length
};

// Reductions over the four 16-lane groups of a wave (lanes l, l^16, l^32, l^48) with the gfx950
// row swaps: permlane16_swap of (x, x) yields {rows 0,0,2,2 ; rows 1,1,3,3} of x, permlane32_swap
// yields {lanes 0-31 twice ; lanes 32-63 twice}. Both steps are symmetric, so every lane ends with
// the same value, and the sum adds (g0 + g1) + (g2 + g3) in every lane.
FS_DEVICE float max_across_groups(float x) {
  auto a = __builtin_amdgcn_permlane16_swap(__float_as_uint(x), __float_as_uint(x), false, false);
  x = fmaxf(__uint_as_float(a[0]), __uint_as_float(a[1]));
  auto b = __builtin_amdgcn_permlane32_swap(__float_as_uint(x), __float_as_uint(x), false, false);
  return fmaxf(__uint_as_float(b[0]), __uint_as_float(b[1]));
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

// ------------------------------------------------------------------------------------------------
// work plan: the (query tile, chunk) items that hold visible keys
// ------------------------------------------------------------------------------------------------
struct AttnItem {
  int32_t b, z, s, qmax;   // batch row, query tile, chunk, furthest query position of the tile
};

FS_DEVICE int tile_qmax(const AttnParams& P, int b, int z) {
  const int row0 = z * QTILE;
  const int nrows = min(QTILE, P.T * P.G - row0);
  const int t0 = row0 / P.G, t1 = (row0 + nrows - 1) / P.G;
  const int* posb = P.pos + (int64_t)b * P.T;
  int q = -1;
  for (int t = t0; t <= t1; ++t) q = max(q, posb[t]);
  return q;
}

FS_DEVICE int tile_chunks(const AttnParams& P, int qmax) { return qmax < 0 ? 0 : min(qmax / P.split + 1, P.nsplit); }

// One workgroup lists every item: first the chunks that lie wholly below their tile's furthest
// query (the full chunks), tile by tile, then the last chunk of each tile. The shorter last chunks
// thus make up the attention kernel's final round, where they even out the finish.
__global__ void __launch_bounds__(PLAN_THREADS) attn_plan_kernel(AttnParams P) {
  __shared__ int sa[PLAN_THREADS], sb[PLAN_THREADS];
  const int tid = threadIdx.x;
  const int qtiles = (P.T * P.G + QTILE - 1) / QTILE;
  const int U = P.B * qtiles;
  int nf = 0;
  for (int u = tid; u < U; u += PLAN_THREADS) nf += max(tile_chunks(P, tile_qmax(P, u / qtiles, u % qtiles)) - 1, 0);
  sa[tid] = nf;
  __syncthreads();
  for (int off = PLAN_THREADS / 2; off > 0; off >>= 1) {
    if (tid < off) sa[tid] += sa[tid + off];
    __syncthreads();
  }
  const int n_full = sa[0];
  __syncthreads();
  int base_full = 0, base_last = 0;
  for (int u0 = 0; u0 < U; u0 += PLAN_THREADS) {
    const int u = u0 + tid;
    int b = 0, z = 0, qm = -1, nch = 0;
    if (u < U) {
      b = u / qtiles;
      z = u - b * qtiles;
      qm = tile_qmax(P, b, z);
      nch = tile_chunks(P, qm);
    }
    const int f = max(nch - 1, 0), l = nch > 0 ? 1 : 0;
    sa[tid] = f;
    sb[tid] = l;
    __syncthreads();
    for (int off = 1; off < PLAN_THREADS; off <<= 1) {   // inclusive scans
      const int xa = tid >= off ? sa[tid - off] : 0;
      const int xb = tid >= off ? sb[tid - off] : 0;
      __syncthreads();
      sa[tid] += xa;
      sb[tid] += xb;
      __syncthreads();
    }
    const int ef = base_full + sa[tid] - f, el = n_full + base_last + sb[tid] - l;
    for (int c = 0; c < f; ++c) P.items[ef + c] = AttnItem{b, z, c, qm};
    if (l) P.items[el] = AttnItem{b, z, nch - 1, qm};
    base_full += sa[PLAN_THREADS - 1];
    base_last += sb[PLAN_THREADS - 1];
    __syncthreads();
  }
  if (tid == 0) P.n_items[0] = n_full + base_last;
}

// ------------------------------------------------------------------------------------------------
// MFMA kernel (bf16)
// ------------------------------------------------------------------------------------------------
// What one wave needs of an item before its first tile load.
struct ItemRegs {
  int b, z, s, qmax;     // wave-uniform
  int rpos[2];           // positions of the lane's two query rows (row = 16*nt + lane%16), -1: none
  int phys;              // lane i: table entry of the chunk's i-th block (-1 past the table)
};

template <int BSZ>
FS_DEVICE void fetch_item(const AttnParams& P, int64_t e_idx, ItemRegs& it) {
  // the list is read-only here: a constant-address-space load keeps it on the scalar unit
  typedef __attribute__((address_space(4))) const AttnItem ConstItem;
  ConstItem* ep = (ConstItem*)(uintptr_t)(P.items + e_idx);
  const AttnItem e{ep->b, ep->z, ep->s, ep->qmax};
  it.b = e.b;
  it.z = e.z;
  it.s = e.s;
  it.qmax = e.qmax;
  const int lane = threadIdx.x & 63, l16 = lane & 15;
  const int row0 = e.z * QTILE;
  const int nrows = min(QTILE, P.T * P.G - row0);
  const int* posb = P.pos + (int64_t)e.b * P.T;
#pragma unroll
  for (int nt = 0; nt < 2; ++nt) {
    const int r = 16 * nt + l16;
    it.rpos[nt] = (r < nrows) ? posb[(row0 + r) / P.G] : -1;
  }
  const int BS = BSZ ? BSZ : P.kv.block_size;
  const int kbeg = e.s * P.split;
  const int kend = min(kbeg + P.split, e.qmax + 1);
  const int first_blk = kbeg / BS;
  const int nblk = (kend - 1) / BS - first_blk + 1;   // <= split/16 + 1 <= 33 lanes
  it.phys = -1;   // raw table entry, checked where it is used so that nothing waits for it here
  if (lane < nblk && first_blk + lane < P.max_blocks) it.phys = P.table[(int64_t)e.b * P.table_stride + first_blk + lane];
}

// One item for one wave: chunk it.s of batch row it.b, KV head hkv, query tile it.z. `next` runs
// once, three tiles before the end (it takes and fetches the wave's next item).
template <int D, int BSZ, class F>
__device__ __attribute__((always_inline)) inline void attn_mfma_item(const AttnParams& P, const ItemRegs& it,
                                                                     int hkv, F&& next) {
  constexpr int KS = D / 32;   // k-steps of the QK^T product
  constexpr int MT = D / 16;   // 16-dim tiles of the PV product
  const int lane = threadIdx.x & 63;
  const int l16 = lane & 15, g = lane >> 4;
  const int b = it.b, s = it.s, qmax = it.qmax;
  const int row0 = it.z * QTILE;
  const int nrows = min(QTILE, P.T * P.G - row0);
  const int rpos[2] = {it.rpos[0], it.rpos[1]};
  const int my_phys = it.phys;
  const int kbeg = s * P.split;
  if (qmax < kbeg) return;  // not listed by the plan; kept as a guard
  const int kend = min(kbeg + P.split, qmax + 1);
  const int ntiles = (kend - kbeg + 15) >> 4;
  const bool two = nrows > 16;
  const int BS = BSZ ? BSZ : P.kv.block_size;
  const int64_t v_dim = BSZ ? BSZ : P.kv.v_dim;   // == block_size (dim-major values)
  const int first_blk = kbeg / BS;

  typedef uint16_t u16;
  const u16* kpool = reinterpret_cast<const u16*>(P.kv.k);
  const u16* vpool = reinterpret_cast<const u16*>(P.kv.v);
  const int64_t k_head_off = (int64_t)hkv * P.kv.k_head;
  const int64_t v_head_off = (int64_t)hkv * P.kv.v_head;

  // Three tile buffers in registers: while tile t is consumed, tiles t+1 and t+2 are in flight.
  // Every load is unconditional (a prefetch past the end re-reads the last tile, an unmapped block
  // reads block 0 and is masked in consume) so that each wait before a consume counts exactly the
  // loads issued after that tile, on every path through the loop.
  bf16x8_t kb0[KS], kb1[KS], kb2[KS];
  short4_t vb0[MT], vb1[MT], vb2[MT];

  auto block_of = [&](int j0) {   // physical block holding key j0, -1 when unmapped
    const int v = __builtin_amdgcn_readlane(my_phys, j0 / BS - first_blk);
    return (v >= 0 && v < P.kv.num_blocks) ? v : -1;
  };

  auto load_tile = [&](int kt, bf16x8_t (&kd)[KS], short4_t (&vd)[MT]) {
    const int j0 = kbeg + 16 * min(kt, ntiles - 1);
    const int phys = block_of(j0);
    const int64_t pb = phys >= 0 ? phys : 0;
    const int slot0 = j0 - (j0 / BS) * BS;
    const u16* kt_ = kpool + pb * P.kv.k_block + k_head_off + (int64_t)(slot0 + l16) * D;
#pragma unroll
    for (int ks = 0; ks < KS; ++ks)   // read once per launch: nontemporal
      kd[ks] = __builtin_nontemporal_load(reinterpret_cast<const bf16x8_t*>(kt_ + 32 * ks + 8 * g));
    const u16* vt_ = vpool + pb * P.kv.v_block + v_head_off + slot0 + 4 * g;
#pragma unroll
    for (int mt = 0; mt < MT; ++mt)
      vd[mt] = __builtin_nontemporal_load(reinterpret_cast<const short4_t*>(vt_ + (int64_t)(16 * mt + l16) * v_dim));
  };

  load_tile(0, kb0, vb0);
  load_tile(1, kb1, vb1);

  // Q fragments (B operand of S^T): Q[row][32*ks + 8*g .. +8]
  const u16* qbase = reinterpret_cast<const u16*>(P.q);
  bf16x8_t qf[2][KS];
#pragma unroll
  for (int nt = 0; nt < 2; ++nt) {
    const int r = row0 + 16 * nt + l16;
    const bool ok = (16 * nt + l16) < nrows;
    const int t = ok ? r / P.G : 0;
    const int h = hkv * P.G + (ok ? r - (r / P.G) * P.G : 0);
    const u16* qr = qbase + (int64_t)b * P.q_sb + (int64_t)t * P.q_st + (int64_t)h * P.q_sh;
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

  auto consume = [&](int kt, const bf16x8_t (&kf)[KS], short4_t (&vf)[MT]) {
    const int j0 = kbeg + 16 * kt;
    const bool tile_valid = block_of(j0) >= 0;
    // keys of an unmapped block, and keys past the furthest query (possibly never written), must not
    // reach the PV product: their values may be anything
    if (!tile_valid || j0 + 15 > qmax) {
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        if (!tile_valid || j0 + 4 * g + i > qmax) {
#pragma unroll
          for (int mt = 0; mt < MT; ++mt) vf[mt][i] = 0;
        }
      }
    }
    float4_t sc[2];
#pragma unroll
    for (int nt = 0; nt < 2; ++nt) {
      sc[nt] = float4_t{0.f, 0.f, 0.f, 0.f};
      if (nt == 0 || two) {
#pragma unroll
        for (int ks = 0; ks < KS; ++ks)
          sc[nt] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(kf[ks], qf[nt][ks], sc[nt], 0, 0, 0);
      }
    }
    short4_t pf[2];
    float alpha[2];
#pragma unroll
    for (int nt = 0; nt < 2; ++nt) {
      float sv[4];
      float tmax = -INFINITY;
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const int key = j0 + 4 * g + i;
        const bool vis = tile_valid && key <= rpos[nt];
        sv[i] = vis ? sc[nt][i] * P.scale_log2 : -INFINITY;
        tmax = fmaxf(tmax, sv[i]);
      }
      tmax = max_across_groups(tmax);
      const float m_new = fmaxf(m_run[nt], tmax);
      alpha[nt] = (m_new == -INFINITY) ? 1.f : exp2f(m_run[nt] - m_new);
      float psum = 0.f;
      float pv[4];
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        pv[i] = (sv[i] == -INFINITY) ? 0.f : exp2f(sv[i] - m_new);
        psum += pv[i];
      }
      pf[nt] = bf16_rne4(pv);
      l_run[nt] = l_run[nt] * alpha[nt] + psum;
      m_run[nt] = m_new;
    }
    // unconditional rescale: a branch here splits the accumulators' live ranges and spills
#pragma unroll
    for (int mt = 0; mt < MT; ++mt)
#pragma unroll
      for (int nt = 0; nt < 2; ++nt) {
        acc[mt][nt][0] *= alpha[nt];
        acc[mt][nt][1] *= alpha[nt];
        acc[mt][nt][2] *= alpha[nt];
        acc[mt][nt][3] *= alpha[nt];
      }
#pragma unroll
    for (int mt = 0; mt < MT; ++mt) {
      acc[mt][0] = __builtin_amdgcn_mfma_f32_16x16x16bf16_1k(vf[mt], pf[0], acc[mt][0], 0, 0, 0);
      if (two) acc[mt][1] = __builtin_amdgcn_mfma_f32_16x16x16bf16_1k(vf[mt], pf[1], acc[mt][1], 0, 0, 0);
    }
  };

  const int kp = max(ntiles - 3, 0);   // the tile before which `next` runs, exactly once
  for (int kt = 0; kt < ntiles; kt += 3) {
    load_tile(kt + 2, kb2, vb2);
    if (kt == kp) next();
    consume(kt, kb0, vb0);
    if (kt + 1 >= ntiles) break;
    load_tile(kt + 3, kb0, vb0);
    if (kt + 1 == kp) next();
    consume(kt + 1, kb1, vb1);
    if (kt + 2 >= ntiles) break;
    load_tile(kt + 4, kb1, vb1);
    if (kt + 2 == kp) next();
    consume(kt + 2, kb2, vb2);
  }

  // write this chunk's partial for every real row of the tile that sees the chunk
#pragma unroll
  for (int nt = 0; nt < 2; ++nt) {
    float lsum = l_run[nt];
    lsum = sum_across_groups(lsum);
    const int r = 16 * nt + l16;
    if (r >= nrows || rpos[nt] < kbeg) continue;
    const int rr = row0 + r;
    const int t = rr / P.G, h = hkv * P.G + (rr - t * P.G);
    const int64_t R = row_index(P, b, t, h);
    float* pa = P.ws_acc + (R * P.nsplit + s) * D;
#pragma unroll
    for (int mt = 0; mt < MT; ++mt)
      *reinterpret_cast<float4_t*>(pa + 16 * mt + 4 * g) = acc[mt][nt];
    if (g == 0) {
      float* pm = P.ws_ml + (R * P.nsplit + s) * 2;
      pm[0] = m_run[nt];
      pm[1] = lsum;
    }
  }
}

// Persistent kernel: as many workgroups as the GPU holds at once, each of hpw waves over the hpw KV
// heads of a head group, so the heads' tiles of a block (neighbours in the pool) stream from one CU
// at about the same time. Plan unit r = (plan item r / ngrp, head group r % ngrp); the units are
// dealt round-robin over the first geff workgroups, geff chosen so that every round but the last is
// full and the last has as few idle workgroups as the count allows. Inside a workgroup the waves
// take (unit, head) pairs from an LDS counter, so waves that the memory system serves faster take
// more; each wave takes and fetches its next pair while the current one still streams.
template <int D, int BSZ>
__global__ void __launch_bounds__(64 * MAX_HEADS_PER_WG) __attribute__((amdgpu_waves_per_eu(2)))
attn_mfma_bf16_kernel(AttnParams P) {
  __shared__ int unit_ctr;
  const int hpw = blockDim.x >> 6;
  const int ngrp = P.kv.n_kv_heads / hpw;
  const int64_t total = (int64_t)P.n_items[0] * ngrp;
  if (total == 0) return;
  const int64_t rounds = (total + gridDim.x - 1) / gridDim.x;
  const int64_t geff = (total + rounds - 1) / rounds;
  if ((int64_t)blockIdx.x >= geff) return;   // both returns are uniform over the workgroup
  // This workgroup's share: plan units r_j = blockIdx.x + j * geff, j < nj, each hpw heads. Its waves
  // take (j, head) pairs in order from an LDS counter, so a wave that streams faster takes more.
  const int64_t nj = (total - blockIdx.x + geff - 1) / geff;
  const int units = (int)(nj * hpw);
  if (threadIdx.x == 0) unit_ctr = 0;
  __syncthreads();
  auto take = [&]() {
    int t = 0;
    if ((threadIdx.x & 63) == 0) t = atomicAdd(&unit_ctr, 1);
    return __builtin_amdgcn_readlane(t, 0);
  };
  auto unit_r = [&](int u) { return (int64_t)blockIdx.x + (int64_t)(u / hpw) * geff; };
  int u = take();
  if (u >= units) return;
  ItemRegs cur, nxt;
  fetch_item<BSZ>(P, unit_r(u) / ngrp, cur);
  for (;;) {
    int un = units;
    // the next unit is taken a few tiles before this one ends, and its metadata fetched then
    attn_mfma_item<D, BSZ>(P, cur, (int)(unit_r(u) % ngrp) * hpw + u % hpw, [&]() {
      un = take();
      fetch_item<BSZ>(P, unit_r(un < units ? un : u) / ngrp, nxt);
    });
    if (un >= units) break;
    cur = nxt;
    u = un;
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
  const T_* qrow = reinterpret_cast<const T_*>(P.q) + (int64_t)b * P.q_sb + (int64_t)t * P.q_st + (int64_t)h * P.q_sh;
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
        for (int d = 0; d < D; ++d) dot = fmaf(qs[d], E::load(kr, (int64_t)d * P.kv.k_dim), dot);
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
  const int D = P.kv.head_dim;
  T_* orow = reinterpret_cast<T_*>(out) + (int64_t)b * o_sb + (int64_t)t * o_st + (int64_t)h * o_sh;
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
  if (kv.k_slot != kv.head_dim || kv.k_dim != 1 || kv.v_slot != 1 || kv.v_dim != kv.block_size) return false;
  if (kv.k_block % 8 || kv.k_head % 8 || kv.v_block % 8 || kv.v_head % 8) return false;
  if ((reinterpret_cast<uintptr_t>(kv.k) | reinterpret_cast<uintptr_t>(kv.v) | reinterpret_cast<uintptr_t>(q)) & 15)
    return false;
  if (q_sb % 8 || q_st % 8 || q_sh % 8) return false;
  return true;
}

int attn_split() {
  static const int split = [] {
    const char* e = getenv("FS_ATTN_SPLIT");
    int v = e ? atoi(e) : 512;
    if (v < 16 || v > 512 || v % 16) v = 512;  // a chunk's block list must fit one wavefront
    return v;
  }();
  return split;
}

// Workgroups of `threads` threads of `fn` that the current device holds at once (cached per device,
// kernel and size).
int64_t resident_wgs(const void* fn, int threads) {
  struct Entry { int dev; const void* fn; int threads; int64_t wgs; };
  static Entry cache[64];
  static int n_cache = 0;
  static std::mutex mu;
  std::lock_guard<std::mutex> lock(mu);
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess) return -1;
  for (int i = 0; i < n_cache; ++i)
    if (cache[i].dev == dev && cache[i].fn == fn && cache[i].threads == threads) return cache[i].wgs;
  int cus = 0, per_cu = 0;
  if (hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess) return -1;
  if (hipOccupancyMaxActiveBlocksPerMultiprocessor(&per_cu, fn, threads, 0) != hipSuccess || per_cu <= 0) return -1;
  const int64_t w = (int64_t)cus * per_cu;
  if (n_cache < 64) cache[n_cache++] = Entry{dev, fn, threads, w};
  return w;
}

int64_t nsplit_for(int32_t max_blocks, int32_t block_size) {
  const int64_t S = (int64_t)max_blocks * block_size;
  return (S + attn_split() - 1) / attn_split();
}

// Upper bound of the plan's length: every (row, query tile, chunk).
int64_t max_items(int32_t B, int32_t T, int32_t n_heads, int32_t max_blocks, int32_t block_size) {
  const int64_t qtiles = ((int64_t)T * n_heads + QTILE - 1) / QTILE;   // n_heads bounds the group size
  return (int64_t)B * qtiles * nsplit_for(max_blocks, block_size);
}

int heads_per_wg(int n_kv_heads) {
  int h = n_kv_heads < MAX_HEADS_PER_WG ? n_kv_heads : MAX_HEADS_PER_WG;
  while (n_kv_heads % h) --h;
  return h;
}

}  // namespace

extern "C" int64_t fs_paged_attention_workspace_size(int32_t B, int32_t T, int32_t n_heads, int32_t head_dim,
                                                     int32_t max_blocks, int32_t block_size) {
  if (B <= 0 || T <= 0 || n_heads <= 0 || head_dim <= 0 || max_blocks <= 0 || block_size <= 0) return 0;
  const int64_t rows = (int64_t)B * T * n_heads;
  const int64_t ns = nsplit_for(max_blocks, block_size);
  const int64_t list = (max_items(B, T, n_heads, max_blocks, block_size) * (int64_t)sizeof(AttnItem) + 255) / 256 * 256;
  return WS_HEADER + list + rows * ns * (head_dim + 2) * (int64_t)sizeof(float) + 256;
}

extern "C" int fs_paged_attention(const void* q, int64_t q_sb, int64_t q_st, int64_t q_sh, const fs_kv_layout* kv,
                                  const int32_t* block_tables, int64_t table_stride, int32_t max_blocks,
                                  const int32_t* positions, int32_t B, int32_t T, int32_t n_heads, float scale,
                                  void* out, int64_t o_sb, int64_t o_st, int64_t o_sh, void* workspace,
                                  int64_t workspace_bytes, void* stream) {
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
  P.nsplit = (int32_t)nsplit_for(max_blocks, kv->block_size);
  P.split = attn_split();
  const int64_t rows = (int64_t)B * T * n_heads;
  char* ws = reinterpret_cast<char*>(workspace);
  const int64_t list = (max_items(B, T, n_heads, max_blocks, kv->block_size) * (int64_t)sizeof(AttnItem) + 255) / 256 * 256;
  P.n_items = reinterpret_cast<int32_t*>(ws);
  P.items = reinterpret_cast<AttnItem*>(ws + WS_HEADER);
  P.ws_acc = reinterpret_cast<float*>(ws + WS_HEADER + list);
  P.ws_ml = P.ws_acc + rows * P.nsplit * kv->head_dim;

  hipStream_t st = fs::as_stream(stream);
  if (mfma_eligible(*kv, q, q_sb, q_st, q_sh)) {
    const bool bs16 = kv->block_size == 16;
    const void* fn = kv->head_dim == 128
                         ? (bs16 ? (const void*)attn_mfma_bf16_kernel<128, 16> : (const void*)attn_mfma_bf16_kernel<128, 0>)
                         : (bs16 ? (const void*)attn_mfma_bf16_kernel<64, 16> : (const void*)attn_mfma_bf16_kernel<64, 0>);
    const int threads = 64 * heads_per_wg(kv->n_kv_heads);
    const int64_t wgs = resident_wgs(fn, threads);
    if (wgs <= 0) {
      fs::set_error("paged_attention: device occupancy query failed");
      return (int)hipErrorUnknown;
    }
    attn_plan_kernel<<<1, PLAN_THREADS, 0, st>>>(P);
    const unsigned grid = (unsigned)wgs;
    if (kv->head_dim == 128) {
      if (bs16) attn_mfma_bf16_kernel<128, 16><<<grid, threads, 0, st>>>(P);
      else attn_mfma_bf16_kernel<128, 0><<<grid, threads, 0, st>>>(P);
    } else {
      if (bs16) attn_mfma_bf16_kernel<64, 16><<<grid, threads, 0, st>>>(P);
      else attn_mfma_bf16_kernel<64, 0><<<grid, threads, 0, st>>>(P);
    }
  } else {
    dim3 grid((unsigned)rows, (unsigned)P.nsplit);
    switch (kv->dtype) {
      case FS_F32: attn_generic_kernel<FS_F32><<<grid, 64, 0, st>>>(P); break;
      case FS_BF16: attn_generic_kernel<FS_BF16><<<grid, 64, 0, st>>>(P); break;
      default: attn_generic_kernel<FS_F16><<<grid, 64, 0, st>>>(P); break;
    }
  }
  if (int e = fs::launch_status("paged_attention")) return e;
  dim3 cgrid((unsigned)((rows + COMBINE_ROWS - 1) / COMBINE_ROWS));
  switch (kv->dtype) {
    case FS_F32: attn_combine_kernel<FS_F32><<<cgrid, 64 * COMBINE_ROWS, 0, st>>>(P, out, o_sb, o_st, o_sh); break;
    case FS_BF16: attn_combine_kernel<FS_BF16><<<cgrid, 64 * COMBINE_ROWS, 0, st>>>(P, out, o_sb, o_st, o_sh); break;
    default: attn_combine_kernel<FS_F16><<<cgrid, 64 * COMBINE_ROWS, 0, st>>>(P, out, o_sb, o_st, o_sh); break;
  }
  return fs::launch_status("paged_attention_combine");
}
