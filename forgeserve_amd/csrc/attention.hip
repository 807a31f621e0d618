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

#include "common.h"

namespace {

constexpr int QTILE = 32;            // query rows per MFMA workgroup
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
};

FS_DEVICE int64_t row_index(const AttnParams& P, int b, int t, int h) { return ((int64_t)b * P.T + t) * P.H + h; }

// ------------------------------------------------------------------------------------------------
// MFMA kernel (bf16)
// ------------------------------------------------------------------------------------------------
// BSZ: the pool's block size when it is known at compile time (16), else 0 (any multiple of 16).
template <int D, int BSZ>
__global__ void __launch_bounds__(64) __attribute__((amdgpu_waves_per_eu(2))) attn_mfma_bf16_kernel(AttnParams P) {
  constexpr int KS = D / 32;   // k-steps of the QK^T product
  constexpr int MT = D / 16;   // 16-dim tiles of the PV product
  const int lane = threadIdx.x;
  const int l16 = lane & 15, g = lane >> 4;
  // heads of one (row, chunk) are adjacent workgroups: their tiles are neighbours in the pool
  const int Hkv = P.kv.n_kv_heads;
  const int s = blockIdx.x / Hkv;
  const int hkv = blockIdx.x - s * Hkv;
  const int b = blockIdx.y;
  const int row0 = blockIdx.z * QTILE;
  const int nrows = min(QTILE, P.T * P.G - row0);
  const int* posb = P.pos + (int64_t)b * P.T;

  // positions of this lane's two rows (row = 16*nt + l16), and the tile's furthest position
  int rpos[2];
  int qmax = -1;
#pragma unroll
  for (int nt = 0; nt < 2; ++nt) {
    const int r = 16 * nt + l16;
    rpos[nt] = (r < nrows) ? posb[(row0 + r) / P.G] : -1;
  }
  {
    const int t0 = row0 / P.G, t1 = (row0 + nrows - 1) / P.G;
    for (int t = t0; t <= t1; ++t) qmax = max(qmax, posb[t]);
  }
  qmax = __builtin_amdgcn_readfirstlane(qmax);  // the same in every lane: keep the loop scalar
  const int kbeg = s * P.split;
  if (qmax < kbeg) return;  // no query of this tile sees this chunk: the combine never reads it
  const int kend = min(kbeg + P.split, qmax + 1);
  const int ntiles = (kend - kbeg + 15) >> 4;
  const bool two = nrows > 16;

  // Q fragments (B operand of S^T): Q[row][32*ks + 8*g .. +8]
  typedef uint16_t u16;
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

  // physical block ids of this chunk (at most P.split/16 + 1 entries), one per lane
  const int BS = BSZ ? BSZ : P.kv.block_size;
  const int64_t v_dim = BSZ ? BSZ : P.kv.v_dim;   // == block_size (dim-major values)
  const int first_blk = kbeg / BS;
  const int nblk = (kend - 1) / BS - first_blk + 1;
  int my_phys = -1;
  if (lane < nblk && first_blk + lane < P.max_blocks) {
    const int v = P.table[(int64_t)b * P.table_stride + first_blk + lane];
    my_phys = (v >= 0 && v < P.kv.num_blocks) ? v : -1;
  }

  const u16* kpool = reinterpret_cast<const u16*>(P.kv.k);
  const u16* vpool = reinterpret_cast<const u16*>(P.kv.v);
  const int64_t k_head_off = (int64_t)hkv * P.kv.k_head;
  const int64_t v_head_off = (int64_t)hkv * P.kv.v_head;

  float4_t acc[MT][2];
#pragma unroll
  for (int mt = 0; mt < MT; ++mt) {
    acc[mt][0] = float4_t{0.f, 0.f, 0.f, 0.f};
    acc[mt][1] = float4_t{0.f, 0.f, 0.f, 0.f};
  }
  float m_run[2] = {-INFINITY, -INFINITY};
  float l_run[2] = {0.f, 0.f};

  // Three tile buffers in registers: while tile t is consumed, tiles t+1 and t+2 are in flight.
  bf16x8_t kb0[KS], kb1[KS], kb2[KS];
  short4_t vb0[MT], vb1[MT], vb2[MT];
  bool ok0 = false, ok1 = false, ok2 = false;

  auto load_tile = [&](int kt, bf16x8_t (&kd)[KS], short4_t (&vd)[MT], bool& valid) {
    const int j0 = kbeg + 16 * kt;
    const int bi = j0 / BS - first_blk;   // < nblk: the tile lies inside the chunk's block list
    const int64_t phys = __builtin_amdgcn_readfirstlane(__shfl(my_phys, bi, 64));  // wave-uniform block id
    valid = phys >= 0;
    const int slot0 = j0 - (j0 / BS) * BS;
    if (valid) {
      const u16* kt_ = kpool + phys * P.kv.k_block + k_head_off + (int64_t)(slot0 + l16) * D;
#pragma unroll
      for (int ks = 0; ks < KS; ++ks)   // read once per launch: nontemporal
        kd[ks] = __builtin_nontemporal_load(reinterpret_cast<const bf16x8_t*>(kt_ + 32 * ks + 8 * g));
      const u16* vt_ = vpool + phys * P.kv.v_block + v_head_off + slot0 + 4 * g;
#pragma unroll
      for (int mt = 0; mt < MT; ++mt)
        vd[mt] = __builtin_nontemporal_load(
            reinterpret_cast<const short4_t*>(vt_ + (int64_t)(16 * mt + l16) * v_dim));
    } else {
#pragma unroll
      for (int ks = 0; ks < KS; ++ks) kd[ks] = bf16x8_t{};
#pragma unroll
      for (int mt = 0; mt < MT; ++mt) vd[mt] = short4_t{0, 0, 0, 0};
    }
  };

  auto consume = [&](int kt, const bf16x8_t (&kf)[KS], short4_t (&vf)[MT], bool tile_valid) {
    const int j0 = kbeg + 16 * kt;
    // keys past the furthest query (possibly never written) must not reach the PV product
    if (j0 + 15 > qmax) {
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        if (j0 + 4 * g + i > qmax) {
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
      tmax = fmaxf(tmax, __shfl_xor(tmax, 16, 64));
      tmax = fmaxf(tmax, __shfl_xor(tmax, 32, 64));
      const float m_new = fmaxf(m_run[nt], tmax);
      alpha[nt] = (m_new == -INFINITY) ? 1.f : exp2f(m_run[nt] - m_new);
      float psum = 0.f;
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const float p = (sv[i] == -INFINITY) ? 0.f : exp2f(sv[i] - m_new);
        pf[nt][i] = (short)f32_to_bf16(p);
        psum += p;
      }
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

  load_tile(0, kb0, vb0, ok0);
  if (ntiles > 1) load_tile(1, kb1, vb1, ok1);
  for (int kt = 0; kt < ntiles; kt += 3) {
    if (kt + 2 < ntiles) load_tile(kt + 2, kb2, vb2, ok2);
    consume(kt, kb0, vb0, ok0);
    if (kt + 1 >= ntiles) break;
    if (kt + 3 < ntiles) load_tile(kt + 3, kb0, vb0, ok0);
    consume(kt + 1, kb1, vb1, ok1);
    if (kt + 2 >= ntiles) break;
    if (kt + 4 < ntiles) load_tile(kt + 4, kb1, vb1, ok1);
    consume(kt + 2, kb2, vb2, ok2);
  }

  // write this chunk's partial for every real row of the tile that sees the chunk
#pragma unroll
  for (int nt = 0; nt < 2; ++nt) {
    float lsum = l_run[nt];
    lsum += __shfl_xor(lsum, 16, 64);
    lsum += __shfl_xor(lsum, 32, 64);
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
template <int DT>
__global__ void __launch_bounds__(64) attn_combine_kernel(AttnParams P, void* out, int64_t o_sb, int64_t o_st,
                                                          int64_t o_sh) {
  typedef Elem<DT> E;
  typedef typename E::T T_;
  const int lane = threadIdx.x;
  const int64_t R = blockIdx.x;
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
  float M = -INFINITY;
  for (int s = 0; s < ns; ++s) M = fmaxf(M, ml[2 * s]);
  float L = 0.f;
  float acc[4] = {0.f, 0.f, 0.f, 0.f};
  const float* pa = P.ws_acc + R * P.nsplit * D;
  for (int s = 0; s < ns; ++s) {
    const float ms = ml[2 * s];
    const float w = (ms == -INFINITY) ? 0.f : exp2f(ms - M);
    L += w * ml[2 * s + 1];
#pragma unroll
    for (int c = 0; c < 4; ++c) {
      const int d = lane + 64 * c;
      if (d < D) acc[c] += w * pa[(int64_t)s * D + d];
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

int64_t nsplit_for(int32_t max_blocks, int32_t block_size) {
  const int64_t S = (int64_t)max_blocks * block_size;
  return (S + attn_split() - 1) / attn_split();
}

}  // namespace

extern "C" int64_t fs_paged_attention_workspace_size(int32_t B, int32_t T, int32_t n_heads, int32_t head_dim,
                                                     int32_t max_blocks, int32_t block_size) {
  if (B <= 0 || T <= 0 || n_heads <= 0 || head_dim <= 0 || max_blocks <= 0 || block_size <= 0) return 0;
  const int64_t rows = (int64_t)B * T * n_heads;
  const int64_t ns = nsplit_for(max_blocks, block_size);
  return rows * ns * (head_dim + 2) * (int64_t)sizeof(float) + 256;
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
  P.ws_acc = reinterpret_cast<float*>(workspace);
  P.ws_ml = P.ws_acc + rows * P.nsplit * kv->head_dim;

  hipStream_t st = fs::as_stream(stream);
  if (mfma_eligible(*kv, q, q_sb, q_st, q_sh)) {
    const int qtiles = (T * P.G + QTILE - 1) / QTILE;
    dim3 grid((unsigned)(P.nsplit * kv->n_kv_heads), (unsigned)B, (unsigned)qtiles);
    const bool bs16 = kv->block_size == 16;
    if (kv->head_dim == 128) {
      if (bs16) attn_mfma_bf16_kernel<128, 16><<<grid, 64, 0, st>>>(P);
      else attn_mfma_bf16_kernel<128, 0><<<grid, 64, 0, st>>>(P);
    } else {
      if (bs16) attn_mfma_bf16_kernel<64, 16><<<grid, 64, 0, st>>>(P);
      else attn_mfma_bf16_kernel<64, 0><<<grid, 64, 0, st>>>(P);
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
  dim3 cgrid((unsigned)rows);
  switch (kv->dtype) {
    case FS_F32: attn_combine_kernel<FS_F32><<<cgrid, 64, 0, st>>>(P, out, o_sb, o_st, o_sh); break;
    case FS_BF16: attn_combine_kernel<FS_BF16><<<cgrid, 64, 0, st>>>(P, out, o_sb, o_st, o_sh); break;
    default: attn_combine_kernel<FS_F16><<<cgrid, 64, 0, st>>>(P, out, o_sb, o_st, o_sh); break;
  }
  return fs::launch_status("paged_attention_combine");
}
