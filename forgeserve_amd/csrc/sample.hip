// Sampling and speculative acceptance over vocab-wide rows, with no host round trip.
//
// Reference: sampling.py:9-21 (probs_from_logits, sample), speculative.py:20-33 (verify_draft) and the
// rollback arithmetic of speculative.py:77.
//
// Every row of V logits is cut into chunks of CH columns. Launch 1 reduces each (row, chunk) to
// (max of y = x/T, sum of exp(y - max), first argmax of x). Later launches merge a row's chunk partials
// in increasing chunk order, so every workgroup that needs a row's softmax gets bit-identical
// (M, S), and every probability is evaluated by one function (ProbFn): p_v = exp(y_v - M) * (1/S),
// y_v = x_v / T a true float32 division, the order in which torch's softmax forms it (sampling.py:13).
// M is torch's max bit for bit; exp and S (a sum in another order) differ from torch's by a few ulps.
//
// torch.multinomial(w, 1) draws argmax_v(w_v / E_v) with E ~ Exp(1) (first index on ties); the
// caller supplies E, so the draw is a deterministic function of (logits, E) and can be compared
// bit for bit with the CPU reference on the same noise.
#include <math.h>

#include <algorithm>
#include <mutex>

#include "common.h"

namespace {

constexpr int THREADS = 256;
constexpr int VEC = 8;                       // consecutive columns per thread group
constexpr int UNROLL = 4;                    // groups per thread per chunk: 4 16-byte loads in flight
constexpr int CH = THREADS * VEC * UNROLL;   // 8192 columns per chunk
constexpr int UNROLL_R = 2;                  // the acceptance's residual and argmax passes:
constexpr int CHR = THREADS * VEC * UNROLL_R;  // 4096 columns per chunk (many workgroups for two rows)

// Arithmetic type of the probabilities: the logits path works on the float32 softmax
// (sampling.py:13), the probabilities path in the dtype it is given.
template <int DT, bool PROBS>
struct ProbType {
  static constexpr int value = PROBS ? DT : FS_F32;
};
constexpr float LOG2E_F = 1.4426950408889634f;

// m: max of x/T (T > 0) or of x (T == 0); s: sum of exp(x/T - m) (T > 0); (av, ai): the first
// argmax of x (T == 0; a vocab-wide pass leaves it unset for T > 0)
typedef SoftmaxStat Stat;

// Rows of a batch of sequences: for sequence b, rows 0..n0-1 come from base0 (row i at
// base0 + b*sb0 + i*si0) and rows n0..n0+n1-1 from base1.
struct RowSet {
  const void* base0;
  int64_t sb0, si0;
  int32_t n0;
  const void* base1;
  int64_t sb1, si1;
  int32_t n1;
};

template <int DT>
FS_DEVICE const typename Elem<DT>::T* row_ptr(const RowSet& rs, int b, int i) {
  typedef typename Elem<DT>::T T_;
  if (i < rs.n0) return reinterpret_cast<const T_*>(rs.base0) + b * rs.sb0 + i * rs.si0;
  return reinterpret_cast<const T_*>(rs.base1) + b * rs.sb1 + (i - rs.n0) * rs.si1;
}

// Load 8 consecutive columns starting at v (a multiple of 8) as f32; columns >= V read as `fill`.
template <int DT>
FS_DEVICE void load8(const typename Elem<DT>::T* row, int64_t v, int64_t V, bool vec_ok, float fill, float (&x)[8]) {
  if (vec_ok && v + 8 <= V) {
    if (DT == FS_F32) {
      const float4_t a = *reinterpret_cast<const float4_t*>(reinterpret_cast<const float*>(row) + v);
      const float4_t c = *reinterpret_cast<const float4_t*>(reinterpret_cast<const float*>(row) + v + 4);
      x[0] = a[0]; x[1] = a[1]; x[2] = a[2]; x[3] = a[3];
      x[4] = c[0]; x[5] = c[1]; x[6] = c[2]; x[7] = c[3];
    } else {
      typedef __attribute__((__vector_size__(4 * sizeof(uint32_t)))) uint32_t u32x4;
      const u32x4 w = *reinterpret_cast<const u32x4*>(reinterpret_cast<const uint16_t*>(row) + v);
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        x[2 * j] = Elem<DT>::to_f32((uint16_t)(w[j] & 0xffffu));
        x[2 * j + 1] = Elem<DT>::to_f32((uint16_t)(w[j] >> 16));
      }
    }
  } else {
#pragma unroll
    for (int j = 0; j < 8; ++j) x[j] = (v + j < V) ? Elem<DT>::load(row, v + j) : fill;
  }
}

// Raw registers of 8 consecutive columns (two 16-byte loads for f32, one for bf16/f16), loaded
// without bounds checks, then converted to f32 apart from the load. A block of loads is issued
// first and converted after a scheduling barrier: a conversion between two loads makes the second
// wait for the first (the compiler places the wait before the conversion).
template <int DT>
struct Raw8 {
  typedef __attribute__((__vector_size__(4 * sizeof(uint32_t)))) uint32_t u32x4;
  u32x4 w[DT == FS_F32 ? 2 : 1];
  FS_DEVICE void load(const typename Elem<DT>::T* row, int64_t v) {
    const u32x4* q = reinterpret_cast<const u32x4*>(row + v);
    w[0] = q[0];
    if (DT == FS_F32) w[DT == FS_F32 ? 1 : 0] = q[1];
  }
  FS_DEVICE void to_f32(float (&x)[8]) const {
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      if (DT == FS_F32) {
        x[j] = __uint_as_float(w[0][j]);
        x[4 + j] = __uint_as_float(w[DT == FS_F32 ? 1 : 0][j]);
      } else {
        x[2 * j] = Elem<DT>::to_f32((uint16_t)(w[0][j] & 0xffffu));
        x[2 * j + 1] = Elem<DT>::to_f32((uint16_t)(w[0][j] >> 16));
      }
    }
  }
};

// Every group u (columns v0 + u * THREADS * VEC .. + 7) of a U-group block is in range and 16-byte
// loadable: false only in a row's last chunk (or for unaligned rows).
template <int U>
FS_DEVICE bool block_in_range(int64_t v0, int64_t V, bool vec_ok) {
  return vec_ok && v0 + (int64_t)(U - 1) * THREADS * VEC + VEC <= V;
}

// U groups of 8 consecutive columns per thread, group u at column v0 + u * THREADS * VEC, as f32;
// columns >= V read as `fill`. In range, the U loads are issued back to back before any conversion.
template <int DT, int U>
FS_DEVICE void load_block(const typename Elem<DT>::T* row, int64_t v0, int64_t V, bool vec_ok, float fill,
                          float (&x)[U][8]) {
  constexpr int64_t STRIDE = (int64_t)THREADS * VEC;
  if (block_in_range<U>(v0, V, vec_ok)) {
    Raw8<DT> r[U];
#pragma unroll
    for (int u = 0; u < U; ++u) r[u].load(row, v0 + u * STRIDE);
    __builtin_amdgcn_sched_barrier(0);
#pragma unroll
    for (int u = 0; u < U; ++u) r[u].to_f32(x[u]);
  } else {
#pragma unroll
    for (int u = 0; u < U; ++u) load8<DT>(row, v0 + u * STRIDE, V, vec_ok, fill, x[u]);
  }
}

// Workgroup reductions in a fixed order (lane butterfly, then waves in index order).
FS_DEVICE float block_max(float v, float* sh) {
  v = wave_max(v);
  __syncthreads();
  if ((threadIdx.x & 63) == 0) sh[threadIdx.x >> 6] = v;
  __syncthreads();
  float r = sh[0];
#pragma unroll
  for (int i = 1; i < THREADS / 64; ++i) r = fmaxf(r, sh[i]);
  return r;
}
FS_DEVICE float block_sum(float v, float* sh) {
  v = wave_sum(v);
  __syncthreads();
  if ((threadIdx.x & 63) == 0) sh[threadIdx.x >> 6] = v;
  __syncthreads();
  float r = sh[0];
#pragma unroll
  for (int i = 1; i < THREADS / 64; ++i) r += sh[i];
  return r;
}
FS_DEVICE void block_argmax(float& v, int& i, float* shv, int* shi) {
  wave_argmax(v, i);
  __syncthreads();
  if ((threadIdx.x & 63) == 0) {
    shv[threadIdx.x >> 6] = v;
    shi[threadIdx.x >> 6] = i;
  }
  __syncthreads();
  v = shv[0];
  i = shi[0];
#pragma unroll
  for (int w = 1; w < THREADS / 64; ++w) argmax_merge(v, i, shv[w], shi[w]);
}

// Merge the chunk partials of one row (increasing chunk order).
FS_DEVICE Stat merge_row(const Stat* st, int nch) {
  Stat r = st[0];
  float M = r.m;
  for (int c = 1; c < nch; ++c) M = fmaxf(M, st[c].m);
  float S = 0.f;
  for (int c = 0; c < nch; ++c) {
    const float mc = st[c].m;
    S += (mc == -INFINITY) ? 0.f : st[c].s * __builtin_amdgcn_exp2f((mc - M) * LOG2E_F);
  }
  for (int c = 1; c < nch; ++c) argmax_merge(r.av, r.ai, st[c].av, st[c].ai);
  r.m = M;
  r.s = S;
  return r;
}

// The probability of logit x in a row with merged statistics (M, S) at temperature T > 0
// (sampling.py:13): y = x / T (a true division; exact and skipped at T == 1), then exp(y - M) times the
// correctly rounded 1/S, the order torch's softmax uses. Every kernel that needs a probability on the
// logits path calls this one function, so the accept test, the residual sums, the candidate keys and
// the exact keys all see the same p_v.
struct ProbFn {
  float T, M, invS;
  FS_DEVICE ProbFn() : T(1.f), M(0.f), invS(1.f) {}
  FS_DEVICE ProbFn(float t, const Stat& st) : T(t), M(st.m), invS(1.f / st.s) {}
  // from y = x / T (vocab-wide passes divide a whole register block under one uniform branch)
  FS_DEVICE float of_y(float y) const { return expf(y - M) * invS; }
  FS_DEVICE float operator()(float x) const { return of_y(T == 1.f ? x : x / T); }
};

// y = x / T in place for a block of registers, under a branch uniform over the workgroup (T is the
// row's or the sequence's), so T == 1 costs nothing; padding (-inf or 0) stays what it was.
template <int U>
FS_DEVICE void divide_by_t(float (&x)[U][8], float T) {
  if (T != 1.f) {
#pragma unroll
    for (int u = 0; u < U; ++u)
#pragma unroll
      for (int j = 0; j < 8; ++j) x[u][j] = x[u][j] / T;
  }
}

// One chunk of one row. T == 0: the first argmax of x. T > 0: (m, s) = (max of y, sum of exp(y - m))
// with y = x / T, a true division (sampling.py:13), so m is the max torch's softmax subtracts. The
// chunk's loads are all issued up front; the values stay in registers for the max pass and the exp
// pass (the sum's exp is the bare exp2; S differs from torch's sum by rounding either way).
template <int DT>
FS_DEVICE Stat chunk_stat(const typename Elem<DT>::T* row, int c, int64_t V, float T, float* shf, int* shi) {
  const bool vec_ok = (V % VEC) == 0 && ((reinterpret_cast<uintptr_t>(row) & 15) == 0);
  float x[UNROLL][8];
  load_block<DT, UNROLL>(row, (int64_t)c * CH + (int64_t)threadIdx.x * VEC, V, vec_ok, -INFINITY, x);
  Stat st;
  if (T <= 0.f) {
    float amv = -INFINITY;
    int ami = 0x7fffffff;
#pragma unroll
    for (int u = 0; u < UNROLL; ++u) {
      const int64_t v0 = (int64_t)c * CH + (int64_t)(threadIdx.x + THREADS * u) * VEC;
#pragma unroll
      for (int j = 0; j < 8; ++j)
        if (v0 + j < V) argmax_merge(amv, ami, x[u][j], (int)(v0 + j));
    }
    block_argmax(amv, ami, shf, shi);
    st.m = st.av = amv;
    st.ai = ami;
    st.s = 0.f;
    return st;
  }
  if (T != 1.f) {
#pragma unroll
    for (int u = 0; u < UNROLL; ++u)
#pragma unroll
      for (int j = 0; j < 8; ++j) x[u][j] = x[u][j] / T;  // padding stays -inf
  }
  float m = -INFINITY;
#pragma unroll
  for (int u = 0; u < UNROLL; ++u)
#pragma unroll
    for (int j = 0; j < 8; ++j) m = fmaxf(m, x[u][j]);
  const float M = block_max(m, shf);
  const float ML = M * LOG2E_F;
  float sum = 0.f;
#pragma unroll
  for (int u = 0; u < UNROLL; ++u)
#pragma unroll
    for (int j = 0; j < 8; ++j) sum += __builtin_amdgcn_exp2f(fmaf(x[u][j], LOG2E_F, -ML));  // exp(-inf) = 0
  st.m = M;
  st.s = block_sum(sum, shf);
  st.av = M;
  st.ai = 0;
  return st;
}

// ------------------------------------------------------------------------------------------------
// launch 1: per-(row, chunk) statistics
// ------------------------------------------------------------------------------------------------
template <int DT>
__global__ void __launch_bounds__(THREADS) stats_kernel(RowSet rs, int64_t V, int nch, const float* __restrict__ temps,
                                                        float t_all, const int32_t* __restrict__ k_eff,
                                                        Stat* __restrict__ out) {
  __shared__ float shf[THREADS / 64];
  __shared__ int shi[THREADS / 64];
  const int c = blockIdx.x;
  const int rho = blockIdx.y;
  const int per = rs.n0 + rs.n1;
  const int b = rho / per, i = rho - b * per;
  if (k_eff) {  // rows a sequence does not use: target rows > k_eff, draft rows >= k_eff
    const int ke = min(max(k_eff[b], 0), rs.n1);
    if (i < rs.n0 ? i > ke : (i - rs.n0) >= ke) return;
  }
  const float T = temps ? temps[b] : t_all;
  const auto* row = row_ptr<DT>(rs, b, i);
  const Stat st = chunk_stat<DT>(row, c, V, T, shf, shi);
  if (threadIdx.x == 0) out[(int64_t)rho * nch + c] = st;
}

// ------------------------------------------------------------------------------------------------
// sampling: argmax over a chunk of p_v / E_v, then a per-row finalize
// ------------------------------------------------------------------------------------------------
template <int DT>
__global__ void __launch_bounds__(THREADS) sample_argmax_kernel(RowSet rs, int64_t V, int nch,
                                                                const float* __restrict__ temps, float t_all,
                                                                const Stat* __restrict__ stats,
                                                                const float* __restrict__ E, int64_t ldE,
                                                                float* __restrict__ pv, int* __restrict__ pi) {
  __shared__ float shf[THREADS / 64];
  __shared__ int shi[THREADS / 64];
  __shared__ Stat shs;
  const int c = blockIdx.x, r = blockIdx.y;
  const float T = temps ? temps[r] : t_all;
  if (T <= 0.f) return;
  const auto* row = row_ptr<DT>(rs, r, 0);
  const float* er = E + (int64_t)r * ldE;
  const bool vec_ok = (V % VEC) == 0 && ((reinterpret_cast<uintptr_t>(row) & 15) == 0) &&
                      ((reinterpret_cast<uintptr_t>(er) & 15) == 0);
  float bv = -INFINITY;
  int bi = 0x7fffffff;
  float x[UNROLL][8], e[UNROLL][8];   // the chunk's loads go out before the row's statistics are merged
  const int64_t vb = (int64_t)c * CH + (int64_t)threadIdx.x * VEC;
  if (block_in_range<UNROLL>(vb, V, vec_ok)) {
    Raw8<DT> rx[UNROLL];
    Raw8<FS_F32> re[UNROLL];
#pragma unroll
    for (int u = 0; u < UNROLL; ++u) {
      rx[u].load(row, vb + u * THREADS * VEC);
      re[u].load(er, vb + u * THREADS * VEC);
    }
    __builtin_amdgcn_sched_barrier(0);
#pragma unroll
    for (int u = 0; u < UNROLL; ++u) {
      rx[u].to_f32(x[u]);
      re[u].to_f32(e[u]);
    }
  } else {
    load_block<DT, UNROLL>(row, vb, V, vec_ok, -INFINITY, x);
    load_block<FS_F32, UNROLL>(er, vb, V, vec_ok, 1.f, e);
  }
  if (threadIdx.x == 0) shs = merge_row(stats + (int64_t)r * nch, nch);
  __syncthreads();
  const ProbFn fs(T, shs);
  divide_by_t(x, T);
#pragma unroll
  for (int u = 0; u < UNROLL; ++u) {
    const int64_t v0 = (int64_t)c * CH + (int64_t)(threadIdx.x + THREADS * u) * VEC;
#pragma unroll
    for (int j = 0; j < 8; ++j) {
      if (v0 + j < V) argmax_merge(bv, bi, fs.of_y(x[u][j]) / e[u][j], (int)(v0 + j));
    }
  }
  block_argmax(bv, bi, shf, shi);
  if (threadIdx.x == 0) {
    pv[(int64_t)r * nch + c] = bv;
    pi[(int64_t)r * nch + c] = bi;
  }
}

__global__ void sample_final_kernel(int R, int nch, const float* __restrict__ temps, float t_all, bool greedy_only,
                                    const Stat* __restrict__ stats, const float* __restrict__ pv,
                                    const int* __restrict__ pi, int64_t* __restrict__ tok, int32_t* __restrict__ tok32,
                                    int64_t ld32) {
  const int r = blockIdx.x * blockDim.x + threadIdx.x;
  if (r >= R) return;
  int best;
  const float T = temps ? temps[r] : t_all;
  if (greedy_only || T <= 0.f) {
    best = merge_row(stats + (int64_t)r * nch, nch).ai;
  } else {
    float v = pv[(int64_t)r * nch];
    best = pi[(int64_t)r * nch];
    for (int c = 1; c < nch; ++c) argmax_merge(v, best, pv[(int64_t)r * nch + c], pi[(int64_t)r * nch + c]);
  }
  tok[r] = best;
  if (tok32) tok32[(int64_t)r * ld32] = best;
}

// ------------------------------------------------------------------------------------------------
// acceptance
// ------------------------------------------------------------------------------------------------
// Logits without given statistics take four launches: the statistics of every (row, 8K-column
// chunk) (accept_stats_kernel), the steps (accept_step_kernel), the draws' chunks (accept_kernel),
// then the draws (accept_draw_kernel); with the statistics given (from the LM head's epilogue), or on
// probabilities, the last three alone.
//   accept_step_kernel, one workgroup per sequence: sequence b's step (merging its rows' chunk
//     statistics when they come from the statistics launch); a greedy sequence is finished here, a
//     sampled one records its first rejected position and that position's row statistics;
//   accept_kernel, one workgroup per (sampled sequence, 4K-column chunk): reads its sequence's step,
//     then its chunk of the Exp(1) row and of the rejected position's rows, all at once, and records
//     the chunk's residual sum and the candidates of the draw;
//   accept_draw_kernel, one wave per sampled sequence: the draw from the chunks' records.
// Every record is read by a later launch than the one that wrote it, so no workgroup waits for
// another and the workspace needs no initial contents.
struct AcceptArgs {
  RowSet rs;             // n0 = K+1 target rows, n1 = K draft rows
  int32_t K;
  int64_t V;
  int nch;               // 8K-column chunks of the statistics pass
  int nchr;              // 4K-column chunks of the residual and argmax passes
  int B;
  const int32_t* draft;  // [B, K]
  const int32_t* k_eff;  // [B] or null (= K)
  const float* temps;    // [B] (ignored for probabilities)
  const float* u;        // [B, K]
  const float* E;        // [B, V]
  int64_t ldE;
  Stat* stats;           // [B*(2K+1)][nch] chunk partials (logits mode)
  Stat* mstats;          // [B*(2K+1)] merged row statistics (logits mode: the step's own)
  bool premerged;        // mstats are the caller's (from the LM head's epilogue): no statistics launch
  Stat* pairstat;        // [B][2] merged statistics of the step's target and draft rows j
  float* resid;          // [B][nchr] residual partial sums of the rejected row pair
  float* cmax;           // [B][nchr] max of the chunk's cheap keys (0: none positive; +inf: rescan)
  int* ncand;            // [B][nchr] candidates of the chunk (> NCAND: the list overflowed)
  int* cand;             // [B][nchr][NCAND] their column indices, in no particular order
  float* candw;          // [B][nchr][NCAND] their weights: r_v at a rejection, p_v for the bonus token
  float* cande;          // [B][nchr][NCAND] their Exp(1) values E_v
  int* jpos;             // [B]   the first rejected proposal, or k_eff
  int32_t* out_tokens;   // [B, K+1]
  int32_t* n_acc;        // [B]
  int32_t* seq_len;      // [B] or null
  float* dbg_p;          // [B, K] or null: p_i(x_i) of the proposals the step tests (the accept test's p)
  float* dbg_q;          // [B, K] or null: q_i(x_i)
  float* dbg_s;          // [B] or null: the residual sum of the rejected position (0: none, or greedy)
};

constexpr int STEP_WAVES = THREADS / 64;
constexpr int STEP_ROWS = 4;      // rows merged per wave and pass

FS_DEVICE int keff_of(const AcceptArgs& A, int b) { return A.k_eff ? min(max(A.k_eff[b], 0), A.K) : A.K; }



// What the outputs need that does not depend on the outcome, loaded by the caller up front (one
// wave): proposal `lane` of sequence b (lane < K) and seq_len[b].
struct OutPre {
  int d0, len0;
};
FS_DEVICE OutPre out_pre(const AcceptArgs& A, int b) {
  const int lane = threadIdx.x & 63;
  return OutPre{lane < A.K ? A.draft[(int64_t)b * A.K + lane] : 0, A.seq_len ? A.seq_len[b] : 0};
}

// The outputs of sequence b, written by one whole wave (lane i: token i, i + 64, ...): the j accepted
// proposals, the extra token, then -1.
FS_DEVICE void write_outputs(const AcceptArgs& A, int b, int j, int extra, const OutPre& pre) {
  const int lane = threadIdx.x & 63;
  int32_t* o = A.out_tokens + (int64_t)b * (A.K + 1);
  for (int i = lane; i <= A.K; i += 64) {
    const int d = i < 64 ? pre.d0 : (i < j ? A.draft[(int64_t)b * A.K + i] : 0);
    o[i] = i < j ? d : (i == j ? extra : -1);
  }
  if (lane == 0) {
    A.n_acc[b] = j;
    if (A.seq_len) A.seq_len[b] = pre.len0 + 1 + j;  // want = cached + 1 + len(accepted) (speculative.py:77)
  }
}

// The chunk statistics of R rows (one wave, lane c holding chunk c of each) merged as merge_row does:
// the max over the chunks, Σ s_c 2^(m_c - M) added in chunk order, the first argmax. The rows'
// reductions are interleaved step by step, so their cross-lane latencies overlap.
template <int R>
FS_DEVICE void merge_rows_wave(const Stat (&st)[R], bool in, int nch, Stat (&out)[R]) {
  float M[R], S[R], term[R], av[R];
  int ai[R];
#pragma unroll
  for (int i = 0; i < R; ++i) {
    M[i] = in ? st[i].m : -INFINITY;
    av[i] = in ? st[i].av : -INFINITY;
    ai[i] = in ? st[i].ai : 0x7fffffff;
    S[i] = 0.f;
  }
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) {
    float oa[R], om[R];
    int oi[R];
#pragma unroll
    for (int i = 0; i < R; ++i) {
      om[i] = __shfl_xor(M[i], o, 64);
      oa[i] = __shfl_xor(av[i], o, 64);
      oi[i] = __shfl_xor(ai[i], o, 64);
    }
#pragma unroll
    for (int i = 0; i < R; ++i) {
      M[i] = fmaxf(M[i], om[i]);
      argmax_merge(av[i], ai[i], oa[i], oi[i]);
    }
  }
#pragma unroll
  for (int i = 0; i < R; ++i)
    term[i] = (!in || st[i].m == -INFINITY) ? 0.f : st[i].s * __builtin_amdgcn_exp2f((st[i].m - M[i]) * LOG2E_F);
  for (int c = 0; c < nch; ++c)
#pragma unroll
    for (int i = 0; i < R; ++i) S[i] += __int_as_float(__builtin_amdgcn_readlane(__float_as_int(term[i]), c));
#pragma unroll
  for (int i = 0; i < R; ++i) out[i] = Stat{M[i], S[i], av[i], ai[i]};
}

// The step of sequence b, run by one whole workgroup. Wave 0 tests every proposal at once, one lane
// each; the first rejection ends the walk (speculative.py:25-29). The rows' statistics it needs, those
// of the first STEP_LDS proposals' rows, are staged in LDS meanwhile: merged from the statistics
// launch's chunk records (each wave takes STEP_ROWS rows at a time, one lane per chunk; every row is
// also written to the workspace), or, given, loaded by waves 1-3 while wave 0 waits for its proposals'
// logits. A greedy sequence is finished here (the extra token is the argmax of target row j); for a
// sampled one the rejected position j and its rows' statistics are recorded for the next launches.
constexpr int STEP_LDS = 64;

template <int DT, bool PROBS>
FS_DEVICE void sequence_step(const AcceptArgs& A, int b, Stat* sh_ms) {
  // sh_ms: target rows 0..STEP_LDS at [r], draft rows 0..STEP_LDS-1 at [STEP_LDS + 1 + r]
  const int per = A.rs.n0 + A.rs.n1;
  const Stat* ms = A.mstats + (int64_t)b * per;
  const int w = threadIdx.x >> 6, lane = threadIdx.x & 63;
  auto slot_of = [&](int r) {   // the LDS slot of row r, or -1
    return r < A.rs.n0 ? (r <= STEP_LDS ? r : -1) : (r - A.rs.n0 < STEP_LDS ? STEP_LDS + 1 + r - A.rs.n0 : -1);
  };
  const int ke = keff_of(A, b);
  const float T = PROBS ? 1.f : A.temps[b];
  auto used = [&](int r) { return r < per && (r < A.rs.n0 ? r <= ke : (r - A.rs.n0) < ke); };
  if (!PROBS && A.premerged && w > 0) {   // the given statistics of the staged rows (waves 1-3)
    for (int t = threadIdx.x - 64; t < 2 * STEP_LDS + 1; t += blockDim.x - 64) {
      const int r = t <= STEP_LDS ? t : A.rs.n0 + t - (STEP_LDS + 1);
      if (used(r)) sh_ms[t] = ms[r];
    }
  }
  // the statistics launch's chunk records of the first STEP_WAVES * STEP_ROWS rows, fetched before
  // wave 0 waits for its proposals
  const bool merge = !PROBS && !A.premerged && A.nch <= 64;
  const Stat none{-INFINITY, 0.f, -INFINITY, 0x7fffffff};
  Stat st0[STEP_ROWS];
  if (merge) {
#pragma unroll
    for (int i = 0; i < STEP_ROWS; ++i) {
      const int r = w + STEP_WAVES * i;
      st0[i] = used(r) && lane < A.nch ? A.stats[((int64_t)b * per + r) * A.nch + lane] : none;
    }
  }
  // wave 0, lane i: proposal i of the first 64 and its logits in the target and draft rows
  int x0 = -1;
  float u0 = 0.f, xp0 = 0.f, xq0 = 0.f;
  const int len0 = A.seq_len && w == 0 ? A.seq_len[b] : 0;
  if (w == 0 && lane < A.K) {
    x0 = A.draft[(int64_t)b * A.K + lane];
    u0 = A.u[(int64_t)b * A.K + lane];
    if (x0 >= 0 && x0 < A.V) {
      xp0 = Elem<DT>::load(row_ptr<DT>(A.rs, b, lane), x0);
      xq0 = Elem<DT>::load(row_ptr<DT>(A.rs, b, A.rs.n0 + lane), x0);
    }
  }
  if (!PROBS && !A.premerged) {   // the statistics launch's records
    Stat* mw = A.mstats + (int64_t)b * per;
    if (merge) {
      for (int r0 = 0; r0 < per; r0 += STEP_WAVES * STEP_ROWS) {
        Stat st[STEP_ROWS];
#pragma unroll
        for (int i = 0; i < STEP_ROWS; ++i) {
          const int r = r0 + w + STEP_WAVES * i;
          if (r0 == 0) {
            st[i] = st0[i];
          } else {
            st[i] = used(r) && lane < A.nch ? A.stats[((int64_t)b * per + r) * A.nch + lane] : none;
          }
        }
        Stat mg[STEP_ROWS];   // rows the sequence does not use merge to `none`, never stored
        merge_rows_wave<STEP_ROWS>(st, lane < A.nch, A.nch, mg);
#pragma unroll
        for (int i = 0; i < STEP_ROWS; ++i) {
          const int r = r0 + w + STEP_WAVES * i;
          if (lane == 0 && used(r)) {
            mw[r] = mg[i];
            if (slot_of(r) >= 0) sh_ms[slot_of(r)] = mg[i];
          }
        }
      }
    } else {
      for (int r = threadIdx.x; r < per; r += blockDim.x)
        if (used(r)) {
          const Stat m = merge_row(A.stats + ((int64_t)b * per + r) * A.nch, A.nch);
          mw[r] = m;
          if (slot_of(r) >= 0) sh_ms[slot_of(r)] = m;
        }
    }
    __threadfence_block();
  }
  __syncthreads();
  // the statistics of target row r (r <= ke) and of draft row r (r < ke)
  auto tstat = [&](int r) { return r <= STEP_LDS ? sh_ms[r] : ms[r]; };
  auto dstat = [&](int r) { return r < STEP_LDS ? sh_ms[STEP_LDS + 1 + r] : ms[A.rs.n0 + r]; };
  if (w != 0) return;
  int j = ke;
  for (int i0 = 0; i0 < ke && j == ke; i0 += 64) {
    const int i = i0 + lane;
    bool accept = false;
    if (i < ke) {
      int x = x0;
      float u = u0, xp = xp0, xq = xq0;
      if (i0 > 0) {   // proposals past the first 64
        x = A.draft[(int64_t)b * A.K + i];
        u = A.u[(int64_t)b * A.K + i];
        if (x >= 0 && x < A.V) {
          xp = Elem<DT>::load(row_ptr<DT>(A.rs, b, i), x);
          xq = Elem<DT>::load(row_ptr<DT>(A.rs, b, A.rs.n0 + i), x);
        }
      }
      if (x >= 0 && x < A.V) {   // an invalid proposal is never accepted
        float px, qx;
        if (PROBS) {
          px = xp;
          qx = xq;
        } else if (T > 0.f) {
          px = ProbFn(T, tstat(i))(xp);
          qx = ProbFn(T, dstat(i))(xq);
        } else {  // one-hot rows of the first argmax (sampling.py:11-12)
          px = tstat(i).ai == x ? 1.f : 0.f;
          qx = dstat(i).ai == x ? 1.f : 0.f;
        }
        const float ratio = qx > 0.f ? Elem<ProbType<DT, PROBS>::value>::round(px / qx) : 1.0f;  // speculative.py:26
        accept = u < fminf(1.0f, ratio);
        if (A.dbg_p) {
          A.dbg_p[(int64_t)b * A.K + i] = px;
          A.dbg_q[(int64_t)b * A.K + i] = qx;
        }
      }
    }
    const uint64_t rejected = __ballot(i < ke && !accept);
    if (rejected) j = i0 + __ffsll((unsigned long long)rejected) - 1;
  }
  if (!PROBS && T <= 0.f) {
    write_outputs(A, b, j, tstat(j).ai, OutPre{x0, len0});
    if (lane == 0 && A.dbg_s) A.dbg_s[b] = 0.f;
  } else if (lane == 0) {   // the outcome for the next launches
    A.jpos[b] = j;
    if (!PROBS) {
      A.pairstat[2 * b] = tstat(j);
      if (j < ke) A.pairstat[2 * b + 1] = dstat(j);
    }
  }
}

// The extra token is argmax_v fl(w_v / E_v) (multinomial as the argmax over Exp(1) noise), with
// w = p for the bonus token or when Σr = 0, and w = fl(r / S) otherwise (speculative.py:30-33); S = Σ r
// is known only once every chunk has summed its part. One pass therefore ranks the columns by cheap
// keys, p_v · rcp(E_v) and r_v · rcp(E_v). p_v, q_v and r_v = max(p_v - q_v, 0) are the exact values
// the final keys use (the same ProbFn, the same subtraction), so the cheap keys differ from the final
// keys (times S) only by the reciprocal and the last two roundings (under 3 float32 ulps, also where
// p_v and q_v nearly cancel) plus, for bf16/f16 probabilities, the rounding of r / S to that dtype. A
// column whose cheap key is below max · (1 - margin) cannot win, with the margin 8 or more times that
// error (2^-18 for float32 arithmetic, 2^-6 for bf16 probabilities, 2^-8 for f16). Each chunk keeps the columns
// within the margin of its own max (its candidates, nearly always one), and the draw scores them
// exactly. Chunks whose list overflowed, sequences whose max is too small for a relative bound, and a
// rejection whose residual sums to 0 (its draw falls back to p / E, which the pass does not rank) are
// rescanned exactly.
constexpr int NCAND = 8;
constexpr float CAND_MIN = 7.888609052210118e-31f;  // 2^-100: below it the bound is not relied on
constexpr float MARGIN_F32 = 1.0f / 262144.0f;     // 2^-18

template <int PD>
struct CandMargin {
  static constexpr float value = PD == FS_F32 ? MARGIN_F32 : (PD == FS_BF16 ? 1.0f / 64.0f : 1.0f / 256.0f);
};

FS_DEVICE float cand_threshold(float mx, float margin) { return isinf(mx) ? mx : mx - mx * margin; }

// p, q, the residual and the exact keys of a column of the rejected pair (the final draw's arithmetic)
template <int DT, bool PROBS>
struct PairRow {
  const typename Elem<DT>::T* pr;
  const typename Elem<DT>::T* qr;
  ProbFn sp, sq;
  FS_DEVICE float p_at(float x) const { return PROBS ? x : sp(x); }
  FS_DEVICE float q_at(float x) const { return PROBS ? x : sq(x); }
  FS_DEVICE float resid(float xp, float xq) const {   // (p - q).clamp(min=0)
    return fmaxf(Elem<ProbType<DT, PROBS>::value>::round(p_at(xp) - q_at(xq)), 0.f);
  }
  FS_DEVICE float key_p(int64_t v, float e) const { return p_at(Elem<DT>::load(pr, v)) / e; }
  FS_DEVICE float key_r(int64_t v, float s, float e) const {   // s > 0
    const float r = resid(Elem<DT>::load(pr, v), Elem<DT>::load(qr, v));
    return Elem<ProbType<DT, PROBS>::value>::round(r / s) / e;
  }
};

// Candidates of one set: the columns whose cheap key reaches the threshold, with the weight and
// Exp(1) value their exact key is computed from (LDS lists, first NCAND kept)
FS_DEVICE void collect(float key, int col, float w, float e, float th, int* n, int* list, float* wl, float* el) {
  if (key >= th) {
    const int k = atomicAdd(n, 1);
    if (k < NCAND) {
      list[k] = col;
      wl[k] = w;
      el[k] = e;
    }
  }
}

// What a pair item learns from its sequence's step (written by the step launch).
struct PairCtx {
  int j;
  Stat sp, sq;
};

template <bool PROBS>
FS_DEVICE PairCtx read_step(const AcceptArgs& A, int b) {
  PairCtx pc;
  pc.j = A.jpos[b];
  if (!PROBS) {
    pc.sp = A.pairstat[2 * b];
    pc.sq = A.pairstat[2 * b + 1];
  }
  return pc;
}

// One chunk of CHR columns of the draw of sequence b: the residual partial sum and the max and
// candidates of the draw's keys (r / E at a rejection, p / E for the bonus token), written as records.
// The rows' addresses depend on the step's outcome, so it is read first and waited for before any
// load of the chunk is issued: issued after them it would queue behind every item's chunk stream.
template <int DT, bool PROBS>
FS_DEVICE void pair_chunk(const AcceptArgs& A, int b, int c, const PairCtx& pc, float* shf, int* sh_n, int* sh_c,
                          float* sh_w, float* sh_e) {
  constexpr int PD = ProbType<DT, PROBS>::value;
  const int ke = keff_of(A, b);
  const float T = PROBS ? 1.f : A.temps[b];
  const int j = pc.j;
  const bool bonus = j >= ke;
  ProbFn sp, sq;
  if (!PROBS) {
    sp = ProbFn(T, pc.sp);
    if (!bonus) sq = ProbFn(T, pc.sq);
  }
  const auto* pr = row_ptr<DT>(A.rs, b, j);
  const auto* qr = bonus ? pr : row_ptr<DT>(A.rs, b, A.rs.n0 + j);
  const bool vec_ok = (A.V % VEC) == 0 &&
                      (((reinterpret_cast<uintptr_t>(pr) | reinterpret_cast<uintptr_t>(qr)) & 15) == 0);
  const float* er = A.E + (int64_t)b * A.ldE;
  const bool evec_ok = (A.V % VEC) == 0 && ((reinterpret_cast<uintptr_t>(er) & 15) == 0);
  __builtin_amdgcn_sched_barrier(0);   // j is in hand before the first load below is issued
  float xp[UNROLL_R][8], xq[UNROLL_R][8], e[UNROLL_R][8];   // every load in flight before any arithmetic
  const int64_t vb = (int64_t)c * CHR + (int64_t)threadIdx.x * VEC;
  if (block_in_range<UNROLL_R>(vb, A.V, vec_ok && evec_ok)) {
    Raw8<DT> rp[UNROLL_R], rq[UNROLL_R];
    Raw8<FS_F32> re[UNROLL_R];
#pragma unroll
    for (int u = 0; u < UNROLL_R; ++u) {   // for the bonus token qr is pr: a second read of the same lines
      rp[u].load(pr, vb + u * THREADS * VEC);
      rq[u].load(qr, vb + u * THREADS * VEC);
      re[u].load(er, vb + u * THREADS * VEC);
    }
    __builtin_amdgcn_sched_barrier(0);
#pragma unroll
    for (int u = 0; u < UNROLL_R; ++u) {
      rp[u].to_f32(xp[u]);
      rq[u].to_f32(xq[u]);
      re[u].to_f32(e[u]);
    }
  } else {
    load_block<DT, UNROLL_R>(pr, vb, A.V, vec_ok, 0.f, xp);
    if (!bonus) load_block<DT, UNROLL_R>(qr, vb, A.V, vec_ok, 0.f, xq);
    load_block<FS_F32, UNROLL_R>(er, vb, A.V, evec_ok, 1.f, e);
  }
  if (!PROBS) {   // y = x / T once per element (the ProbFn arithmetic, divided ahead)
    divide_by_t(xp, T);
    if (!bonus) divide_by_t(xq, T);
  }
  // One set of cheap keys: p / E for the bonus token, r / E at a rejection. The p / E set of a
  // rejection is needed only when the residual sums to 0; its chunks are then rescanned exactly.
  float ls = 0.f, mk = 0.f;
  float ak[UNROLL_R][8];   // cheap keys (0 past the row)
  float wv[UNROLL_R][8];   // the exact keys' weights: p_v for the bonus token, r_v at a rejection
#pragma unroll
  for (int u = 0; u < UNROLL_R; ++u) {
    const int64_t v0 = (int64_t)c * CHR + (int64_t)(threadIdx.x + THREADS * u) * VEC;
#pragma unroll
    for (int jj = 0; jj < 8; ++jj) {
      const bool in = v0 + jj < A.V;
      const float re = __builtin_amdgcn_rcpf(e[u][jj]);
      const float p = PROBS ? xp[u][jj] : sp.of_y(xp[u][jj]);
      if (bonus) {
        wv[u][jj] = p;
        ak[u][jj] = in ? p * re : 0.f;
      } else {   // (p - q).clamp(min=0), rounded to the probability dtype
        const float q = PROBS ? xq[u][jj] : sq.of_y(xq[u][jj]);
        const float r = in ? fmaxf(Elem<PD>::round(p - q), 0.f) : 0.f;
        ls += r;
        wv[u][jj] = r;
        ak[u][jj] = r * re;
      }
      mk = fmaxf(mk, ak[u][jj]);
    }
  }
  const float tot = bonus ? 0.f : block_sum(ls, shf);
  const float cm = block_max(mk, shf);
  if (threadIdx.x == 0) sh_n[0] = 0;
  __syncthreads();
  const float th = cm > 0.f ? cand_threshold(cm, bonus ? MARGIN_F32 : CandMargin<PD>::value) : INFINITY;
#pragma unroll
  for (int u = 0; u < UNROLL_R; ++u) {
    const int64_t v0 = (int64_t)c * CHR + (int64_t)(threadIdx.x + THREADS * u) * VEC;
#pragma unroll
    for (int jj = 0; jj < 8; ++jj)
      collect(ak[u][jj], (int)(v0 + jj), wv[u][jj], e[u][jj], th, &sh_n[0], sh_c, sh_w, sh_e);
  }
  __syncthreads();
  const int64_t o = (int64_t)b * A.nchr + c;
  if (threadIdx.x < 64) {   // wave 0 writes the chunk's records
    const int n = cm > 0.f ? sh_n[0] : 0;
    if ((int)threadIdx.x < NCAND && (int)threadIdx.x < n) {
      A.cand[o * NCAND + threadIdx.x] = sh_c[threadIdx.x];
      A.candw[o * NCAND + threadIdx.x] = sh_w[threadIdx.x];
      A.cande[o * NCAND + threadIdx.x] = sh_e[threadIdx.x];
    }
    if (threadIdx.x == 0) {
      A.resid[o] = tot;
      A.cmax[o] = cm;
      A.ncand[o] = n;
    }
  }
}

// The draw of sequence b, run by one wave from the records of its chunks: S summed
// over the chunks in increasing order, then the exact keys of the candidates of every chunk whose max
// reaches the margin (first index on ties); writes the tokens, n_accepted and the rollback length.
// Chunks are taken 32 at a time, lanes l and l + 32 on chunk l: both fetch its records, each half of
// its candidates' (column, weight, E), all at once, so a draw waits for one round trip; only a chunk
// that is rescanned (its list overflowed, or the bound is not relied on) reads the logits and E again.
constexpr int DRAW_CHUNKS = 32;
constexpr int CAND_HALF = NCAND / 2;

template <int DT, bool PROBS>
FS_DEVICE void final_draw(const AcceptArgs& A, int b) {
  constexpr int PD = ProbType<DT, PROBS>::value;
  const int lane = threadIdx.x;
  const int cl = lane & (DRAW_CHUNKS - 1), half = lane / DRAW_CHUNKS;
  const int64_t o0 = (int64_t)b * A.nchr;
  struct Chunk {
    float rc, cmx;
    int n;
    int col[CAND_HALF];
    float w[CAND_HALF], e[CAND_HALF];
  };
  auto fetch = [&](int c0) {   // chunk c0 + cl, candidates half * CAND_HALF .. (zeros past the last chunk)
    Chunk k;
    const bool in = c0 + cl < A.nchr;
    const int64_t o = o0 + (in ? c0 + cl : 0);
    k.rc = in ? A.resid[o] : 0.f;
    k.cmx = in ? A.cmax[o] : 0.f;
    k.n = in ? A.ncand[o] : 0;
#pragma unroll
    for (int i = 0; i < CAND_HALF; ++i) {
      const int64_t q = o * NCAND + half * CAND_HALF + i;
      k.col[i] = in ? A.cand[q] : 0;
      k.w[i] = in ? A.candw[q] : 0.f;
      k.e[i] = in ? A.cande[q] : 1.f;
    }
    return k;
  };
  // every load that depends on nothing goes out before the first is used (a greedy sequence, finished
  // by its step, reads stale records and returns)
  const Chunk k0 = fetch(0);
  const OutPre pre = out_pre(A, b);
  const PairCtx pc = read_step<PROBS>(A, b);
  const float T = PROBS ? 1.f : A.temps[b];
  const int ke = keff_of(A, b);
  if (T <= 0.f) return;
  const int j = pc.j;
  const bool bonus = j >= ke;
  float s = 0.f;
  if (!bonus) {
    for (int c0 = 0; c0 < A.nchr; c0 += DRAW_CHUNKS) {
      const float rc = c0 == 0 ? k0.rc : (c0 + cl < A.nchr ? A.resid[o0 + c0 + cl] : 0.f);
      const int n = min(DRAW_CHUNKS, A.nchr - c0);
      for (int k = 0; k < n; ++k) s += __int_as_float(__builtin_amdgcn_readlane(__float_as_int(rc), k));
    }
    s = Elem<PD>::round(s);
  }
  // set p: w = p (speculative.py:31, 33): the bonus token, or a rejection whose residual sums to 0,
  // whose chunks were not ranked for p / E and are all rescanned; set r: w = r / S
  const bool set_r = !bonus && s > 0.f;
  const bool rescan_all = !bonus && !set_r;
  float gmax = 0.f;
  if (!rescan_all) {
    for (int c0 = 0; c0 < A.nchr; c0 += DRAW_CHUNKS)
      gmax = fmaxf(gmax, c0 == 0 ? k0.cmx : (c0 + cl < A.nchr ? A.cmax[o0 + c0 + cl] : 0.f));
    gmax = wave_max(gmax);
  }
  const bool trust = !rescan_all && gmax >= CAND_MIN;
  const float th = cand_threshold(gmax, set_r ? CandMargin<PD>::value : MARGIN_F32);
  ProbFn sp, sq;
  if (!PROBS) {
    sp = ProbFn(T, pc.sp);
    if (!bonus) sq = ProbFn(T, pc.sq);
  }
  const auto* pr = row_ptr<DT>(A.rs, b, j);
  const PairRow<DT, PROBS> pair{pr, bonus ? pr : row_ptr<DT>(A.rs, b, A.rs.n0 + j), sp, sq};
  const float* er = A.E + (int64_t)b * A.ldE;
  auto key = [&](int64_t col) { return set_r ? pair.key_r(col, s, er[col]) : pair.key_p(col, er[col]); };
  float v = -INFINITY;
  int extra = 0x7fffffff;
  for (int c0 = 0; c0 < A.nchr; c0 += DRAW_CHUNKS) {
    const Chunk k = c0 == 0 ? k0 : fetch(c0);
    const bool keep = c0 + cl < A.nchr && (!trust || k.cmx >= th);
    const bool listed = keep && trust && k.n <= NCAND;
    if (listed) {   // this half of the chunk's candidates, scored from their records (the exact keys)
#pragma unroll
      for (int i = 0; i < CAND_HALF; ++i)
        if (half * CAND_HALF + i < k.n)
          argmax_merge(v, extra, set_r ? Elem<PD>::round(k.w[i] / s) / k.e[i] : k.w[i] / k.e[i], k.col[i]);
    }
    uint64_t rescan = __ballot(keep && !listed && half == 0);
    while (rescan) {   // exact rescan of the chunk by the whole wave
      const int l = __ffsll((unsigned long long)rescan) - 1;
      rescan &= rescan - 1;
      const int c = c0 + l;
      const int64_t hi = min((int64_t)(c + 1) * CHR, A.V);
      for (int64_t col = (int64_t)c * CHR + lane; col < hi; col += 64) argmax_merge(v, extra, key(col), (int)col);
    }
  }
  wave_argmax(v, extra);
  write_outputs(A, b, j, extra, pre);
  if (lane == 0 && A.dbg_s) A.dbg_s[b] = s;
}

// statistics launch (logits without given statistics): per-(row, chunk) statistics of every row a
// sequence uses
template <int DT>
__global__ void __launch_bounds__(THREADS) accept_stats_kernel(AcceptArgs A) {
  __shared__ float shf[THREADS / 64];
  __shared__ int shi[THREADS / 64];
  const int c = blockIdx.x;
  const int rho = blockIdx.y;
  const int per = A.rs.n0 + A.rs.n1;
  const int b = rho / per, i = rho - b * per;
  const int ke = keff_of(A, b);
  if (i < A.rs.n0 ? i > ke : (i - A.rs.n0) >= ke) return;  // a row this sequence does not use
  const float T = A.temps[b];
  const auto* row = row_ptr<DT>(A.rs, b, i);
  const Stat st = chunk_stat<DT>(row, c, A.V, T, shf, shi);
  if (threadIdx.x == 0) A.stats[(int64_t)rho * A.nch + c] = st;
}

// B step items, one sequence each.
template <int DT, bool PROBS>
__global__ void __launch_bounds__(THREADS) accept_step_kernel(AcceptArgs A) {
  __shared__ Stat sh_ms[2 * STEP_LDS + 1];
  sequence_step<DT, PROBS>(A, blockIdx.x, sh_ms);
}

// B * nchr pair items (sequence by sequence).
template <int DT, bool PROBS>
__global__ void __launch_bounds__(THREADS) accept_kernel(AcceptArgs A) {
  __shared__ float shf[THREADS / 64];
  __shared__ int sh_n[1];
  __shared__ int sh_c[NCAND];
  __shared__ float sh_w[NCAND], sh_e[NCAND];
  const int item = blockIdx.x;
  const int b = item / A.nchr, c = item - b * A.nchr;
  // a pair item of a sampled sequence (greedy sequences were finished by their step)
  const float T = PROBS ? 1.f : A.temps[b];
  const PairCtx pc = read_step<PROBS>(A, b);   // loaded with T (stale for a greedy sequence, unused)
  if (T <= 0.f) return;
  pair_chunk<DT, PROBS>(A, b, c, pc, shf, sh_n, sh_c, sh_w, sh_e);
}

// B draws, one wave each.
template <int DT, bool PROBS>
__global__ void __launch_bounds__(64) accept_draw_kernel(AcceptArgs A) {
  final_draw<DT, PROBS>(A, blockIdx.x);
}

// ------------------------------------------------------------------------------------------------
// probs_from_logits
// ------------------------------------------------------------------------------------------------
template <int DT>
__global__ void __launch_bounds__(THREADS) probs_kernel(RowSet rs, int64_t V, int nch, float T,
                                                        const Stat* __restrict__ stats, void* __restrict__ out,
                                                        int64_t ldo) {
  __shared__ Stat shs;
  const int c = blockIdx.x, r = blockIdx.y;
  if (threadIdx.x == 0) shs = merge_row(stats + (int64_t)r * nch, nch);
  __syncthreads();
  const Stat st = shs;
  const auto* row = row_ptr<DT>(rs, r, 0);
  for (int u = 0; u < UNROLL * VEC; ++u) {
    const int64_t v = (int64_t)c * CH + (int64_t)u * THREADS + threadIdx.x;
    if (v >= V) break;
    if (T > 0.f) {
      reinterpret_cast<float*>(out)[(int64_t)r * ldo + v] = ProbFn(T, st)(Elem<DT>::load(row, v));
    } else {
      Elem<DT>::store(reinterpret_cast<typename Elem<DT>::T*>(out), (int64_t)r * ldo + v, v == st.ai ? 1.f : 0.f);
    }
  }
}

// ------------------------------------------------------------------------------------------------
// row statistics from per-block partials (the LM head GEMM's epilogue)
// ------------------------------------------------------------------------------------------------
// One workgroup per row, one pass: each thread folds blocks p = tid, tid + THREADS, ... in order into
// a running (max, sum) (the sum rescaled when the max grows) and a first argmax; the threads are then
// combined in the block-reduction order. Row m's records are at parts + m * ld; the merged record
// goes to out[(m / group) * gstride + m % group + offset].
__global__ void __launch_bounds__(THREADS) row_stats_merge_kernel(const Stat* __restrict__ parts, int64_t ld,
                                                                  int64_t nparts, Stat* __restrict__ out, int group,
                                                                  int64_t gstride, int64_t offset) {
  __shared__ float shf[THREADS / 64];
  __shared__ int shi[THREADS / 64];
  const int64_t m = blockIdx.x;
  const Stat* pr = parts + m * ld;
  float mt = -INFINITY, st = 0.f, av = -INFINITY;
  int ai = 0x7fffffff;
  for (int64_t p = threadIdx.x; p < nparts; p += THREADS) {
    const Stat x = pr[p];
    argmax_merge(av, ai, x.av, x.ai);
    if (x.m == -INFINITY) continue;
    if (x.m > mt) {
      st = st * __builtin_amdgcn_exp2f((mt - x.m) * LOG2E_F) + x.s;   // exp2(-inf) = 0 while empty
      mt = x.m;
    } else {
      st += x.s * __builtin_amdgcn_exp2f((x.m - mt) * LOG2E_F);
    }
  }
  const float M = block_max(mt, shf);
  block_argmax(av, ai, shf, shi);
  const float S = block_sum(mt == -INFINITY ? 0.f : st * __builtin_amdgcn_exp2f((mt - M) * LOG2E_F), shf);
  if (threadIdx.x == 0) out[(m / group) * gstride + m % group + offset] = Stat{M, S, av, ai};
}

// ------------------------------------------------------------------------------------------------
// workspace carving
// ------------------------------------------------------------------------------------------------
struct Carve {
  char* p;
  int64_t used = 0;
  template <typename T>
  T* take(int64_t n) {
    T* r = reinterpret_cast<T*>(p + used);
    used += ((n * (int64_t)sizeof(T) + 255) / 256) * 256;
    return r;
  }
};

int64_t nchunks(int64_t V) { return (V + CH - 1) / CH; }

int64_t nchunks_r(int64_t V) { return (V + CHR - 1) / CHR; }

int64_t accept_ws(int64_t B, int64_t K, int64_t V) {
  const int64_t nch = nchunks(V), nchr = nchunks_r(V);
  auto r = [](int64_t n) { return ((n + 255) / 256) * 256; };
  return r(B * (2 * K + 1) * nch * (int64_t)sizeof(Stat)) + r(B * (2 * K + 1) * (int64_t)sizeof(Stat)) +
         r(B * 2 * (int64_t)sizeof(Stat)) + 3 * r(B * nchr * 4) + 3 * r(B * nchr * NCAND * 4) + r(B * 4);
}

void carve_accept(AcceptArgs& A, void* workspace, int64_t B, int64_t K, int nch, int nchr) {
  Carve cv{reinterpret_cast<char*>(workspace)};
  A.stats = cv.take<Stat>(B * (2 * K + 1) * nch);
  A.mstats = cv.take<Stat>(B * (2 * K + 1));
  A.pairstat = cv.take<Stat>(B * 2);
  A.resid = cv.take<float>(B * nchr);
  A.cmax = cv.take<float>(B * nchr);
  A.ncand = cv.take<int>(B * nchr);
  A.cand = cv.take<int>(B * nchr * NCAND);
  A.candw = cv.take<float>(B * nchr * NCAND);
  A.cande = cv.take<float>(B * nchr * NCAND);
  A.jpos = cv.take<int>(B);
  A.premerged = false;
}

bool dtype_ok(int32_t dt) { return dt == FS_F32 || dt == FS_BF16 || dt == FS_F16; }

// The statistics launch (logits without given statistics), then B step items, B * nchr pair items
// and B draws.
template <int DT>
int launch_accept(const AcceptArgs& A, bool probs, hipStream_t s) {
  const int64_t total = (int64_t)A.B * A.nchr;
  if (total * THREADS >= ((int64_t)1 << 32))
    return fs::arg_error("spec_accept: %lld work items exceed one launch", (long long)total);
  if (probs) {
    accept_step_kernel<DT, true><<<dim3((unsigned)A.B), THREADS, 0, s>>>(A);
    accept_kernel<DT, true><<<dim3((unsigned)total), THREADS, 0, s>>>(A);
    accept_draw_kernel<DT, true><<<dim3((unsigned)A.B), 64, 0, s>>>(A);
  } else {
    const int per = A.rs.n0 + A.rs.n1;
    if (!A.premerged) accept_stats_kernel<DT><<<dim3((unsigned)A.nch, (unsigned)(A.B * per)), THREADS, 0, s>>>(A);
    accept_step_kernel<DT, false><<<dim3((unsigned)A.B), THREADS, 0, s>>>(A);
    accept_kernel<DT, false><<<dim3((unsigned)total), THREADS, 0, s>>>(A);
    accept_draw_kernel<DT, false><<<dim3((unsigned)A.B), 64, 0, s>>>(A);
  }
  return fs::launch_status("spec_accept");
}

}  // namespace

extern "C" int64_t fs_sampling_workspace_size(int64_t R, int64_t V) {
  if (R <= 0 || V <= 0) return 0;
  const int64_t nch = nchunks(V);
  auto r = [](int64_t n) { return ((n + 255) / 256) * 256; };
  return r(R * nch * (int64_t)sizeof(Stat)) + 2 * r(R * nch * 4) + r(4);
}

extern "C" int64_t fs_spec_accept_workspace_size(int32_t B, int32_t K, int64_t V) {
  if (B <= 0 || K < 0 || V <= 0) return 0;
  return accept_ws(B, K, V);
}

extern "C" int fs_sample_logits(const void* logits, int64_t ld, int64_t R, int64_t V, const float* temperature,
                                float temperature_all, const float* E, int64_t ldE, int32_t dtype, int64_t* tokens_out,
                                int32_t* tokens_out32, int64_t ld_tok32, void* workspace, int64_t workspace_bytes,
                                void* stream) {
  FS_CHECK_ARG(logits && tokens_out && workspace, "sample_logits: null pointer");
  FS_CHECK_ARG(dtype_ok(dtype), "sample_logits: dtype %d", dtype);
  FS_CHECK_ARG(R >= 0 && V > 0 && V < 0x7fffffff && ld >= V, "sample_logits: R %lld V %lld", (long long)R,
               (long long)V);
  FS_CHECK_ARG(temperature || temperature_all >= 0.f, "sample_logits: temperature %f", (double)temperature_all);
  FS_CHECK_ARG(!E || ldE >= V, "sample_logits: ldE %lld < V", (long long)ldE);
  FS_CHECK_ARG(workspace_bytes >= fs_sampling_workspace_size(R, V), "sample_logits: workspace too small");
  FS_CHECK_ARG(R <= 65535, "sample_logits: at most 65535 rows per call");
  if (R == 0) return 0;
  const int nch = (int)nchunks(V);
  Carve cv{reinterpret_cast<char*>(workspace)};
  Stat* st = cv.take<Stat>(R * nch);
  float* pv = cv.take<float>(R * nch);
  int* pi = cv.take<int>(R * nch);
  RowSet rs{logits, ld, 0, 1, nullptr, 0, 0, 0};
  hipStream_t s = fs::as_stream(stream);
  const bool greedy_only = E == nullptr;
  // with no noise every row takes the argmax; the statistics pass then only needs the argmax
  const float t_stats = greedy_only ? 0.f : temperature_all;
  const float* t_ptr = greedy_only ? nullptr : temperature;
#define FS_LAUNCH(DT)                                                                                                  \
  stats_kernel<DT><<<dim3((unsigned)nch, (unsigned)R), THREADS, 0, s>>>(rs, V, nch, t_ptr, t_stats, nullptr, st);     \
  if (!greedy_only)                                                                                                    \
    sample_argmax_kernel<DT><<<dim3((unsigned)nch, (unsigned)R), THREADS, 0, s>>>(rs, V, nch, temperature,             \
                                                                                 temperature_all, st, E, ldE, pv, pi);
  switch (dtype) {
    case FS_F32: FS_LAUNCH(FS_F32); break;
    case FS_BF16: FS_LAUNCH(FS_BF16); break;
    default: FS_LAUNCH(FS_F16); break;
  }
#undef FS_LAUNCH
  sample_final_kernel<<<dim3((unsigned)((R + 63) / 64)), 64, 0, s>>>((int)R, nch, temperature, temperature_all,
                                                                     greedy_only, st, pv, pi, tokens_out, tokens_out32,
                                                                     ld_tok32);
  return fs::launch_status("sample_logits");
}

extern "C" int fs_probs_from_logits(const void* logits, int64_t ld, int64_t R, int64_t V, float temperature,
                                    int32_t dtype, void* out, int64_t ldo, int32_t out_dtype, void* workspace,
                                    int64_t workspace_bytes, void* stream) {
  FS_CHECK_ARG(logits && out && workspace, "probs_from_logits: null pointer");
  FS_CHECK_ARG(dtype_ok(dtype), "probs_from_logits: dtype %d", dtype);
  FS_CHECK_ARG(temperature >= 0.f, "probs_from_logits: temperature %f", (double)temperature);
  FS_CHECK_ARG(temperature > 0.f ? out_dtype == FS_F32 : out_dtype == dtype,
               "probs_from_logits: out dtype must be f32 (T > 0) or the logits dtype (T == 0)");
  FS_CHECK_ARG(R >= 0 && R <= 65535 && V > 0 && V < 0x7fffffff && ld >= V && ldo >= V, "probs_from_logits: shapes");
  FS_CHECK_ARG(workspace_bytes >= fs_sampling_workspace_size(R, V), "probs_from_logits: workspace too small");
  if (R == 0) return 0;
  const int nch = (int)nchunks(V);
  Carve cv{reinterpret_cast<char*>(workspace)};
  Stat* st = cv.take<Stat>(R * nch);
  RowSet rs{logits, ld, 0, 1, nullptr, 0, 0, 0};
  hipStream_t s = fs::as_stream(stream);
  dim3 grid((unsigned)nch, (unsigned)R);
#define FS_LAUNCH(DT)                                                                           \
  stats_kernel<DT><<<grid, THREADS, 0, s>>>(rs, V, nch, nullptr, temperature, nullptr, st);  \
  probs_kernel<DT><<<grid, THREADS, 0, s>>>(rs, V, nch, temperature, st, out, ldo);
  switch (dtype) {
    case FS_F32: FS_LAUNCH(FS_F32); break;
    case FS_BF16: FS_LAUNCH(FS_BF16); break;
    default: FS_LAUNCH(FS_F16); break;
  }
#undef FS_LAUNCH
  return fs::launch_status("probs_from_logits");
}

namespace {
int spec_accept_impl(const void* tgt, int64_t tgt_sb, int64_t tgt_si, const void* dft, int64_t dft_sb, int64_t dft_si,
                     int32_t B, int32_t K, int64_t V, int32_t dtype, const int32_t* draft_tokens, const int32_t* k_eff,
                     const float* temperature, const float* u, const float* E, int64_t ldE, int32_t* out_tokens,
                     int32_t* n_accepted, int32_t* seq_len, float* p_x, float* q_x, float* res_sum,
                     const void* row_stats, void* workspace, int64_t workspace_bytes, void* stream) {
  FS_CHECK_ARG(tgt && temperature && out_tokens && n_accepted && workspace, "spec_accept: null pointer");
  FS_CHECK_ARG((p_x == nullptr) == (q_x == nullptr) && (p_x == nullptr) == (res_sum == nullptr),
               "spec_accept: p_x, q_x and res_sum are given together or not at all");
  FS_CHECK_ARG(K == 0 || (dft && draft_tokens && u), "spec_accept: null draft inputs");
  FS_CHECK_ARG(E != nullptr, "spec_accept: E (Exp(1) noise) is required");
  FS_CHECK_ARG(dtype_ok(dtype), "spec_accept: dtype %d", dtype);
  FS_CHECK_ARG(B > 0 && B <= 65535 && K >= 0 && V > 0 && V < 0x7fffffff, "spec_accept: B %d K %d V %lld", B, K,
               (long long)V);
  FS_CHECK_ARG(workspace_bytes >= accept_ws(B, K, V), "spec_accept: workspace %lld < %lld", (long long)workspace_bytes,
               (long long)accept_ws(B, K, V));
  const int nch = (int)nchunks(V);
  AcceptArgs A;
  A.rs = RowSet{tgt, tgt_sb, tgt_si, K + 1, dft ? dft : tgt, dft_sb, dft_si, K};
  A.K = K;
  A.V = V;
  A.nch = nch;
  A.nchr = (int)nchunks_r(V);
  A.B = B;
  A.draft = draft_tokens;
  A.k_eff = k_eff;
  A.temps = temperature;
  A.u = u;
  A.E = E;
  A.ldE = ldE;
  A.out_tokens = out_tokens;
  A.n_acc = n_accepted;
  A.seq_len = seq_len;
  A.dbg_p = p_x;
  A.dbg_q = q_x;
  A.dbg_s = res_sum;
  carve_accept(A, workspace, B, K, nch, A.nchr);
  if (row_stats) {
    FS_CHECK_ARG((reinterpret_cast<uintptr_t>(row_stats) & 15) == 0, "spec_accept: row statistics not 16-byte aligned");
    A.mstats = const_cast<Stat*>(reinterpret_cast<const Stat*>(row_stats));   // read only
  }
  A.premerged = row_stats != nullptr;
  hipStream_t s = fs::as_stream(stream);
  switch (dtype) {
    case FS_F32: return launch_accept<FS_F32>(A, false, s);
    case FS_BF16: return launch_accept<FS_BF16>(A, false, s);
    default: return launch_accept<FS_F16>(A, false, s);
  }
}
}  // namespace

extern "C" int fs_spec_accept(const void* tgt, int64_t tgt_sb, int64_t tgt_si, const void* dft, int64_t dft_sb,
                              int64_t dft_si, int32_t B, int32_t K, int64_t V, int32_t dtype,
                              const int32_t* draft_tokens, const int32_t* k_eff, const float* temperature,
                              const float* u, const float* E, int64_t ldE, int32_t* out_tokens, int32_t* n_accepted,
                              int32_t* seq_len, float* p_x, float* q_x, float* res_sum, void* workspace,
                              int64_t workspace_bytes, void* stream) {
  return spec_accept_impl(tgt, tgt_sb, tgt_si, dft, dft_sb, dft_si, B, K, V, dtype, draft_tokens, k_eff, temperature, u,
                          E, ldE, out_tokens, n_accepted, seq_len, p_x, q_x, res_sum, nullptr, workspace,
                          workspace_bytes, stream);
}

extern "C" int fs_spec_accept_stats(const void* tgt, int64_t tgt_sb, int64_t tgt_si, const void* dft, int64_t dft_sb,
                                    int64_t dft_si, int32_t B, int32_t K, int64_t V, int32_t dtype,
                                    const int32_t* draft_tokens, const int32_t* k_eff, const float* temperature,
                                    const float* u, const float* E, int64_t ldE, const void* row_stats,
                                    int32_t* out_tokens, int32_t* n_accepted, int32_t* seq_len, float* p_x,
                                    float* q_x, float* res_sum, void* workspace, int64_t workspace_bytes,
                                    void* stream) {
  FS_CHECK_ARG(row_stats != nullptr, "spec_accept_stats: null row statistics");
  return spec_accept_impl(tgt, tgt_sb, tgt_si, dft, dft_sb, dft_si, B, K, V, dtype, draft_tokens, k_eff, temperature, u,
                          E, ldE, out_tokens, n_accepted, seq_len, p_x, q_x, res_sum, row_stats, workspace,
                          workspace_bytes, stream);
}

// ------------------------------------------------------------------------------------------------
// the acceptance without a caller workspace (for callers that cannot allocate)
// ------------------------------------------------------------------------------------------------
// Scratch of fs_spec_accept_noalloc: a fixed device array that each GPU holds for the life of the
// process. Its size bounds the shapes that entry point takes (batch 512 at k = 8 and a 128256-token
// vocabulary needs 3.96 MiB). Calls on one GPU share it: calls that overlap on one device race.
constexpr int64_t NOALLOC_SCRATCH_BYTES = (int64_t)4 << 20;
static __device__ __align__(256) char scratch[NOALLOC_SCRATCH_BYTES];

namespace {
constexpr int MAX_DEVICES = 64;
std::mutex scratch_mu;
void* scratch_ptr[MAX_DEVICES] = {};   // the array's device address on each GPU, looked up once per device

// The scratch address on the current device: hipGetSymbolAddress the first time a device calls, with
// that device current (outside any stream capture), the cached pointer afterwards. The acceptance
// needs no initial contents in its workspace. In host code `scratch` only names a host-side stand-in
// for the array, so kernels always receive this pointer.
int scratch_on_current_device(hipStream_t stream, void** out) {
  int dev = -1;
  hipError_t e = hipGetDevice(&dev);
  if (e != hipSuccess) {
    fs::set_error("spec_accept_noalloc: hipGetDevice: %s", hipGetErrorString(e));
    return (int)e;
  }
  if (dev < 0 || dev >= MAX_DEVICES) return fs::arg_error("spec_accept_noalloc: device %d (at most %d)", dev, MAX_DEVICES);
  std::lock_guard<std::mutex> lock(scratch_mu);
  if (!scratch_ptr[dev]) {
    hipStreamCaptureStatus cs = hipStreamCaptureStatusNone;
    e = hipStreamIsCapturing(stream, &cs);
    if (e != hipSuccess) {
      fs::set_error("spec_accept_noalloc: hipStreamIsCapturing: %s", hipGetErrorString(e));
      return (int)e;
    }
    if (cs != hipStreamCaptureStatusNone)
      return fs::arg_error("spec_accept_noalloc: the first call on device %d is being captured; make one call "
                           "on this device before capturing", dev);
    void* p = nullptr;
    e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
    if (e != hipSuccess || p == nullptr) {
      fs::set_error("spec_accept_noalloc: hipGetSymbolAddress: %s", hipGetErrorString(e));
      return e != hipSuccess ? (int)e : (int)hipErrorInvalidSymbol;
    }
    scratch_ptr[dev] = p;
  }
  *out = scratch_ptr[dev];
  return 0;
}
}  // namespace

extern "C" int fs_spec_accept_noalloc(const void* tgt, int64_t tgt_sb, int64_t tgt_si, const void* dft, int64_t dft_sb,
                                      int64_t dft_si, int32_t B, int32_t K, int64_t V, int32_t dtype,
                                      const int32_t* draft_tokens, const int32_t* k_eff, const float* temperature,
                                      const float* u, const float* E, int64_t ldE, const void* row_stats,
                                      int32_t* out_tokens, int32_t* n_accepted, int32_t* seq_len, void* stream) {
  FS_CHECK_ARG(B > 0 && B <= 65535 && K >= 0 && K <= 65535 && V > 0 && V < 0x7fffffff,
               "spec_accept_noalloc: B %d K %d V %lld", B, K, (long long)V);
  const int64_t need = accept_ws(B, K, V);
  FS_CHECK_ARG(need <= NOALLOC_SCRATCH_BYTES,
               "spec_accept_noalloc: B %d K %d V %lld needs %lld bytes of scratch, more than the %lld this entry "
               "point holds per device; use fs_spec_accept with a workspace",
               B, K, (long long)V, (long long)need, (long long)NOALLOC_SCRATCH_BYTES);
  void* ws = nullptr;
  if (int rc = scratch_on_current_device(fs::as_stream(stream), &ws)) return rc;
  return spec_accept_impl(tgt, tgt_sb, tgt_si, dft, dft_sb, dft_si, B, K, V, dtype, draft_tokens, k_eff, temperature, u,
                          E, ldE, out_tokens, n_accepted, seq_len, nullptr, nullptr, nullptr, row_stats, ws,
                          NOALLOC_SCRATCH_BYTES, stream);
}

extern "C" int fs_row_stats_merge(const void* parts, int64_t parts_ld, int64_t nparts, int64_t M, void* out,
                                  int32_t group, int64_t gstride, int64_t offset, void* stream) {
  FS_CHECK_ARG(parts && out, "row_stats_merge: null pointer");
  FS_CHECK_ARG(nparts > 0 && parts_ld >= nparts && M >= 0 && M <= 0x7fffffff && group >= 1 && gstride >= 0 &&
                   offset >= 0,
               "row_stats_merge: nparts %lld ld %lld M %lld group %d", (long long)nparts, (long long)parts_ld,
               (long long)M, group);
  if (M == 0) return 0;
  row_stats_merge_kernel<<<dim3((unsigned)M), THREADS, 0, fs::as_stream(stream)>>>(
      reinterpret_cast<const Stat*>(parts), parts_ld, nparts, reinterpret_cast<Stat*>(out), group, gstride, offset);
  return fs::launch_status("row_stats_merge");
}

extern "C" int fs_verify_probs(const void* p, int64_t ldp, const void* q, int64_t ldq, int32_t K, int64_t V,
                               int32_t dtype, const int32_t* draft_tokens, const float* u, const float* E,
                               int32_t* out_tokens, int32_t* n_accepted, void* workspace, int64_t workspace_bytes,
                               void* stream) {
  FS_CHECK_ARG(p && E && out_tokens && n_accepted && workspace, "verify_probs: null pointer");
  FS_CHECK_ARG(K == 0 || (q && draft_tokens && u), "verify_probs: null draft inputs");
  FS_CHECK_ARG(dtype_ok(dtype), "verify_probs: dtype %d", dtype);
  FS_CHECK_ARG(K >= 0 && V > 0 && V < 0x7fffffff, "verify_probs: K %d V %lld", K, (long long)V);
  FS_CHECK_ARG(workspace_bytes >= accept_ws(1, K, V), "verify_probs: workspace too small");
  const int nch = (int)nchunks(V);
  AcceptArgs A;
  A.rs = RowSet{p, 0, ldp, K + 1, q ? q : p, 0, ldq, K};
  A.K = K;
  A.V = V;
  A.nch = nch;
  A.nchr = (int)nchunks_r(V);
  A.B = 1;
  A.draft = draft_tokens;
  A.k_eff = nullptr;
  A.temps = nullptr;
  A.u = u;
  A.E = E;
  A.ldE = V;
  A.out_tokens = out_tokens;
  A.n_acc = n_accepted;
  A.seq_len = nullptr;
  A.dbg_p = A.dbg_q = A.dbg_s = nullptr;
  carve_accept(A, workspace, 1, K, nch, A.nchr);
  hipStream_t s = fs::as_stream(stream);
  switch (dtype) {
    case FS_F32: return launch_accept<FS_F32>(A, true, s);
    case FS_BF16: return launch_accept<FS_BF16>(A, true, s);
    default: return launch_accept<FS_F16>(A, true, s);
  }
}

namespace {
// One row of the round-to-round bookkeeping of speculative.py:71-85, on the device: the row's
// n_accepted a and committed tokens res[1 .. a+1] (an acceptance's output row) advance its length by
// a + 1 and its token budget by the same; the row is done once the budget is spent or a committed
// token is its EOS. Then the next round's inputs are written exactly as the host stages them: (prev,
// last) ids, k_eff = min(k, budget - 1), the draft steps' positions (step i feeds position n-1+i while
// i < k_eff; steps below `first` are fed by the pair at pos0) and the verify window's positions
// (n-1+t for t <= k_eff). A done row, and a row that was done already, gets k_eff 0 and only -1
// positions: it reads no keys, writes no cache entry and its results are ignored.
__global__ void __launch_bounds__(256) spec_advance_kernel(const int32_t* __restrict__ res, int64_t res_ld, int32_t B,
                                                           int32_t k, int32_t first, int32_t* __restrict__ n,
                                                           int32_t* __restrict__ budget, const int32_t* __restrict__ eos,
                                                           int32_t* __restrict__ done, int64_t* __restrict__ ids,
                                                           int64_t* __restrict__ last, int32_t* __restrict__ keff,
                                                           int32_t* __restrict__ pos0, int32_t* __restrict__ posd,
                                                           int32_t* __restrict__ posv) {
  const int r = blockIdx.x * blockDim.x + threadIdx.x;
  if (r >= B) return;
  bool dn = done[r] != 0;
  int nn = n[r], bud = budget[r];
  int64_t prev = ids[2 * r], lst = ids[2 * r + 1];
  if (!dn) {
    const int32_t* row = res + (int64_t)r * res_ld;
    const int a = min(max(row[0], 0), k);
    const int e = eos[r];
    bool hit = false;
    for (int j = 0; j <= a; ++j) hit = hit || (e >= 0 && row[1 + j] == e);
    nn += a + 1;
    bud -= a + 1;
    prev = a >= 1 ? (int64_t)row[a] : lst;
    lst = row[1 + a];
    dn = hit || bud <= 0;
  }
  const int ke = dn ? 0 : min(k, max(bud - 1, 0));
  n[r] = nn;
  budget[r] = bud;
  done[r] = dn ? 1 : 0;
  ids[2 * r] = prev;
  ids[2 * r + 1] = lst;
  last[r] = lst;
  keff[r] = ke;
  pos0[2 * r] = ke > 0 ? (nn > 1 ? nn - 2 : -1) : -1;
  pos0[2 * r + 1] = ke > 0 ? nn - 1 : -1;
  for (int i = first; i < k; ++i) posd[(int64_t)(i - first) * B + r] = ke > i ? nn - 1 + i : -1;
  for (int t = 0; t <= k; ++t) posv[(int64_t)r * (k + 1) + t] = (!dn && t <= ke) ? nn - 1 + t : -1;
}
}  // namespace

extern "C" int fs_spec_advance(const int32_t* res, int64_t res_ld, int32_t B, int32_t k, int32_t first, int32_t* n,
                               int32_t* budget, const int32_t* eos, int32_t* done, int64_t* ids, int64_t* last,
                               int32_t* keff, int32_t* pos0, int32_t* posd, int32_t* posv, void* stream) {
  FS_CHECK_ARG(res && n && budget && eos && done && ids && last && keff && pos0 && posv, "spec_advance: null pointer");
  FS_CHECK_ARG(B >= 0 && k >= 0 && (first == 0 || first == 1) && res_ld >= k + 2 && (k <= first || posd),
               "spec_advance: B %d k %d first %d res_ld %lld", B, k, first, (long long)res_ld);
  if (B == 0) return 0;
  spec_advance_kernel<<<dim3((unsigned)((B + 255) / 256)), 256, 0, fs::as_stream(stream)>>>(
      res, res_ld, B, k, first, n, budget, eos, done, ids, last, keff, pos0, posd, posv);
  return fs::launch_status("spec_advance");
}
