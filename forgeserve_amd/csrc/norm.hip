// Row-wise ops of the decoder block: residual add + RMSNorm, SwiGLU gate, embedding lookup.
//
// Reference: model.py:29-31 (RMSNorm), model.py:93 (silu(gate) * up), model.py:104-106 (pre-norm
// residual block), model.py:134-135 (embedding). Reductions run in a fixed order that depends only
// on the row length, so a row's result does not depend on how many rows are in the batch.
#include "common.h"

namespace {

constexpr int NORM_THREADS = 256;

template <int DT>
__global__ void __launch_bounds__(NORM_THREADS) add_rmsnorm_kernel(
    const typename Elem<DT>::T* __restrict__ x, int64_t ldx, const typename Elem<DT>::T* __restrict__ delta,
    int64_t ldd, typename Elem<DT>::T* __restrict__ x_out, int64_t ldxo, const typename Elem<DT>::T* __restrict__ w,
    typename Elem<DT>::T* __restrict__ y, int64_t ldy, int64_t N, float eps) {
  typedef Elem<DT> E;
  __shared__ float red[NORM_THREADS / 64];
  const int64_t m = blockIdx.x;
  const auto* xr = x + m * ldx;
  const auto* dr = delta ? delta + m * ldd : nullptr;
  auto* xo = x_out ? x_out + m * ldxo : nullptr;
  float sq = 0.f;
  for (int64_t i = threadIdx.x; i < N; i += NORM_THREADS) {
    float v = E::load(xr, i);
    if (dr) v = E::round(v + E::load(dr, i));
    if (xo) E::store(xo, i, v);
    sq += v * v;
  }
  sq = wave_sum(sq);
  if ((threadIdx.x & 63) == 0) red[threadIdx.x >> 6] = sq;
  __syncthreads();
  float tot = 0.f;
#pragma unroll
  for (int i = 0; i < NORM_THREADS / 64; ++i) tot += red[i];
  const float r = 1.0f / sqrtf(tot / (float)N + eps);
  auto* yr = y + m * ldy;
  for (int64_t i = threadIdx.x; i < N; i += NORM_THREADS) {
    float v = E::load(xr, i);
    if (dr) v = E::round(v + E::load(dr, i));
    const float n = E::round(v * r);
    E::store(yr, i, n * E::load(w, i));
  }
}

// 16-bit rows, 8 elements per 16-byte access, the whole row in registers (N <= NORM_VEC_MAX): one
// pass over memory. The arithmetic and its order are add_rmsnorm_kernel's, except the sum of squares:
// each thread adds its 8-element groups in order, then the lanes and waves are added as there.
typedef __attribute__((__vector_size__(4 * sizeof(uint32_t)))) uint32_t u32x4_t;
constexpr int NORM_VEC_GROUPS = 4;                                   // 8-element groups per thread
constexpr int64_t NORM_VEC_MAX = NORM_THREADS * 8 * NORM_VEC_GROUPS;   // 8192 elements

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

template <int DT>
__global__ void __launch_bounds__(NORM_THREADS) add_rmsnorm_vec_kernel(
    const uint16_t* __restrict__ x, int64_t ldx, const uint16_t* __restrict__ delta, int64_t ldd,
    uint16_t* __restrict__ x_out, int64_t ldxo, const uint16_t* __restrict__ w, uint16_t* __restrict__ y, int64_t ldy,
    int64_t N, float eps) {
  __shared__ float red[NORM_THREADS / 64];
  const int64_t m = blockIdx.x;
  const int ng = (int)(N / 8);   // 8-element groups in the row; thread t takes t, t + NORM_THREADS, ...
  float v[NORM_VEC_GROUPS][8];
  u32x4_t xr[NORM_VEC_GROUPS], dr[NORM_VEC_GROUPS], wr[NORM_VEC_GROUPS];
#pragma unroll
  for (int u = 0; u < NORM_VEC_GROUPS; ++u) {   // every load in flight before any arithmetic
    const int gi = threadIdx.x + NORM_THREADS * u;
    if (gi < ng) {
      xr[u] = *reinterpret_cast<const u32x4_t*>(x + m * ldx + 8 * gi);
      if (delta) dr[u] = *reinterpret_cast<const u32x4_t*>(delta + m * ldd + 8 * gi);
      wr[u] = *reinterpret_cast<const u32x4_t*>(w + 8 * gi);
    }
  }
  float sq = 0.f;
#pragma unroll
  for (int u = 0; u < NORM_VEC_GROUPS; ++u) {
    const int gi = threadIdx.x + NORM_THREADS * u;
    if (gi >= ng) continue;
    unpack8<DT>(xr[u], v[u]);
    if (delta) {
      float d[8];
      unpack8<DT>(dr[u], d);
#pragma unroll
      for (int j = 0; j < 8; ++j) v[u][j] = Elem<DT>::round(v[u][j] + d[j]);
      if (x_out) *reinterpret_cast<u32x4_t*>(x_out + m * ldxo + 8 * gi) = pack8<DT>(v[u]);
    }
#pragma unroll
    for (int j = 0; j < 8; ++j) sq += v[u][j] * v[u][j];
  }
  sq = wave_sum(sq);
  if ((threadIdx.x & 63) == 0) red[threadIdx.x >> 6] = sq;
  __syncthreads();
  float tot = 0.f;
#pragma unroll
  for (int i = 0; i < NORM_THREADS / 64; ++i) tot += red[i];
  const float r = 1.0f / sqrtf(tot / (float)N + eps);
#pragma unroll
  for (int u = 0; u < NORM_VEC_GROUPS; ++u) {
    const int gi = threadIdx.x + NORM_THREADS * u;
    if (gi >= ng) continue;
    float wv[8], o[8];
    unpack8<DT>(wr[u], wv);
#pragma unroll
    for (int j = 0; j < 8; ++j) o[j] = Elem<DT>::round(v[u][j] * r) * wv[j];
    *reinterpret_cast<u32x4_t*>(y + m * ldy + 8 * gi) = pack8<DT>(o);
  }
}

// The same kernel for x = a split-K GEMM's output: x[m] = round(sum over s of parts[s][m], in split
// order), then the residual: x_out = round(x + residual), y = rmsnorm(x_out) * w. This is the GEMM's
// reduction (gemm_splitk_reduce_kernel) followed by add_rmsnorm_vec_kernel on its output, in one pass.
// SPLITS > 0: that many partials, all loaded before the first add; 0: `splits` of them, one at a time.
// G > 0: the row is exactly G groups per thread (N = NORM_THREADS * 8 * G): every group's loads are
// issued before the first is used (with a bounds branch around each group, the compiler waits for a
// group's loads before issuing the next group's); G == 0: any N up to NORM_VEC_MAX, group by group.
template <int DT, int SPLITS, int G>
__global__ void __launch_bounds__(NORM_THREADS) splitk_add_rmsnorm_kernel(
    const float* __restrict__ parts, int splits, int64_t part_stride, const uint16_t* __restrict__ residual,
    int64_t ldr, uint16_t* __restrict__ x_out, int64_t ldxo, const uint16_t* __restrict__ w, uint16_t* __restrict__ y,
    int64_t ldy, int64_t N, float eps) {
  __shared__ float red[NORM_THREADS / 64];
  const int64_t m = blockIdx.x;
  const int ng = (int)(N / 8);
  float v[NORM_VEC_GROUPS][8];
  float sq = 0.f;
  if constexpr (G > 0 && SPLITS > 0) {
    static_assert(G <= NORM_VEC_GROUPS, "at most NORM_VEC_GROUPS groups per thread");
    float4_t q0[G][SPLITS], q1[G][SPLITS];
    u32x4_t rr[G];
#pragma unroll
    for (int u = 0; u < G; ++u) {
      const int gi = threadIdx.x + NORM_THREADS * u;
      const float* p0 = parts + m * N + 8 * gi;
#pragma unroll
      for (int sp = 0; sp < SPLITS; ++sp) {
        q0[u][sp] = *reinterpret_cast<const float4_t*>(p0 + sp * part_stride);
        q1[u][sp] = *reinterpret_cast<const float4_t*>(p0 + sp * part_stride + 4);
      }
      rr[u] = *reinterpret_cast<const u32x4_t*>(residual + m * ldr + 8 * gi);
    }
    __builtin_amdgcn_sched_barrier(0);
#pragma unroll
    for (int u = 0; u < G; ++u) {
      const int gi = threadIdx.x + NORM_THREADS * u;
      float4_t a0 = q0[u][0], a1 = q1[u][0];
#pragma unroll
      for (int sp = 1; sp < SPLITS; ++sp)
#pragma unroll
        for (int j = 0; j < 4; ++j) {
          a0[j] += q0[u][sp][j];
          a1[j] += q1[u][sp][j];
        }
      float d[8];
      unpack8<DT>(rr[u], d);
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        v[u][j] = Elem<DT>::round(Elem<DT>::round(a0[j]) + d[j]);
        v[u][j + 4] = Elem<DT>::round(Elem<DT>::round(a1[j]) + d[j + 4]);
      }
      *reinterpret_cast<u32x4_t*>(x_out + m * ldxo + 8 * gi) = pack8<DT>(v[u]);
#pragma unroll
      for (int j = 0; j < 8; ++j) sq += v[u][j] * v[u][j];
    }
  } else {
#pragma unroll
  for (int u = 0; u < NORM_VEC_GROUPS; ++u) {
    const int gi = threadIdx.x + NORM_THREADS * u;
    if (gi >= ng) continue;
    const float* p0 = parts + m * N + 8 * gi;
    float4_t a0, a1;
    if (SPLITS > 0) {
      float4_t q0[SPLITS > 0 ? SPLITS : 1], q1[SPLITS > 0 ? SPLITS : 1];
#pragma unroll
      for (int sp = 0; sp < SPLITS; ++sp) {
        q0[sp] = *reinterpret_cast<const float4_t*>(p0 + sp * part_stride);
        q1[sp] = *reinterpret_cast<const float4_t*>(p0 + sp * part_stride + 4);
      }
      a0 = q0[0];
      a1 = q1[0];
#pragma unroll
      for (int sp = 1; sp < SPLITS; ++sp)
#pragma unroll
        for (int j = 0; j < 4; ++j) {
          a0[j] += q0[sp][j];
          a1[j] += q1[sp][j];
        }
    } else {
      a0 = *reinterpret_cast<const float4_t*>(p0);
      a1 = *reinterpret_cast<const float4_t*>(p0 + 4);
      for (int sp = 1; sp < splits; ++sp) {
        const float4_t b0 = *reinterpret_cast<const float4_t*>(p0 + sp * part_stride);
        const float4_t b1 = *reinterpret_cast<const float4_t*>(p0 + sp * part_stride + 4);
#pragma unroll
        for (int j = 0; j < 4; ++j) {
          a0[j] += b0[j];
          a1[j] += b1[j];
        }
      }
    }
    float d[8];
    unpack8<DT>(*reinterpret_cast<const u32x4_t*>(residual + m * ldr + 8 * gi), d);
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      v[u][j] = Elem<DT>::round(Elem<DT>::round(a0[j]) + d[j]);
      v[u][j + 4] = Elem<DT>::round(Elem<DT>::round(a1[j]) + d[j + 4]);
    }
    *reinterpret_cast<u32x4_t*>(x_out + m * ldxo + 8 * gi) = pack8<DT>(v[u]);
#pragma unroll
    for (int j = 0; j < 8; ++j) sq += v[u][j] * v[u][j];
  }
  }
  sq = wave_sum(sq);
  if ((threadIdx.x & 63) == 0) red[threadIdx.x >> 6] = sq;
  __syncthreads();
  float tot = 0.f;
#pragma unroll
  for (int i = 0; i < NORM_THREADS / 64; ++i) tot += red[i];
  const float r = 1.0f / sqrtf(tot / (float)N + eps);
#pragma unroll
  for (int u = 0; u < (G > 0 && SPLITS > 0 ? G : NORM_VEC_GROUPS); ++u) {
    const int gi = threadIdx.x + NORM_THREADS * u;
    if (gi >= ng) continue;
    float wv[8], o[8];
    unpack8<DT>(*reinterpret_cast<const u32x4_t*>(w + 8 * gi), wv);
#pragma unroll
    for (int j = 0; j < 8; ++j) o[j] = Elem<DT>::round(v[u][j] * r) * wv[j];
    *reinterpret_cast<u32x4_t*>(y + m * ldy + 8 * gi) = pack8<DT>(o);
  }
}

// silu(gate) * up on 16-bit rows, 8 columns per thread and 16-byte accesses (F % 8 == 0); the same
// per-element arithmetic as silu_mul_kernel.
template <int DT>
__global__ void __launch_bounds__(256) silu_mul_vec_kernel(const uint16_t* __restrict__ gu, int64_t ldgu,
                                                           uint16_t* __restrict__ h, int64_t ldh, int64_t M,
                                                           int64_t F) {
  const int64_t groups = F / 8, total = M * groups;
  for (int64_t i = blockIdx.x * (int64_t)blockDim.x + threadIdx.x; i < total; i += (int64_t)gridDim.x * blockDim.x) {
    const int64_t m = i / groups, c = 8 * (i - m * groups);
    float g[8], u[8], o[8];
    unpack8<DT>(*reinterpret_cast<const u32x4_t*>(gu + m * ldgu + c), g);
    unpack8<DT>(*reinterpret_cast<const u32x4_t*>(gu + m * ldgu + F + c), u);
#pragma unroll
    for (int j = 0; j < 8; ++j) o[j] = silu_times<DT>(g[j], u[j]);
    *reinterpret_cast<u32x4_t*>(h + m * ldh + c) = pack8<DT>(o);
  }
}

template <int DT>
__global__ void __launch_bounds__(256) silu_mul_kernel(const typename Elem<DT>::T* __restrict__ gu, int64_t ldgu,
                                                       typename Elem<DT>::T* __restrict__ h, int64_t ldh, int64_t M,
                                                       int64_t F) {
  typedef Elem<DT> E;
  const int64_t total = M * F;
  for (int64_t i = blockIdx.x * (int64_t)blockDim.x + threadIdx.x; i < total; i += (int64_t)gridDim.x * blockDim.x) {
    const int64_t m = i / F, n = i - m * F;
    const float gv = E::load(gu, m * ldgu + n);
    const float uv = E::load(gu, m * ldgu + F + n);
    E::store(h, m * ldh + n, silu_times<DT>(gv, uv));
  }
}

template <typename T>
__global__ void __launch_bounds__(256) embedding_kernel(const int64_t* __restrict__ ids, const T* __restrict__ w,
                                                        int64_t d, int64_t vocab, T* __restrict__ out, int64_t ldo) {
  const int64_t m = blockIdx.x;
  const int64_t id = ids[m];
  T* o = out + m * ldo;
  if (id < 0 || id >= vocab) {
    for (int64_t i = threadIdx.x; i < d; i += blockDim.x) o[i] = T(0);
    return;
  }
  const T* r = w + id * d;
  for (int64_t i = threadIdx.x; i < d; i += blockDim.x) o[i] = r[i];
}

// The same with 16-byte copies (rows of a multiple of 16 bytes, 16-byte aligned).
__global__ void __launch_bounds__(256) embedding_vec_kernel(const int64_t* __restrict__ ids,
                                                            const u32x4_t* __restrict__ w, int64_t d16,
                                                            int64_t vocab, u32x4_t* __restrict__ out,
                                                            int64_t ldo16) {
  const int64_t m = blockIdx.x;
  const int64_t id = ids[m];
  u32x4_t* o = out + m * ldo16;
  if (id < 0 || id >= vocab) {
    for (int64_t i = threadIdx.x; i < d16; i += blockDim.x) o[i] = u32x4_t{0u, 0u, 0u, 0u};
    return;
  }
  const u32x4_t* r = w + id * d16;
  for (int64_t i = threadIdx.x; i < d16; i += blockDim.x) o[i] = r[i];
}

bool dtype_ok(int32_t dt) { return dt == FS_F32 || dt == FS_BF16 || dt == FS_F16; }

}  // namespace

extern "C" int fs_splitk_add_rmsnorm(const float* parts, int32_t splits, const void* residual, int64_t ldr,
                                     void* x_out, int64_t ldxo, const void* weight, void* y, int64_t ldy, int64_t M,
                                     int64_t N, float eps, int32_t dtype, void* stream) {
  FS_CHECK_ARG(parts && residual && x_out && weight && y, "splitk_add_rmsnorm: null pointer");
  FS_CHECK_ARG(dtype == FS_BF16 || dtype == FS_F16, "splitk_add_rmsnorm: dtype %d (16-bit only)", dtype);
  FS_CHECK_ARG(splits >= 1 && M >= 0 && N > 0 && N % 8 == 0 && N <= NORM_VEC_MAX,
               "splitk_add_rmsnorm: splits %d M %lld N %lld", splits, (long long)M, (long long)N);
  auto al16 = [](const void* p) { return (reinterpret_cast<uintptr_t>(p) & 15) == 0; };
  FS_CHECK_ARG(al16(parts) && al16(residual) && al16(x_out) && al16(weight) && al16(y) && ldr % 8 == 0 &&
                   ldxo % 8 == 0 && ldy % 8 == 0,
               "splitk_add_rmsnorm: 16-byte aligned rows");
  if (M == 0) return 0;
  hipStream_t s = fs::as_stream(stream);
  // Short batches (latency-bound: a decode step's rows) take whole groups per thread with every load
  // issued up front, at most 8 partial groups in registers per thread; long ones (bandwidth-bound,
  // where issuing every load at once measured slower: 448 rows 9.4 -> 10.2 us) go group by group. The
  // two forms do the same arithmetic in the same order, so a row's bits do not depend on M.
  const int64_t gpt = N % (NORM_THREADS * 8) == 0 ? N / (NORM_THREADS * 8) : 0;
  const int g = M <= 128 && (gpt == 1 || gpt == 2 || gpt == 4) && gpt * splits <= 8 ? (int)gpt : 0;
#define FS_LAUNCH_PARTS(DT, S, G)                                                                               \
  splitk_add_rmsnorm_kernel<DT, S, G><<<dim3((unsigned)M), NORM_THREADS, 0, s>>>(                            \
      parts, splits, M * N, (const uint16_t*)residual, ldr, (uint16_t*)x_out, ldxo, (const uint16_t*)weight,      \
      (uint16_t*)y, ldy, N, eps)
#define FS_LAUNCH_G(DT, S)                                                                                      \
  if (g == 1) FS_LAUNCH_PARTS(DT, S, 1);                                                                      \
  else if (g == 2 && (S) <= 4) FS_LAUNCH_PARTS(DT, S, (S) <= 4 ? 2 : 0);                                     \
  else if (g == 4 && (S) <= 2) FS_LAUNCH_PARTS(DT, S, (S) <= 2 ? 4 : 0);                                     \
  else FS_LAUNCH_PARTS(DT, S, 0);
#define FS_LAUNCH_DT(DT)                                                                                        \
  switch (splits) {                                                                                           \
    case 2: FS_LAUNCH_G(DT, 2); break;                                                                        \
    case 4: FS_LAUNCH_G(DT, 4); break;                                                                        \
    case 8: FS_LAUNCH_G(DT, 8); break;                                                                        \
    default: FS_LAUNCH_PARTS(DT, 0, 0); break;                                                                \
  }
  if (dtype == FS_BF16) FS_LAUNCH_DT(FS_BF16)
  else FS_LAUNCH_DT(FS_F16)
#undef FS_LAUNCH_DT
#undef FS_LAUNCH_G
#undef FS_LAUNCH_PARTS
  return fs::launch_status("splitk_add_rmsnorm");
}

extern "C" int fs_add_rmsnorm(const void* x, int64_t ldx, const void* delta, int64_t ldd, void* x_out, int64_t ldxo,
                              const void* weight, void* y, int64_t ldy, int64_t M, int64_t N, float eps,
                              int32_t dtype, void* stream) {
  FS_CHECK_ARG(x && weight && y, "add_rmsnorm: null pointer");
  FS_CHECK_ARG(dtype_ok(dtype), "add_rmsnorm: dtype %d", dtype);
  FS_CHECK_ARG(M >= 0 && N > 0, "add_rmsnorm: M %lld N %lld", (long long)M, (long long)N);
  if (M == 0) return 0;
  hipStream_t s = fs::as_stream(stream);
  auto al16 = [](const void* p) { return (reinterpret_cast<uintptr_t>(p) & 15) == 0; };
  if (dtype != FS_F32 && N % 8 == 0 && N <= NORM_VEC_MAX && ldx % 8 == 0 && (!delta || ldd % 8 == 0) &&
      (!x_out || ldxo % 8 == 0) && ldy % 8 == 0 && al16(x) && (!delta || al16(delta)) && (!x_out || al16(x_out)) &&
      al16(weight) && al16(y)) {
#define FS_LAUNCH_VEC(DT)                                                                                      \
  add_rmsnorm_vec_kernel<DT><<<dim3((unsigned)M), NORM_THREADS, 0, s>>>(                                    \
      (const uint16_t*)x, ldx, (const uint16_t*)delta, ldd, (uint16_t*)x_out, ldxo, (const uint16_t*)weight,      \
      (uint16_t*)y, ldy, N, eps)
    if (dtype == FS_BF16) FS_LAUNCH_VEC(FS_BF16);
    else FS_LAUNCH_VEC(FS_F16);
#undef FS_LAUNCH_VEC
    return fs::launch_status("add_rmsnorm");
  }
#define FS_LAUNCH(DT)                                                                                          \
  add_rmsnorm_kernel<DT><<<dim3((unsigned)M), NORM_THREADS, 0, s>>>(                                        \
      (const typename Elem<DT>::T*)x, ldx, (const typename Elem<DT>::T*)delta, ldd, (typename Elem<DT>::T*)x_out, \
      ldxo, (const typename Elem<DT>::T*)weight, (typename Elem<DT>::T*)y, ldy, N, eps)
  switch (dtype) {
    case FS_F32: FS_LAUNCH(FS_F32); break;
    case FS_BF16: FS_LAUNCH(FS_BF16); break;
    default: FS_LAUNCH(FS_F16); break;
  }
#undef FS_LAUNCH
  return fs::launch_status("add_rmsnorm");
}

extern "C" int fs_silu_mul(const void* gu, int64_t ldgu, void* h, int64_t ldh, int64_t M, int64_t F, int32_t dtype,
                           void* stream) {
  FS_CHECK_ARG(gu && h, "silu_mul: null pointer");
  FS_CHECK_ARG(dtype_ok(dtype), "silu_mul: dtype %d", dtype);
  FS_CHECK_ARG(M >= 0 && F > 0 && ldgu >= 2 * F && ldh >= F, "silu_mul: shapes");
  if (M == 0) return 0;
  hipStream_t s = fs::as_stream(stream);
  if (dtype != FS_F32 && F % 8 == 0 && ldgu % 8 == 0 && ldh % 8 == 0 && (reinterpret_cast<uintptr_t>(gu) & 15) == 0 &&
      (reinterpret_cast<uintptr_t>(h) & 15) == 0) {
    int64_t vblocks = (M * (F / 8) + 255) / 256;
    if (vblocks > 16384) vblocks = 16384;
    if (dtype == FS_BF16)
      silu_mul_vec_kernel<FS_BF16><<<dim3((unsigned)vblocks), 256, 0, s>>>((const uint16_t*)gu, ldgu, (uint16_t*)h, ldh,
                                                                           M, F);
    else
      silu_mul_vec_kernel<FS_F16><<<dim3((unsigned)vblocks), 256, 0, s>>>((const uint16_t*)gu, ldgu, (uint16_t*)h, ldh,
                                                                          M, F);
    return fs::launch_status("silu_mul");
  }
  int64_t blocks = (M * F + 255) / 256;
  if (blocks > 16384) blocks = 16384;
#define FS_LAUNCH(DT)                                                                                         \
  silu_mul_kernel<DT><<<dim3((unsigned)blocks), 256, 0, s>>>((const typename Elem<DT>::T*)gu, ldgu,        \
                                                             (typename Elem<DT>::T*)h, ldh, M, F)
  switch (dtype) {
    case FS_F32: FS_LAUNCH(FS_F32); break;
    case FS_BF16: FS_LAUNCH(FS_BF16); break;
    default: FS_LAUNCH(FS_F16); break;
  }
#undef FS_LAUNCH
  return fs::launch_status("silu_mul");
}

extern "C" int fs_embedding(const int64_t* ids, int64_t M, const void* weight, int64_t d_model, int64_t vocab,
                            void* out, int64_t ldo, int32_t dtype, void* stream) {
  FS_CHECK_ARG(ids && weight && out, "embedding: null pointer");
  FS_CHECK_ARG(dtype_ok(dtype), "embedding: dtype %d", dtype);
  FS_CHECK_ARG(M >= 0 && d_model > 0 && vocab > 0 && ldo >= d_model, "embedding: shapes");
  if (M == 0) return 0;
  hipStream_t s = fs::as_stream(stream);
  const int64_t es = dtype == FS_F32 ? 4 : 2;   // bytes per element
  if ((d_model * es) % 16 == 0 && (ldo * es) % 16 == 0 &&
      ((reinterpret_cast<uintptr_t>(weight) | reinterpret_cast<uintptr_t>(out)) & 15) == 0) {
    embedding_vec_kernel<<<dim3((unsigned)M), 256, 0, s>>>(ids, (const u32x4_t*)weight, d_model * es / 16, vocab,
                                                          (u32x4_t*)out, ldo * es / 16);
    return fs::launch_status("embedding");
  }
  if (dtype == FS_F32)
    embedding_kernel<float><<<dim3((unsigned)M), 256, 0, s>>>(ids, (const float*)weight, d_model, vocab,
                                                             (float*)out, ldo);
  else
    embedding_kernel<uint16_t><<<dim3((unsigned)M), 256, 0, s>>>(ids, (const uint16_t*)weight, d_model, vocab,
                                                                (uint16_t*)out, ldo);
  return fs::launch_status("embedding");
}
