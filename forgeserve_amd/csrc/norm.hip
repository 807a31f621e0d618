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
    const float sg = E::round(gv / (1.0f + expf(-gv)));
    E::store(h, m * ldh + n, sg * uv);
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

bool dtype_ok(int32_t dt) { return dt == FS_F32 || dt == FS_BF16 || dt == FS_F16; }

}  // namespace

extern "C" int fs_add_rmsnorm(const void* x, int64_t ldx, const void* delta, int64_t ldd, void* x_out, int64_t ldxo,
                              const void* weight, void* y, int64_t ldy, int64_t M, int64_t N, float eps,
                              int32_t dtype, void* stream) {
  FS_CHECK_ARG(x && weight && y, "add_rmsnorm: null pointer");
  FS_CHECK_ARG(dtype_ok(dtype), "add_rmsnorm: dtype %d", dtype);
  FS_CHECK_ARG(M >= 0 && N > 0, "add_rmsnorm: M %lld N %lld", (long long)M, (long long)N);
  if (M == 0) return 0;
  hipStream_t s = fs::as_stream(stream);
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
  if (dtype == FS_F32)
    embedding_kernel<float><<<dim3((unsigned)M), 256, 0, s>>>(ids, (const float*)weight, d_model, vocab,
                                                             (float*)out, ldo);
  else
    embedding_kernel<uint16_t><<<dim3((unsigned)M), 256, 0, s>>>(ids, (const uint16_t*)weight, d_model, vocab,
                                                                (uint16_t*)out, ldo);
  return fs::launch_status("embedding");
}
