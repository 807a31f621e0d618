// Counter-based random numbers for per-request streams (the speculative Engine's draws).
//
// The reference's Engine draws every sampled token from one generator in running-row order
// (engine.py:41, 126-133), so a request's tokens depend on which requests share its batch. Batched
// speculation keys each request's randomness instead: row b of a call has a 64-bit key (derived by
// the caller from (seed, request id, position)), and the variate at (key, slot, column j) is a pure
// function of those three numbers. A request therefore draws the same numbers whatever else is in
// the batch and whatever the round's k is; one launch fills every row of a round.
//
// Generator: Philox4x32-10 (Salmon, Moraes, Dror, Shaw, "Parallel random numbers: as easy as 1, 2,
// 3", SC'11): counter (j / 2, slot, 0, 0), key (low, high 32 bits of the row's key), ten rounds with
// the published multipliers and Weyl increments. One call gives four 32-bit words w0..w3; column 2i
// uses (w0, w1) and column 2i + 1 uses (w2, w3).
//   uniform:  u = (w_a >> 8) * 2^-24, in [0, 1) on the 24-bit grid torch.rand uses for float32.
//   Exp(1):   E = -log1p(-t) with t = (1 + (w_a >> 9) * 2^-23) * 2^-(1 + clz(w_b)), a uniform in
//             (0, 1) whose relative resolution is 2^-23 down to 2^-33 (clz of a uniform word is
//             geometric), so E is never 0 and small E (the draws' large keys w / E) keep full
//             precision.
#include <math.h>

#include "common.h"

namespace {

constexpr uint32_t PHILOX_M0 = 0xD2511F53u, PHILOX_M1 = 0xCD9E8D57u;
constexpr uint32_t PHILOX_W0 = 0x9E3779B9u, PHILOX_W1 = 0xBB67AE85u;

struct Words {
  uint32_t w[4];
};

FS_DEVICE Words philox4x32_10(uint32_t c0, uint32_t c1, uint32_t c2, uint32_t c3, uint32_t k0, uint32_t k1) {
#pragma unroll
  for (int r = 0; r < 10; ++r) {
    const uint64_t p0 = (uint64_t)PHILOX_M0 * c0;
    const uint64_t p1 = (uint64_t)PHILOX_M1 * c2;
    const uint32_t hi0 = (uint32_t)(p0 >> 32), lo0 = (uint32_t)p0;
    const uint32_t hi1 = (uint32_t)(p1 >> 32), lo1 = (uint32_t)p1;
    c0 = hi1 ^ c1 ^ k0;
    c1 = lo1;
    c2 = hi0 ^ c3 ^ k1;
    c3 = lo0;
    k0 += PHILOX_W0;
    k1 += PHILOX_W1;
  }
  return Words{{c0, c1, c2, c3}};
}

FS_DEVICE float to_uniform(uint32_t a) { return (float)(a >> 8) * 5.9604644775390625e-8f; }  // 2^-24

FS_DEVICE float to_exponential(uint32_t a, uint32_t b) {
  const int z = b ? __clz(b) : 32;
  const float mant = 1.0f + (float)(a >> 9) * 1.1920928955078125e-7f;   // [1, 2), 2^-23 steps
  const float t = ldexpf(mant, -(1 + z));                              // (0, 1)
  return -log1pf(-t);
}

constexpr int THREADS = 256;

// grid: x = column pairs / THREADS, y = row (fastest) + slot * B
__global__ void __launch_bounds__(THREADS) keyed_noise_kernel(const uint64_t* __restrict__ keys, int32_t B,
                                                              int32_t slot0, int64_t n, int32_t kind,
                                                              float* __restrict__ out, int64_t ld_row,
                                                              int64_t ld_slot) {
  const int64_t pair = (int64_t)blockIdx.x * THREADS + threadIdx.x;
  const int64_t j = 2 * pair;
  if (j >= n) return;
  const int b = blockIdx.y % B, s = blockIdx.y / B;
  const uint64_t key = keys[b];
  const Words w = philox4x32_10((uint32_t)pair, (uint32_t)(slot0 + s), 0u, 0u, (uint32_t)key, (uint32_t)(key >> 32));
  float v0, v1;
  if (kind == FS_RNG_UNIFORM) {
    v0 = to_uniform(w.w[0]);
    v1 = to_uniform(w.w[2]);
  } else {
    v0 = to_exponential(w.w[0], w.w[1]);
    v1 = to_exponential(w.w[2], w.w[3]);
  }
  float* o = out + (int64_t)s * ld_slot + (int64_t)b * ld_row + j;
  if (j + 1 < n && (reinterpret_cast<uintptr_t>(o) & 7) == 0) {
    typedef __attribute__((__vector_size__(2 * sizeof(float)))) float float2_t;
    *reinterpret_cast<float2_t*>(o) = float2_t{v0, v1};
  } else {
    o[0] = v0;
    if (j + 1 < n) o[1] = v1;
  }
}

}  // namespace

extern "C" int fs_keyed_noise(const uint64_t* keys, int32_t B, int32_t slot0, int32_t n_slots, int64_t n,
                              int32_t kind, float* out, int64_t ld_row, int64_t ld_slot, void* stream) {
  FS_CHECK_ARG(keys && out, "keyed_noise: null pointer");
  FS_CHECK_ARG(kind == FS_RNG_UNIFORM || kind == FS_RNG_EXP, "keyed_noise: kind %d", kind);
  FS_CHECK_ARG(B >= 0 && n_slots >= 0 && n >= 0 && slot0 >= 0 && (int64_t)slot0 + n_slots <= 0x7fffffff,
               "keyed_noise: B %d slots %d+%d n %lld", B, slot0, n_slots, (long long)n);
  FS_CHECK_ARG((int64_t)B * n_slots <= 65535 && (n + 1) / 2 <= (int64_t)0x7fffffff,
               "keyed_noise: at most 65535 rows x slots and 2^32 columns per call");
  FS_CHECK_ARG(B <= 1 || ld_row >= n, "keyed_noise: ld_row %lld < n %lld", (long long)ld_row, (long long)n);
  FS_CHECK_ARG(n_slots <= 1 || ld_slot >= (B - 1) * ld_row + n, "keyed_noise: slots overlap");
  if (B == 0 || n_slots == 0 || n == 0) return 0;
  const int64_t pairs = (n + 1) / 2;
  const dim3 grid((unsigned)((pairs + THREADS - 1) / THREADS), (unsigned)(B * n_slots));
  keyed_noise_kernel<<<grid, THREADS, 0, fs::as_stream(stream)>>>(keys, B, slot0, n, kind, out, ld_row, ld_slot);
  return fs::launch_status("keyed_noise");
}
