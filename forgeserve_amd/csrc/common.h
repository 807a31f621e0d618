// Shared device/host helpers for the forgeserve_amd gfx950 kernels.
//
// Numeric conventions (they decide bit-level parity with the PyTorch CPU reference):
//   * bf16 <-> f32 conversions are round-to-nearest-even, as c10::BFloat16 does.
//   * Every elementwise op that the reference performs in the tensor dtype is rounded to that dtype
//     after the op (torch's CPU kernels compute bf16 ops in f32 and round each result).
//   * The library is compiled with -ffp-contract=off: a*b - c*d stays two roundings, as in torch.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include "../../include/forgeserve_amd.h"

#define FS_DEVICE __device__ __forceinline__

// Offset of key dim d within a key (fs_kv_layout: plain k_dim stride, or 8-dim groups k_group apart).
FS_DEVICE int64_t key_dim_off(const fs_kv_layout& kv, int d) {
  return kv.k_group ? (int64_t)(d >> 3) * kv.k_group + (d & 7) : (int64_t)d * kv.k_dim;
}
// Distance between a key's 8-dim groups when its dims are contiguous within a group (k_dim == 1).
FS_DEVICE int64_t key_group_stride(const fs_kv_layout& kv) { return kv.k_group ? kv.k_group : 8; }

typedef __attribute__((__vector_size__(8 * sizeof(__bf16)))) __bf16 bf16x8_t;
typedef __attribute__((__vector_size__(4 * sizeof(short)))) short short4_t;
typedef __attribute__((__vector_size__(4 * sizeof(float)))) float float4_t;

// ------------------------------------------------------------------------------------------------
// scalar conversions
// ------------------------------------------------------------------------------------------------
FS_DEVICE float bf16_to_f32(uint16_t h) { return __uint_as_float(((uint32_t)h) << 16); }

FS_DEVICE uint16_t f32_to_bf16(float f) {
  uint32_t u = __float_as_uint(f);
  if ((u & 0x7fffffffu) > 0x7f800000u) return (uint16_t)((u >> 16) | 0x40u);  // quiet NaN
  u += 0x7fffu + ((u >> 16) & 1u);
  return (uint16_t)(u >> 16);
}

FS_DEVICE float f16_to_f32(uint16_t h) { return (float)__builtin_bit_cast(_Float16, h); }
FS_DEVICE uint16_t f32_to_f16(float f) { return __builtin_bit_cast(uint16_t, (_Float16)f); }  // RNE

// Storage-type traits: load/store one element as f32, and round an f32 to what the dtype can hold.
template <int DT> struct Elem;
template <> struct Elem<FS_F32> {
  typedef float T;
  static FS_DEVICE float load(const T* p, int64_t i) { return p[i]; }
  static FS_DEVICE void store(T* p, int64_t i, float v) { p[i] = v; }
  static FS_DEVICE float round(float v) { return v; }
  static FS_DEVICE float to_f32(T v) { return v; }
};
template <> struct Elem<FS_BF16> {
  typedef uint16_t T;
  static FS_DEVICE float load(const T* p, int64_t i) { return bf16_to_f32(p[i]); }
  static FS_DEVICE void store(T* p, int64_t i, float v) { p[i] = f32_to_bf16(v); }
  static FS_DEVICE float round(float v) { return bf16_to_f32(f32_to_bf16(v)); }
  static FS_DEVICE float to_f32(T v) { return bf16_to_f32(v); }
  static FS_DEVICE T store_bits(float v) { return f32_to_bf16(v); }
};
template <> struct Elem<FS_F16> {
  typedef uint16_t T;
  static FS_DEVICE float load(const T* p, int64_t i) { return f16_to_f32(p[i]); }
  static FS_DEVICE void store(T* p, int64_t i, float v) { p[i] = f32_to_f16(v); }
  static FS_DEVICE float round(float v) { return f16_to_f32(f32_to_f16(v)); }
  static FS_DEVICE float to_f32(T v) { return f16_to_f32(v); }
  static FS_DEVICE T store_bits(float v) { return f32_to_f16(v); }
};

// ------------------------------------------------------------------------------------------------
// wavefront (64-lane) reductions
// ------------------------------------------------------------------------------------------------
// silu(g) * u as a 16-bit SwiGLU computes it (model.py:93): silu rounded to the dtype, then the
// product, which the caller rounds when it stores it; g and u are dtype values. Every kernel that
// forms this product calls this one function, so their results agree bit for bit.
template <int DT>
FS_DEVICE float silu_times(float g, float u) {
  return Elem<DT>::round(g / (1.0f + expf(-g))) * u;
}

FS_DEVICE float wave_max(float v) {
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) v = fmaxf(v, __shfl_xor(v, o, 64));
  return v;
}
FS_DEVICE float wave_sum(float v) {
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) v += __shfl_xor(v, o, 64);
  return v;
}

// (value, index) argmax where the larger value wins and equal values keep the lower index: the
// first-occurrence rule of torch.argmax.
FS_DEVICE void argmax_merge(float& v, int& i, float ov, int oi) {
  if (ov > v || (ov == v && oi < i)) { v = ov; i = oi; }
}
FS_DEVICE void wave_argmax(float& v, int& i) {
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) {
    float ov = __shfl_xor(v, o, 64);
    int oi = __shfl_xor(i, o, 64);
    argmax_merge(v, i, ov, oi);
  }
}

// Softmax statistics of a run of logits x at temperature T: m = max of y = x/T, s = Σ exp(y - m),
// and the first argmax (av, ai) of x. Runs are merged in a fixed order wherever they are combined.
struct SoftmaxStat {
  float m, s, av;
  int ai;
};

// Accesses that cross workgroups within one launch, whatever XCD each runs on: agent-scope relaxed
// atomic stores and loads (global_store/global_load with the device-coherence bit: no L2 of one XCD
// holds a value another XCD cannot see).
FS_DEVICE void st_ag(float* p, float v) { __hip_atomic_store(p, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT); }
FS_DEVICE void st_ag(int* p, int v) { __hip_atomic_store(p, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT); }
FS_DEVICE void st_ag(unsigned* p, unsigned v) {
  __hip_atomic_store(p, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
FS_DEVICE float ld_ag(const float* p) {
  return __hip_atomic_load(const_cast<float*>(p), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
FS_DEVICE int ld_ag(const int* p) {
  return __hip_atomic_load(const_cast<int*>(p), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
FS_DEVICE unsigned ld_ag(const unsigned* p) {
  return __hip_atomic_load(const_cast<unsigned*>(p), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
// This wave's stores have completed (vmcnt(0)), with no memory access moved across by the compiler.
FS_DEVICE void stores_done() {
  __atomic_signal_fence(__ATOMIC_SEQ_CST);
  __builtin_amdgcn_s_waitcnt(0x0F70);
  __atomic_signal_fence(__ATOMIC_SEQ_CST);
}
// Count one more completed item; true for the item that completes the count (the counter wraps to 0).
FS_DEVICE bool count_in(unsigned* c, unsigned total) {
  const unsigned old = __builtin_amdgcn_atomic_inc32(c, total - 1u, __ATOMIC_RELAXED, "agent");
  __atomic_signal_fence(__ATOMIC_SEQ_CST);
  return old == total - 1u;
}

// ------------------------------------------------------------------------------------------------
// host side: error reporting shared by every entry point
// ------------------------------------------------------------------------------------------------
namespace fs {
void set_error(const char* fmt, ...);
int arg_error(const char* fmt, ...);           // sets the message, returns FS_ERR_ARG
int launch_status(const char* what);           // hipGetLastError after a launch -> 0 or >0
inline hipStream_t as_stream(void* s) { return reinterpret_cast<hipStream_t>(s); }
}  // namespace fs

#define FS_CHECK_ARG(cond, ...) \
  do {                           \
    if (!(cond)) return fs::arg_error(__VA_ARGS__); \
  } while (0)
