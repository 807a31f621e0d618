// Dense projections: C[M,N] = A[M,K] . B[N,K]^T (+ R), the nn.Linear of model.py:57-60, 88-90, 119
// (tied head) with the residual add of model.py:105-106 fused into the epilogue.
//
// bf16 path: v_mfma_f32_16x16x32_bf16 tiles, LDS double buffering, f32 accumulation, one rounding.
// Every output element accumulates its K products in increasing k, 32 at a time, in one MFMA
// accumulator, whatever the tile shape or M: a row's result does not depend on the batch it is in
// (the draft step, the verify pass and prefill give identical rows for identical inputs).
// f32 (and unaligned bf16) path: LDS-tiled VALU kernel, one fmaf chain per output in increasing k.
#include "common.h"

namespace {

// ------------------------------------------------------------------------------------------------
// bf16 MFMA kernel
// ------------------------------------------------------------------------------------------------
constexpr int BK = 64;
constexpr int LDS_PITCH = BK + 8;  // bf16 elements per LDS row (16 B pad against bank conflicts)

template <int BM, int BN>
__global__ void __launch_bounds__(256) gemm_bf16_kernel(const uint16_t* __restrict__ A, int64_t lda,
                                                        const uint16_t* __restrict__ B, int64_t ldb,
                                                        uint16_t* __restrict__ C, int64_t ldc,
                                                        const uint16_t* __restrict__ R, int64_t ldr, int64_t M,
                                                        int64_t N, int64_t K, int tiles_n) {
  constexpr int WM = BM / 2, WN = BN / 2;           // 2x2 waves
  constexpr int TM = WM / 16, TN = WN / 16;         // MFMA tiles per wave
  constexpr int A_CHUNKS = BM * BK / 8 / 256;       // 16-byte chunks per thread per stage
  constexpr int B_CHUNKS = BN * BK / 8 / 256;
  __shared__ __attribute__((aligned(16))) uint16_t As[2][BM * LDS_PITCH];
  __shared__ __attribute__((aligned(16))) uint16_t Bs[2][BN * LDS_PITCH];

  const int tid = threadIdx.x;
  const int lane = tid & 63, wave = tid >> 6;
  const int l16 = lane & 15, g = lane >> 4;
  const int wm = wave >> 1, wn = wave & 1;
  const int tile = blockIdx.x;
  const int64_t m0 = (int64_t)(tile / tiles_n) * BM;
  const int64_t n0 = (int64_t)(tile % tiles_n) * BN;

  typedef __attribute__((__vector_size__(4 * sizeof(uint32_t)))) uint32_t u32x4;
  u32x4 ra[A_CHUNKS], rb[B_CHUNKS];

  auto gload = [&](int64_t k0) {
#pragma unroll
    for (int i = 0; i < A_CHUNKS; ++i) {
      const int c = tid + 256 * i;
      const int row = c / (BK / 8), kc = (c % (BK / 8)) * 8;
      int64_t gr = m0 + row;
      gr = gr < M ? gr : M - 1;
      const int64_t gk = k0 + kc;
      if (gk < K)
        ra[i] = *reinterpret_cast<const u32x4*>(A + gr * lda + gk);
      else
        ra[i] = u32x4{0, 0, 0, 0};
    }
#pragma unroll
    for (int i = 0; i < B_CHUNKS; ++i) {
      const int c = tid + 256 * i;
      const int row = c / (BK / 8), kc = (c % (BK / 8)) * 8;
      int64_t gr = n0 + row;
      gr = gr < N ? gr : N - 1;
      const int64_t gk = k0 + kc;
      if (gk < K)
        rb[i] = *reinterpret_cast<const u32x4*>(B + gr * ldb + gk);
      else
        rb[i] = u32x4{0, 0, 0, 0};
    }
  };
  auto sstore = [&](int buf) {
#pragma unroll
    for (int i = 0; i < A_CHUNKS; ++i) {
      const int c = tid + 256 * i;
      const int row = c / (BK / 8), kc = (c % (BK / 8)) * 8;
      *reinterpret_cast<u32x4*>(&As[buf][row * LDS_PITCH + kc]) = ra[i];
    }
#pragma unroll
    for (int i = 0; i < B_CHUNKS; ++i) {
      const int c = tid + 256 * i;
      const int row = c / (BK / 8), kc = (c % (BK / 8)) * 8;
      *reinterpret_cast<u32x4*>(&Bs[buf][row * LDS_PITCH + kc]) = rb[i];
    }
  };

  float4_t acc[TM][TN];
#pragma unroll
  for (int i = 0; i < TM; ++i)
#pragma unroll
    for (int j = 0; j < TN; ++j) acc[i][j] = float4_t{0.f, 0.f, 0.f, 0.f};

  const int nk = (int)((K + BK - 1) / BK);
  gload(0);
  sstore(0);
  __syncthreads();
  for (int kt = 0; kt < nk; ++kt) {
    const int cur = kt & 1;
    if (kt + 1 < nk) gload((int64_t)(kt + 1) * BK);
#pragma unroll
    for (int ks = 0; ks < BK / 32; ++ks) {
      bf16x8_t af[TM], bf[TN];
#pragma unroll
      for (int i = 0; i < TM; ++i)
        af[i] = *reinterpret_cast<const bf16x8_t*>(&As[cur][(wm * WM + 16 * i + l16) * LDS_PITCH + 32 * ks + 8 * g]);
#pragma unroll
      for (int j = 0; j < TN; ++j)
        bf[j] = *reinterpret_cast<const bf16x8_t*>(&Bs[cur][(wn * WN + 16 * j + l16) * LDS_PITCH + 32 * ks + 8 * g]);
#pragma unroll
      for (int i = 0; i < TM; ++i)
#pragma unroll
        for (int j = 0; j < TN; ++j) acc[i][j] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(bf[j], af[i], acc[i][j], 0, 0, 0);
    }
    if (kt + 1 < nk) {
      sstore(cur ^ 1);
      __syncthreads();
    }
  }

  // acc[i][j] (A = B-tile, B = A-tile) holds C^T: lane (l16, g) has columns n = 16j + 4g + r, row m = 16i + l16
#pragma unroll
  for (int i = 0; i < TM; ++i) {
    const int64_t row = m0 + wm * WM + 16 * i + l16;
    if (row >= M) continue;
#pragma unroll
    for (int j = 0; j < TN; ++j) {
      const int64_t col0 = n0 + wn * WN + 16 * j + 4 * g;
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        const int64_t col = col0 + r;
        if (col >= N) continue;
        float v = Elem<FS_BF16>::round(acc[i][j][r]);
        if (R) v = v + bf16_to_f32(R[row * ldr + col]);
        C[row * ldc + col] = f32_to_bf16(v);
      }
    }
  }
}

// ------------------------------------------------------------------------------------------------
// bf16 MFMA kernel with an LDS ring fed by direct global->LDS loads (M > 64, K % 64 == 0)
//
// 4 waves in 2x2 compute a BM x BN tile of C. K advances in 64-deep stages; NS stages live in LDS and
// NS-1 are in flight while one is consumed. Every 16-byte chunk of a stage is copied by
// global_load_lds_dwordx4 (lane l of an instruction lands at LDS base + 16*l), so in-flight data
// costs no VGPRs. Rows are stored with their eight 16-byte chunks XOR-swizzled by (row & 7): the
// MFMA operand reads (ds_read_b128, 8 lanes per bank cycle) are conflict-free. The loads are issued
// from inline asm, so the waits are explicit (`s_waitcnt vmcnt`) and one barrier per stage orders
// the LDS ring. Operand roles, k order and the one-accumulator chain match gemm_bf16_kernel.
// ------------------------------------------------------------------------------------------------
#pragma clang diagnostic push
#pragma clang diagnostic ignored "-Winline-asm"
FS_DEVICE void dma16(const void* g, uint32_t lds) {
  const uint32_t l = __builtin_amdgcn_readfirstlane(lds);  // the LDS base is the same for the whole wave
  asm volatile("s_mov_b32 m0, %1\n\tglobal_load_lds_dwordx4 %0, off" ::"v"(g), "s"(l) : "memory", "m0");
}
// the same copy marked non-temporal: the weights stream through once, and keeping them out of the way
// in L2 leaves the activation panel (re-read by every column tile) resident (about 3% at M = 448)
FS_DEVICE void dma16_nt(const void* g, uint32_t lds) {
  const uint32_t l = __builtin_amdgcn_readfirstlane(lds);
  asm volatile("s_mov_b32 m0, %1\n\tglobal_load_lds_dwordx4 %0, off nt" ::"v"(g), "s"(l) : "memory", "m0");
}
#pragma clang diagnostic pop

template <int N>
FS_DEVICE void wait_vm() {
  asm volatile("s_waitcnt vmcnt(%0)" ::"n"(N) : "memory");
}

// Row statistics epilogue (the LM head feeding sampling and acceptance, sampling.py:13): for every
// output row and every WN-column block of a wave, the softmax statistics of the stored (bf16-rounded)
// values x at that row's temperature (y = x / T, a true division; y = x at T == 1 and at T == 0,
// whose rows use only the argmax), written to stats[row * ld + column / WN].
struct RowStatsOut {
  const float* temp;    // [M], or null for T = 1
  SoftmaxStat* stats;   // row m's nparts records at stats + m * ld
  int64_t nparts, ld;
};

// SWIGLU: W holds [gate; up] (N/2 rows each) and the tile's output columns are interleaved, column
// 2j = gate row j and 2j + 1 = up row j, so that each lane's four consecutive columns are two (gate, up)
// pairs; the epilogue stores silu(gate) * up to C[row][j] (model.py:93) instead of the products.
// SERIAL: the workgroup runs the `serial` K splits of its tile one after the other (gridDim.y == 1):
// each split's chain starts from zero as a split-K workgroup's does, and its result is added to a
// running f32 sum in increasing split order, the additions the split-K reduction makes, so the output
// equals the split-K path's bit for bit with no partials written.
template <int BM, int BN, int NS, int WGM = 2, int WGN = 2, bool STATS = false, bool PRIO = false, bool SWIGLU = false,
          bool SERIAL = false>
__global__ void __launch_bounds__(64 * WGM * WGN) gemm_bf16_lds_kernel(const uint16_t* __restrict__ X, int64_t ldx,
                                                            const uint16_t* __restrict__ W, int64_t ldw,
                                                            uint16_t* __restrict__ C, int64_t ldc,
                                                            const uint16_t* __restrict__ R, int64_t ldr, int64_t M,
                                                            int64_t N, int64_t K, int tiles_m, int ntiles,
                                                            float* __restrict__ part, RowStatsOut rs, int serial) {
  constexpr int KB = 64;                       // k per stage
  constexpr int ROWB = KB * 2;                 // bytes per stage row (128)
  constexpr int NW = WGM * WGN;                // waves: WGM along M, WGN along N
  constexpr int XB = BM * ROWB, WB = BN * ROWB, STAGE = XB + WB;
  constexpr int WM = BM / WGM, WN = BN / WGN, TM = WM / 16, TN = WN / 16;
  // A stage is T copies of 1 KB (one global_load_lds_dwordx4 of 64 lanes): copies q < XQ fill the X
  // block, the rest the W block. Wave w issues copies w, w + NW, ...: GH of them if w < T % NW,
  // else GL (tiles of 224 rows do not split evenly over 8 waves).
  constexpr int XQ = XB / 1024, T = STAGE / 1024, GI = (T + NW - 1) / NW;
  constexpr int GL = T / NW, GH = (T % NW) ? GL + 1 : GL;
  static_assert(XB % 1024 == 0 && WB % 1024 == 0, "tile rows must fill whole 1 KB copies");
  static_assert(WM % 16 == 0 && WN % 16 == 0, "wave tiles are whole 16x16 MFMA tiles");
  static_assert(NS * STAGE <= 160 * 1024, "LDS ring larger than a CU's LDS");
  static_assert(NS >= 2 && NS <= 4, "wait_stages covers up to two stages in flight behind the awaited one");
  __shared__ __attribute__((aligned(1024))) char smem[NS * STAGE];

  // XCD-aware order: workgroup ids go round-robin over the 8 XCDs; give each XCD a contiguous range
  // of tiles, M fastest inside groups of at most 8 row tiles, so the tiles an XCD runs at once share
  // both their activation and their weight k-slabs through its L2. (With all of M in one column of
  // tiles, a long batch re-read its whole activation panel for every column of weight tiles.) With
  // 8 row tiles or fewer this is plain M-fastest order.
  const int per_xcd = (ntiles + 7) / 8;
  const int tile = (blockIdx.x % 8) * per_xcd + blockIdx.x / 8;
  if (tile >= ntiles) return;
  const int tiles_n = ntiles / tiles_m;
  const int grp = tile / (8 * tiles_n), first = 8 * grp, gm = min(tiles_m - first, 8);
  const int in_grp = tile - grp * 8 * tiles_n;
  const int64_t m0 = (int64_t)(first + in_grp % gm) * BM;
  const int64_t n0 = (int64_t)(in_grp / gm) * BN;

  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int l16 = lane & 15, g = lane >> 4;
  const int wm = wave / WGN, wn = wave % WGN;
  const uint32_t lds0 = (uint32_t)(uintptr_t)smem;

  // this lane's source row/chunk for each of its copies (fixed across stages but for k0). Chunk P of
  // a block is row P >> 3, physical chunk P & 7, which holds logical chunk (P & 7) ^ (row & 7).
  const uint16_t* src[GI];
#pragma unroll
  for (int i = 0; i < GI; ++i) {
    const int q0 = i * NW + wave, q = q0 < T ? q0 : 0;
    const bool in_x = q < XQ;
    const int P = (in_x ? q : q - XQ) * 64 + lane;
    const int r = P >> 3, c = (P & 7) ^ (r & 7);
    int64_t gr = (in_x ? m0 : n0) + r;
    const int64_t lim = in_x ? M : N;
    gr = gr < lim ? gr : lim - 1;
    if (SWIGLU && !in_x) gr = (gr & 1) ? N / 2 + (gr >> 1) : (gr >> 1);   // interleaved column -> weight row
    src[i] = in_x ? X + gr * ldx + 8 * c : W + gr * ldw + 8 * c;
  }
  const bool hi = wave < T % NW;
  // split-K: workgroup row blockIdx.y takes the k-range [split*K/S, (split+1)*K/S)
  const int split = blockIdx.y;
  const int nk = (int)(K / KB) / (int)gridDim.y;
  const int64_t kbase = (int64_t)split * nk * KB;
  auto issue = [&](int kt) {
    const uint32_t base = lds0 + (uint32_t)((kt % NS) * STAGE);
    const int64_t k0 = kbase + (int64_t)kt * KB;
#pragma unroll
    for (int i = 0; i < GI; ++i) {
      const int q = i * NW + wave;
      if (q < T) {
        if (q >= XQ) dma16_nt(src[i] + k0, base + (uint32_t)(q * 1024));   // a weight copy
        else dma16(src[i] + k0, base + (uint32_t)(q * 1024));
      }
    }
  };
  // wait until at most `later` stages' copies (issued after the one being waited for) are in flight
  auto wait_stages = [&](int later) {
    if (hi || GH == GL) {
      if (later >= 2) wait_vm<2 * GH>();
      else if (later == 1) wait_vm<GH>();
      else wait_vm<0>();
    } else {
      if (later >= 2) wait_vm<2 * GL>();
      else if (later == 1) wait_vm<GL>();
      else wait_vm<0>();
    }
  };

  float4_t acc[TM][TN], sum[TM][TN];
#pragma unroll
  for (int i = 0; i < TM; ++i)
#pragma unroll
    for (int j = 0; j < TN; ++j) acc[i][j] = float4_t{0.f, 0.f, 0.f, 0.f};
  // SERIAL: fold the finished split's chain into the running sum and restart the chain from zero
  const int nks = SERIAL ? nk / serial : nk;
  auto fold = [&](bool first) {
#pragma unroll
    for (int i = 0; i < TM; ++i)
#pragma unroll
      for (int j = 0; j < TN; ++j) {
#pragma unroll
        for (int r = 0; r < 4; ++r) sum[i][j][r] = first ? acc[i][j][r] : sum[i][j][r] + acc[i][j][r];
        acc[i][j] = float4_t{0.f, 0.f, 0.f, 0.f};
      }
  };

#pragma unroll
  for (int s = 0; s < NS - 1; ++s)
    if (s < nk) issue(s);

  for (int kt = 0; kt < nk; ++kt) {
    if (SERIAL && kt > 0 && kt % nks == 0) fold(kt == nks);
    // stages issued after kt and still allowed in flight: min(NS - 2, nk - 1 - kt)
    wait_stages(min(NS - 2, nk - 1 - kt));
    __syncthreads();  // stage kt has landed for every wave; stage kt-1 is no longer being read
    if (kt + NS - 1 < nk) issue(kt + NS - 1);
    const char* st = smem + (kt % NS) * STAGE;
#pragma unroll
    for (int ks = 0; ks < KB / 32; ++ks) {
      bf16x8_t xf[TM], wf[TN];
#pragma unroll
      for (int i = 0; i < TM; ++i) {
        const int r = wm * WM + 16 * i + l16, c = (4 * ks + g) ^ (r & 7);
        xf[i] = *reinterpret_cast<const bf16x8_t*>(st + r * ROWB + 16 * c);
      }
#pragma unroll
      for (int j = 0; j < TN; ++j) {
        const int r = wn * WN + 16 * j + l16, c = (4 * ks + g) ^ (r & 7);
        wf[j] = *reinterpret_cast<const bf16x8_t*>(st + XB + r * ROWB + 16 * c);
      }
      // with 4 waves per SIMD, the wave holding its operands issues its MFMA block ahead of the others
      if (PRIO) __builtin_amdgcn_s_setprio(1);
#pragma unroll
      for (int i = 0; i < TM; ++i)
#pragma unroll
        for (int j = 0; j < TN; ++j) acc[i][j] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(wf[j], xf[i], acc[i][j], 0, 0, 0);
      if (PRIO) __builtin_amdgcn_s_setprio(0);
    }
  }
  if (SERIAL) {   // the last split, then the sum takes the accumulators' place in the epilogue
    fold(nk == nks);
#pragma unroll
    for (int i = 0; i < TM; ++i)
#pragma unroll
      for (int j = 0; j < TN; ++j) acc[i][j] = sum[i][j];
  }

  // acc[i][j]: lane (l16, g) holds C[m = 16i + l16][n = 16j + 4g + r], r = 0..3 (wave-local)
  if (SWIGLU) {   // (no split, no residual on this path; N % 4 == 0)
#pragma unroll
    for (int i = 0; i < TM; ++i) {
      const int64_t row = m0 + wm * WM + 16 * i + l16;
      if (row >= M) continue;
#pragma unroll
      for (int j = 0; j < TN; ++j) {
        const int64_t col0 = n0 + wn * WN + 16 * j + 4 * g;
        if (col0 >= N) continue;
        float v[4];
#pragma unroll
        for (int r = 0; r < 4; ++r) v[r] = Elem<FS_BF16>::round(acc[i][j][r]);
        const uint32_t h0 = f32_to_bf16(silu_times<FS_BF16>(v[0], v[1]));
        const uint32_t h1 = f32_to_bf16(silu_times<FS_BF16>(v[2], v[3]));
        *reinterpret_cast<uint32_t*>(C + row * ldc + col0 / 2) = h0 | (h1 << 16);
      }
    }
    return;
  }
  if (part) {   // split-K: f32 partial of this k-range, summed in split order by gemm_splitk_reduce_kernel
#pragma unroll
    for (int i = 0; i < TM; ++i) {
      const int64_t row = m0 + wm * WM + 16 * i + l16;
      if (row >= M) continue;
#pragma unroll
      for (int j = 0; j < TN; ++j) {
        const int64_t col0 = n0 + wn * WN + 16 * j + 4 * g;   // N % 4 == 0 on this path
        if (col0 < N) *reinterpret_cast<float4_t*>(part + ((int64_t)split * M + row) * N + col0) = acc[i][j];
      }
    }
    return;
  }
#pragma unroll
  for (int i = 0; i < TM; ++i) {
    const int64_t row = m0 + wm * WM + 16 * i + l16;
    if (row >= M) continue;
#pragma unroll
    for (int j = 0; j < TN; ++j) {
      const int64_t col0 = n0 + wn * WN + 16 * j + 4 * g;
      uint16_t o[4];
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        float v = Elem<FS_BF16>::round(acc[i][j][r]);
        if (R && col0 + r < N) v = v + bf16_to_f32(R[row * ldr + col0 + r]);
        o[r] = f32_to_bf16(v);
      }
      if (col0 + 3 < N && ((ldc | col0) & 3) == 0) {
        typedef __attribute__((__vector_size__(2 * sizeof(uint32_t)))) uint32_t u32x2;
        *reinterpret_cast<u32x2*>(C + row * ldc + col0) =
            u32x2{(uint32_t)o[0] | ((uint32_t)o[1] << 16), (uint32_t)o[2] | ((uint32_t)o[3] << 16)};
      } else {
#pragma unroll
        for (int r = 0; r < 4; ++r)
          if (col0 + r < N) C[row * ldc + col0 + r] = o[r];
      }
    }
  }
  if (STATS) {   // (no residual on this path: the statistics are of the rounded products)
    constexpr float L2E = 1.4426950408889634f;
    const int64_t p = (n0 + wn * WN) / WN;
#pragma unroll
    for (int i = 0; i < TM; ++i) {
      // the four lanes l16 + 16g share a row: their shuffles never mix rows, so rows past M are
      // harmless and are simply not written
      const int64_t row = m0 + wm * WM + 16 * i + l16;
      const float temp = (rs.temp && row < M) ? rs.temp[row] : 1.f;
      // y = x / T in place of the products (the logits are stored already); the division only where
      // some row of the wave has a temperature other than 0 and 1
      const bool div = __any(temp != 1.f && temp > 0.f);
      float ym = -INFINITY, av = -INFINITY;
      int ai = 0x7fffffff;
#pragma unroll
      for (int j = 0; j < TN; ++j) {
        const int64_t col0 = n0 + wn * WN + 16 * j + 4 * g;
#pragma unroll
        for (int r = 0; r < 4; ++r) {
          const float v = Elem<FS_BF16>::round(acc[i][j][r]);
          const float y = (div && temp != 1.f && temp > 0.f) ? v / temp : v;
          acc[i][j][r] = y;
          if (col0 + r >= N) continue;
          ym = fmaxf(ym, y);
          argmax_merge(av, ai, v, (int)(col0 + r));
        }
      }
#pragma unroll
      for (int o = 16; o <= 32; o <<= 1) {
        ym = fmaxf(ym, __shfl_xor(ym, o, 64));
        const float ov = __shfl_xor(av, o, 64);
        const int oi = __shfl_xor(ai, o, 64);
        argmax_merge(av, ai, ov, oi);
      }
      const float ml = ym * L2E;
      float se = 0.f;
#pragma unroll
      for (int j = 0; j < TN; ++j) {
        const int64_t col0 = n0 + wn * WN + 16 * j + 4 * g;
#pragma unroll
        for (int r = 0; r < 4; ++r)
          if (col0 + r < N) se += __builtin_amdgcn_exp2f(fmaf(acc[i][j][r], L2E, -ml));
      }
      se += __shfl_xor(se, 16, 64);   // (g0 + g1) + (g2 + g3) in every lane
      se += __shfl_xor(se, 32, 64);
      if (g == 0 && row < M && p < rs.nparts) rs.stats[row * rs.ld + p] = SoftmaxStat{ym, ym == -INFINITY ? 0.f : se, av, ai};
    }
  }
}

// C = round(sum_s part[s]) (+ R, rounded again): the split-K partials added in increasing split order,
// then the same epilogue as the unsplit kernel. Four consecutive elements per thread (N % 4 == 0).
__global__ void __launch_bounds__(256) gemm_splitk_reduce_kernel(const float* __restrict__ part, int splits,
                                                                 int64_t M, int64_t N, uint16_t* __restrict__ C,
                                                                 int64_t ldc, const uint16_t* __restrict__ R,
                                                                 int64_t ldr) {
  const int64_t e = ((int64_t)blockIdx.x * 256 + threadIdx.x) * 4;
  if (e >= M * N) return;
  const int64_t row = e / N, col = e - row * N;
  float4_t a = *reinterpret_cast<const float4_t*>(part + e);
  for (int sp = 1; sp < splits; ++sp) {
    const float4_t b = *reinterpret_cast<const float4_t*>(part + (int64_t)sp * M * N + e);
    a[0] += b[0];
    a[1] += b[1];
    a[2] += b[2];
    a[3] += b[3];
  }
  uint16_t o[4];
#pragma unroll
  for (int r = 0; r < 4; ++r) {
    float v = Elem<FS_BF16>::round(a[r]);
    if (R) v = v + bf16_to_f32(R[row * ldr + col + r]);
    o[r] = f32_to_bf16(v);
  }
  if (((ldc | col) & 3) == 0) {
    typedef __attribute__((__vector_size__(2 * sizeof(uint32_t)))) uint32_t u32x2;
    *reinterpret_cast<u32x2*>(C + row * ldc + col) =
        u32x2{(uint32_t)o[0] | ((uint32_t)o[1] << 16), (uint32_t)o[2] | ((uint32_t)o[3] << 16)};
  } else {
#pragma unroll
    for (int r = 0; r < 4; ++r) C[row * ldc + col + r] = o[r];
  }
}

// ------------------------------------------------------------------------------------------------
// VALU kernel (f32 / f16 / unaligned bf16): 64x64 tile, 16-deep k stages, 4x4 outputs per thread
// ------------------------------------------------------------------------------------------------
template <int DT>
__global__ void __launch_bounds__(256) gemm_valu_kernel(const typename Elem<DT>::T* __restrict__ A, int64_t lda,
                                                        const typename Elem<DT>::T* __restrict__ B, int64_t ldb,
                                                        typename Elem<DT>::T* __restrict__ C, int64_t ldc,
                                                        const typename Elem<DT>::T* __restrict__ R, int64_t ldr,
                                                        int64_t M, int64_t N, int64_t K, int tiles_n) {
  typedef Elem<DT> E;
  constexpr int T = 64, KB = 16;
  __shared__ float As[KB][T + 4];
  __shared__ float Bs[KB][T + 4];
  const int tid = threadIdx.x;
  const int tile = blockIdx.x;
  const int64_t m0 = (int64_t)(tile / tiles_n) * T;
  const int64_t n0 = (int64_t)(tile % tiles_n) * T;
  const int tx = tid & 15, ty = tid >> 4;
  float acc[4][4] = {};
  for (int64_t k0 = 0; k0 < K; k0 += KB) {
    for (int c = tid; c < T * KB; c += 256) {
      const int r = c / KB, kk = c % KB;
      const int64_t gk = k0 + kk;
      const int64_t am = m0 + r, bn = n0 + r;
      As[kk][r] = (am < M && gk < K) ? E::load(A, am * lda + gk) : 0.f;
      Bs[kk][r] = (bn < N && gk < K) ? E::load(B, bn * ldb + gk) : 0.f;
    }
    __syncthreads();
#pragma unroll
    for (int kk = 0; kk < KB; ++kk) {
      float a[4], b[4];
#pragma unroll
      for (int i = 0; i < 4; ++i) a[i] = As[kk][ty * 4 + i];
#pragma unroll
      for (int j = 0; j < 4; ++j) b[j] = Bs[kk][tx * 4 + j];
#pragma unroll
      for (int i = 0; i < 4; ++i)
#pragma unroll
        for (int j = 0; j < 4; ++j) acc[i][j] = fmaf(a[i], b[j], acc[i][j]);
    }
    __syncthreads();
  }
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const int64_t row = m0 + ty * 4 + i;
    if (row >= M) continue;
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const int64_t col = n0 + tx * 4 + j;
      if (col >= N) continue;
      float v = E::round(acc[i][j]);
      if (R) v = v + E::load(R, row * ldr + col);
      E::store(C, row * ldc + col, v);
    }
  }
}

bool aligned16(const void* p) { return (reinterpret_cast<uintptr_t>(p) & 15) == 0; }

// Split-K factor of a bf16 GEMM with K % 64 == 0. It depends on (N, K) only, never on M, so a row's
// arithmetic (the k-ranges and the order their partials are added) is the same whatever the batch:
// a decode step and a verify pass produce bit-identical rows. Narrow outputs (N < 16384) are split
// so that a 64-row decode step still spreads its weight stream over the whole GPU.
int split_for(int64_t N, int64_t K) {
  if (K % 64) return 1;
  int s = 1;
  while (s < 8 && N * (2 * s) <= 16384 && (K / 64) % (2 * s) == 0 && K / (2 * s) >= 512) s *= 2;
  return s;
}

// The LDS-kernel configuration a shape runs with. M <= 64 (a decode step) takes 64-row tiles. Larger
// M takes 224-row tiles when they pad M less than 128- and 256-row tiles would (the verify pass,
// M = 64 * 7 = 448, is exactly two), else 256- or 128-row tiles. Every configuration runs the same
// MFMA over the same k order, so the tile shape never changes a result.
struct LdsCfg {
  int bm, bn, wgm, wgn;
};

// Share of the CU slots a grid of `tiles` workgroups keeps busy (one tile per CU at a time, 256 CUs).
double tile_fill(int64_t tiles) {
  constexpr int64_t kCUs = 256;
  return (double)tiles / (double)(kCUs * ((tiles + kCUs - 1) / kCUs));
}

LdsCfg lds_cfg(int64_t M, int64_t N, int splits, bool stats = false) {
  // 64-row tiles; very wide outputs (an LM head) take 128 columns per tile, still 32 per wave, and
  // with the statistics epilogue (the draft head, 128256 columns) 256 columns over 16 waves: 501
  // tiles fit the CUs' 512 slots in one pass (189 -> 168 us at the 8B draft head's shape)
  if (M <= 64)
    return N * splits >= 65536 ? (stats ? LdsCfg{64, 256, 2, 8} : LdsCfg{64, 128, 2, 4}) : LdsCfg{64, 64, 2, 2};
  auto pad = [&](int64_t bm) { return (M + bm - 1) / bm * bm - M; };
  if (pad(224) < pad(128) && pad(224) < pad(256)) {
    const int64_t tm = (M + 223) / 224;
    if (stats) {   // 16 waves of 32-column blocks: the blocks a 64-row head's statistics use too
      const int64_t t256 = tm * ((N + 255) / 256);
      return t256 >= 192 ? LdsCfg{224, 256, 2, 8} : LdsCfg{224, 128, 2, 4};
    }
    // the width whose tile count fills the CUs best, weighted by the throughput a tile of that
    // width reaches (measured on the decoder's projections at M = 448: wider tiles re-read less)
    struct Cand {
      LdsCfg cf;
      double eff;
    };
    const Cand cands[] = {{{224, 256, 2, 8}, 1.0}, {{224, 224, 7, 2}, 0.97}, {{224, 128, 2, 4}, 0.85},
                          {{224, 96, 7, 2}, 0.8}};
    LdsCfg best = cands[0].cf;
    double best_score = -1.0;
    for (const Cand& c : cands) {
      const double score = tile_fill(tm * ((N + c.cf.bn - 1) / c.cf.bn) * splits) * c.eff;
      if (score > best_score) best_score = score, best = c.cf;
    }
    return best;
  }
  const int64_t t256 = ((M + 255) / 256) * ((N + 255) / 256) * splits;
  const int64_t t128 = ((M + 127) / 128) * ((N + 255) / 256) * splits;
  if (t256 >= 192) return LdsCfg{256, 256, 4, 2};
  if (t128 >= 128) return LdsCfg{128, 256, 2, 4};
  return LdsCfg{128, 128, 2, 4};
}

template <bool STATS, bool SWIGLU = false>
void launch_lds(const uint16_t* a, int64_t lda, const uint16_t* b, int64_t ldb, uint16_t* c, int64_t ldc,
                const uint16_t* r, int64_t ldr, int64_t M, int64_t N, int64_t K, int splits, float* part,
                RowStatsOut rs, hipStream_t s) {
  const LdsCfg cf = lds_cfg(M, N, splits, STATS);
  const int tm = (int)((M + cf.bm - 1) / cf.bm), nt = tm * (int)((N + cf.bn - 1) / cf.bn);
  const dim3 grid((unsigned)(8 * ((nt + 7) / 8)), (unsigned)splits);
#define FS_LDS_LAUNCH(BM_, BN_, NS_, WGM_, WGN_, PRIO_)                                                       \
  gemm_bf16_lds_kernel<BM_, BN_, NS_, WGM_, WGN_, STATS, PRIO_, SWIGLU><<<grid, 64 * WGM_ * WGN_, 0, s>>>(      \
      a, lda, b, ldb, c, ldc, r, ldr, M, N, K, tm, nt, part, rs, 1)
  // 64 x 256 with a 2-stage ring (80 KB of LDS) and 64 x 128 with a 3-stage ring (72 KB): two
  // workgroups share a CU, so one's epilogue (the head's statistics) overlaps the other's weight stream
  if (cf.bm == 64 && cf.bn == 256) FS_LDS_LAUNCH(64, 256, 2, 2, 8, false);
  else if (cf.bm == 64 && cf.bn == 128) FS_LDS_LAUNCH(64, 128, 3, 2, 4, false);
  else if (cf.bm == 64) FS_LDS_LAUNCH(64, 64, 4, 2, 2, false);
  else if (cf.bm == 224 && cf.bn == 256 && cf.wgn == 8) FS_LDS_LAUNCH(224, 256, 2, 2, 8, true);
  else if (cf.bm == 224 && cf.bn == 256) FS_LDS_LAUNCH(224, 256, 2, 2, 4, false);
  else if (cf.bm == 224 && cf.bn == 224) FS_LDS_LAUNCH(224, 224, 2, 7, 2, false);
  else if (cf.bm == 224 && cf.bn == 96) FS_LDS_LAUNCH(224, 96, 3, 7, 2, false);
  else if (cf.bm == 224) FS_LDS_LAUNCH(224, 128, 3, 2, 4, false);
  else if (cf.bm == 256) FS_LDS_LAUNCH(256, 256, 2, 4, 2, false);
  else if (cf.bn == 256) FS_LDS_LAUNCH(128, 256, 3, 2, 4, false);
  else FS_LDS_LAUNCH(128, 128, 4, 2, 4, false);
#undef FS_LDS_LAUNCH
}

bool lds_ok(const void* A, int64_t lda, const void* B, int64_t ldb, int64_t K) {
  return K % 64 == 0 && lda % 8 == 0 && ldb % 8 == 0 && aligned16(A) && aligned16(B);
}

// A split-K shape whose unsplit 256 x 128 tiles alone fill the GPU twice over (a long prefill) runs its
// K splits one after the other inside each workgroup: the split-K arithmetic without the f32 partials.
// Only for splits of at most 2048 k: there the partials' HBM traffic costs more than the narrower tile
// the running sum forces (measured at M = 32768: the o projection 1.80 -> 1.38 ms, qkv even); with
// 3584-k splits (the down projection) the 256 x 256 tiles and their partials are faster (3.9 vs 4.6 ms).
constexpr int kSerialTiles = 512;
bool serial_for(int64_t M, int64_t N, int64_t K, int splits) {
  return splits > 1 && K / splits <= 2048 && ((M + 255) / 256) * ((N + 127) / 128) >= kSerialTiles;
}

void launch_serial(const uint16_t* a, int64_t lda, const uint16_t* b, int64_t ldb, uint16_t* c, int64_t ldc,
                   const uint16_t* r, int64_t ldr, int64_t M, int64_t N, int64_t K, int splits, hipStream_t s) {
  // 256 x 128 tiles, 8 waves of 64 x 64 (the running sum doubles the accumulators), 3-stage ring (144 KB)
  const int tm = (int)((M + 255) / 256), nt = tm * (int)((N + 127) / 128);
  gemm_bf16_lds_kernel<256, 128, 3, 4, 2, false, false, false, true>
      <<<dim3((unsigned)(8 * ((nt + 7) / 8)), 1u), 512, 0, s>>>(a, lda, b, ldb, c, ldc, r, ldr, M, N, K, tm, nt,
                                                                nullptr, RowStatsOut{}, splits);
}

}  // namespace

extern "C" int64_t fs_gemm_row_stats_parts(int64_t M, int64_t N, int64_t K) {
  if (M <= 0 || N <= 0 || K <= 0 || K % 64 || split_for(N, K) != 1) return 0;
  const LdsCfg cf = lds_cfg(M, N, 1, true);
  const int64_t wn = cf.bn / cf.wgn;
  return (N + wn - 1) / wn;
}

extern "C" int fs_gemm_row_stats(const void* A, int64_t lda, const void* B, int64_t ldb, void* C, int64_t ldc,
                                 int64_t M, int64_t N, int64_t K, const float* temperature, void* stats,
                                 int64_t stats_ld, int64_t nparts, void* stream) {
  FS_CHECK_ARG(A && B && C && stats, "gemm_row_stats: null pointer");
  FS_CHECK_ARG(M >= 0 && N > 0 && N < 0x7fffffff && K > 0, "gemm_row_stats: M %lld N %lld K %lld", (long long)M,
               (long long)N, (long long)K);
  FS_CHECK_ARG(lda >= K && ldb >= K && ldc >= N, "gemm_row_stats: leading dimensions");
  FS_CHECK_ARG(lds_ok(A, lda, B, ldb, K), "gemm_row_stats: needs K %% 64 == 0 and 16-byte aligned rows");
  const int64_t want = fs_gemm_row_stats_parts(M, N, K);
  FS_CHECK_ARG(want > 0 && nparts == want, "gemm_row_stats: nparts %lld, the shape needs %lld", (long long)nparts,
               (long long)want);
  FS_CHECK_ARG(stats_ld >= nparts && (reinterpret_cast<uintptr_t>(stats) & 15) == 0,
               "gemm_row_stats: stats_ld %lld < nparts (or stats not 16-byte aligned)", (long long)stats_ld);
  if (M == 0) return 0;
  launch_lds<true>((const uint16_t*)A, lda, (const uint16_t*)B, ldb, (uint16_t*)C, ldc, nullptr, 0, M, N, K, 1, nullptr,
                   RowStatsOut{temperature, reinterpret_cast<SoftmaxStat*>(stats), nparts, stats_ld},
                   fs::as_stream(stream));
  return fs::launch_status("gemm_row_stats");
}

extern "C" int32_t fs_gemm_splits(int64_t N, int64_t K, int32_t dtype) {
  if (N <= 0 || K <= 0 || dtype != FS_BF16 || N % 4) return 1;
  return split_for(N, K);
}

extern "C" int32_t fs_gemm_serial(int64_t M, int64_t N, int64_t K, int32_t dtype) {
  if (M <= 0) return 0;
  return serial_for(M, N, K, fs_gemm_splits(N, K, dtype)) ? 1 : 0;
}

extern "C" int fs_gemm_partials(const void* A, int64_t lda, const void* B, int64_t ldb, int64_t M, int64_t N, int64_t K,
                                int32_t dtype, void* partials, int64_t partials_bytes, void* stream) {
  FS_CHECK_ARG(A && B && partials, "gemm_partials: null pointer");
  FS_CHECK_ARG(dtype == FS_BF16, "gemm_partials: bf16 only (dtype %d)", dtype);
  FS_CHECK_ARG(M >= 0 && N > 0 && K > 0 && lda >= K && ldb >= K, "gemm_partials: M %lld N %lld K %lld",
               (long long)M, (long long)N, (long long)K);
  FS_CHECK_ARG(lds_ok(A, lda, B, ldb, K) && N % 4 == 0, "gemm_partials: needs K %% 64 == 0, N %% 4 == 0, aligned rows");
  const int splits = split_for(N, K);
  FS_CHECK_ARG(splits > 1, "gemm_partials: N %lld K %lld does not split K", (long long)N, (long long)K);
  const int64_t need = (int64_t)splits * M * N * (int64_t)sizeof(float);
  FS_CHECK_ARG(partials_bytes >= need && (reinterpret_cast<uintptr_t>(partials) & 15) == 0,
               "gemm_partials: %lld < %lld bytes (or unaligned)", (long long)partials_bytes, (long long)need);
  if (M == 0) return 0;
  launch_lds<false>((const uint16_t*)A, lda, (const uint16_t*)B, ldb, nullptr, 0, nullptr, 0, M, N, K, splits,
                    reinterpret_cast<float*>(partials), RowStatsOut{}, fs::as_stream(stream));
  return fs::launch_status("gemm_partials");
}

extern "C" int fs_gemm_swiglu(const void* A, int64_t lda, const void* B, int64_t ldb, void* H, int64_t ldh, int64_t M,
                              int64_t F, int64_t K, int32_t dtype, void* stream) {
  FS_CHECK_ARG(A && B && H, "gemm_swiglu: null pointer");
  FS_CHECK_ARG(dtype == FS_BF16, "gemm_swiglu: bf16 only (dtype %d)", dtype);
  FS_CHECK_ARG(M >= 0 && F > 0 && F % 2 == 0 && 2 * F < 0x7fffffff && K > 0 && lda >= K && ldb >= K && ldh >= F &&
                   ldh % 2 == 0 && (reinterpret_cast<uintptr_t>(H) & 3) == 0,
               "gemm_swiglu: M %lld F %lld K %lld (F even, ldh even, H 4-byte aligned)", (long long)M, (long long)F,
               (long long)K);
  FS_CHECK_ARG(lds_ok(A, lda, B, ldb, K), "gemm_swiglu: needs K %% 64 == 0 and 16-byte aligned rows");
  FS_CHECK_ARG(split_for(2 * F, K) == 1, "gemm_swiglu: F %lld K %lld splits K", (long long)F, (long long)K);
  if (M == 0) return 0;
  launch_lds<false, true>((const uint16_t*)A, lda, (const uint16_t*)B, ldb, (uint16_t*)H, ldh, nullptr, 0, M, 2 * F, K,
                          1, nullptr, RowStatsOut{}, fs::as_stream(stream));
  return fs::launch_status("gemm_swiglu");
}

extern "C" int64_t fs_gemm_workspace_size(int64_t M, int64_t N, int64_t K, int32_t dtype) {
  if (M <= 0 || N <= 0 || K <= 0 || dtype != FS_BF16) return 0;
  const int s = split_for(N, K);
  return s > 1 && !serial_for(M, N, K, s) ? (int64_t)s * M * N * (int64_t)sizeof(float) : 0;
}

extern "C" int fs_gemm(const void* A, int64_t lda, const void* B, int64_t ldb, void* C, int64_t ldc, const void* R,
                       int64_t ldr, int64_t M, int64_t N, int64_t K, int32_t dtype, void* workspace,
                       int64_t workspace_bytes, void* stream) {
  FS_CHECK_ARG(A && B && C, "gemm: null pointer");
  FS_CHECK_ARG(dtype == FS_F32 || dtype == FS_BF16 || dtype == FS_F16, "gemm: dtype %d", dtype);
  FS_CHECK_ARG(M >= 0 && N > 0 && K > 0, "gemm: M %lld N %lld K %lld", (long long)M, (long long)N, (long long)K);
  FS_CHECK_ARG(lda >= K && ldb >= K && ldc >= N && (!R || ldr >= N), "gemm: leading dimensions");
  if (M == 0) return 0;
  hipStream_t s = fs::as_stream(stream);
  const bool mfma = dtype == FS_BF16 && K % 8 == 0 && lda % 8 == 0 && ldb % 8 == 0 && aligned16(A) && aligned16(B);
  if (mfma && lds_ok(A, lda, B, ldb, K)) {
    const uint16_t* a = (const uint16_t*)A;
    const uint16_t* b = (const uint16_t*)B;
    const int splits = N % 4 == 0 ? split_for(N, K) : 1;
    if (serial_for(M, N, K, splits)) {
      launch_serial(a, lda, b, ldb, (uint16_t*)C, ldc, (const uint16_t*)R, ldr, M, N, K, splits, s);
      return fs::launch_status("gemm_bf16_lds_serial");
    }
    float* part = nullptr;
    if (splits > 1) {
      const int64_t need = (int64_t)splits * M * N * (int64_t)sizeof(float);
      FS_CHECK_ARG(workspace && workspace_bytes >= need && (reinterpret_cast<uintptr_t>(workspace) & 15) == 0,
                   "gemm: workspace %lld < %lld bytes (or unaligned)", (long long)workspace_bytes, (long long)need);
      part = reinterpret_cast<float*>(workspace);
    }
    uint16_t* c = splits > 1 ? nullptr : (uint16_t*)C;
    launch_lds<false>(a, lda, b, ldb, c, ldc, (const uint16_t*)R, ldr, M, N, K, splits, part, RowStatsOut{}, s);
    if (int e = fs::launch_status("gemm_bf16_lds")) return e;
    if (splits > 1) {
      const int64_t n4 = M * N / 4;
      gemm_splitk_reduce_kernel<<<dim3((unsigned)((n4 + 255) / 256)), 256, 0, s>>>(part, splits, M, N, (uint16_t*)C,
                                                                                   ldc, (const uint16_t*)R, ldr);
      return fs::launch_status("gemm_splitk_reduce");
    }
    return 0;
  }
  if (mfma) {   // K % 64 != 0: register-staged MFMA tiles, no split
    const uint16_t* a = (const uint16_t*)A;
    const uint16_t* b = (const uint16_t*)B;
    if (M > 64) {
      const int tm = (int)((M + 127) / 128), tn = (int)((N + 127) / 128);
      gemm_bf16_kernel<128, 128><<<dim3((unsigned)(tm * tn)), 256, 0, s>>>(a, lda, b, ldb, (uint16_t*)C, ldc,
                                                                           (const uint16_t*)R, ldr, M, N, K, tn);
    } else {
      const int tm = (int)((M + 63) / 64), tn = (int)((N + 63) / 64);
      gemm_bf16_kernel<64, 64><<<dim3((unsigned)(tm * tn)), 256, 0, s>>>(a, lda, b, ldb, (uint16_t*)C, ldc,
                                                                         (const uint16_t*)R, ldr, M, N, K, tn);
    }
    return fs::launch_status("gemm_bf16");
  }
  const int tm = (int)((M + 63) / 64), tn = (int)((N + 63) / 64);
  dim3 grid((unsigned)(tm * tn));
  switch (dtype) {
    case FS_F32:
      gemm_valu_kernel<FS_F32><<<grid, 256, 0, s>>>((const float*)A, lda, (const float*)B, ldb, (float*)C, ldc,
                                                   (const float*)R, ldr, M, N, K, tn);
      break;
    case FS_BF16:
      gemm_valu_kernel<FS_BF16><<<grid, 256, 0, s>>>((const uint16_t*)A, lda, (const uint16_t*)B, ldb, (uint16_t*)C,
                                                    ldc, (const uint16_t*)R, ldr, M, N, K, tn);
      break;
    default:
      gemm_valu_kernel<FS_F16><<<grid, 256, 0, s>>>((const uint16_t*)A, lda, (const uint16_t*)B, ldb, (uint16_t*)C,
                                                   ldc, (const uint16_t*)R, ldr, M, N, K, tn);
      break;
  }
  return fs::launch_status("gemm_valu");
}
