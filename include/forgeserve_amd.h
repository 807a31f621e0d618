/*
 * forgeserve_amd: C ABI of the MI355X (gfx950) speculative-decoding hot path.
 *
 * Every pointer is caller-owned device memory unless stated otherwise; the library allocates
 * nothing. Every call is asynchronous on the HIP stream passed as `stream` (a hipStream_t, NULL for
 * the null stream) and returns
 *     0                 on success,
 *     FS_ERR_ARG (<0)   for an argument error found on the host (nothing was launched),
 *     > 0               a hipError_t reported by the launch.
 * fs_last_error() returns a thread-local message for the last non-zero return.
 *
 * Strides are in elements. Element types are given by a dtype code (FS_F32, FS_BF16, FS_F16).
 * Positions are int32; a negative position marks a padding token of a ragged batch: its KV slot is
 * not written and its attention output row is zero (the reference has no padding tokens; ragged
 * batches are this library's extension for batched speculation).
 *
 * The reference (forgeserve, pure PyTorch) has no C interface. Each entry point names the Python
 * function it replaces; forgeserve_amd/_lib.py is a ctypes binding of every entry point.
 */
#ifndef FORGESERVE_AMD_H
#define FORGESERVE_AMD_H

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define FS_F32 0
#define FS_BF16 1
#define FS_F16 2

#define FS_ERR_ARG (-1)

/* Layout of one layer of a paged KV pool.
 * Key element (block, head, slot, dim) lives at k[block*k_block + head*k_head + slot*k_slot + dim*k_dim],
 * or, when k_group != 0 (then k_dim == 1 and head_dim % 8 == 0), at
 * k[block*k_block + head*k_head + slot*k_slot + (dim/8)*k_group + dim%8]: keys stored as 8-dim groups.
 * Value element likewise with the v_* strides. The fast attention path wants dim-major values
 * (v_slot == 1, v_dim == block_size: a block's 16 keys of one dim are 32 contiguous bytes) and either
 * slot-major keys (k_slot == head_dim, k_dim == 1, k_group == 0) or grouped keys (k_slot == 8,
 * k_group == 8*block_size: a block's 16 keys of one 8-dim group are 256 contiguous bytes, so each
 * 16-byte-per-lane load of a key tile is one contiguous 1 KB run). */
typedef struct fs_kv_layout {
  void* k;
  void* v;
  int64_t k_block, k_head, k_slot, k_dim;
  int64_t v_block, v_head, v_slot, v_dim;
  int32_t block_size;
  int32_t n_kv_heads;
  int32_t head_dim;
  int32_t dtype;
  int64_t num_blocks; /* block ids outside [0, num_blocks) are never dereferenced */
  int64_t k_group;    /* 0: key dims at dim*k_dim; else the stride between 8-dim groups of a key */
} fs_kv_layout;

const char* fs_last_error(void);
/* 3 since fs_kv_layout gained k_group (a caller built against an older layout struct must be rebuilt). */
int fs_abi_version(void);

/* ---------------------------------------------------------------------------------------------- */
/* KV cache                                                                                         */
/* ---------------------------------------------------------------------------------------------- */

/* Fused rotary embedding + paged KV write for one layer of one forward.
 * Replaces model.py:64-67 (q/k/v split and apply_rope, model.py:40-45) and the scatter of
 * paged.py:74-78. qkv holds n_tokens rows of [q (n_heads*head_dim) | k | v] (the fused projection
 * output), row stride qkv_stride. Token m belongs to batch row m / T. Rotary: half-split rotation
 * at positions[m] with cos/sin rounded to the dtype (model.py:42-45); tables are f32
 * [rope_len, head_dim/2]. The key/value of token m go to cache position slots[m] (slots == NULL:
 * the rotary position, as in a paged view; a contiguous cache appends at its length instead,
 * kv.py:21-24). q_out receives the rotated queries, row stride q_stride, layout
 * [n_tokens, n_heads, head_dim]. */
int fs_qkv_rope_write(const void* qkv, int64_t qkv_stride, int64_t n_tokens, int32_t T, int32_t n_heads,
                      const int32_t* positions, const int32_t* slots, const float* rope_cos, const float* rope_sin,
                      int32_t rope_len, const int32_t* block_tables, int64_t table_stride,
                      int32_t max_blocks, const fs_kv_layout* kv, void* q_out, int64_t q_stride,
                      void* stream);

/* Scatter already-rotated keys/values into the pool: paged.py:74-78.
 * k_new/v_new element (b, h, t, d) at base + b*s_b + h*s_h + t*s_t + d (dim contiguous). */
int fs_paged_kv_write(const void* k_new, const void* v_new, int64_t s_b, int64_t s_h, int64_t s_t,
                      int32_t B, int32_t T, const int32_t* positions, const int32_t* block_tables,
                      int64_t table_stride, int32_t max_blocks, const fs_kv_layout* kv, void* stream);

/* fs_qkv_rope_write for packed prefill (varlen): n_tokens rows of several sequences back to back, with
 * no padding; token m uses table row token_row[m] (0 <= token_row[m] < n_rows: other tokens are
 * neither rotated nor written, and their q rows are zeros) at positions[m]. Replaces the same lines
 * as fs_qkv_rope_write for a prefill of several prompts at once (engine.py:80-95 prefills one prompt
 * of T = prompt length per step through paged.py:71-82). */
int fs_qkv_rope_write_varlen(const void* qkv, int64_t qkv_stride, int64_t n_tokens, int32_t n_heads,
                             const int32_t* positions, const int32_t* token_row, int32_t n_rows,
                             const float* rope_cos, const float* rope_sin, int32_t rope_len,
                             const int32_t* block_tables, int64_t table_stride, int32_t max_blocks,
                             const fs_kv_layout* kv, void* q_out, int64_t q_stride, void* stream);

/* fs_qkv_rope_write fed by the split-K partials of the QKV projection instead of its output: parts is
 * [splits][n_tokens][n_cols] f32 as fs_gemm_partials writes it (n_cols = (n_heads + 2*n_kv_heads) *
 * head_dim); each element is the partials added in increasing split order and rounded to the pool's
 * dtype, exactly what fs_gemm would have stored, then rotated and written as fs_qkv_rope_write does.
 * Replaces the same lines (model.py:64-67, 40-45; paged.py:74-78) with the projection's reduction
 * (model.py:57-60) folded in. 16-bit pools with head_dim/2 % 8 == 0 and 16-byte aligned data only. */
int fs_qkv_rope_write_partials(const float* parts, int32_t splits, int64_t n_tokens, int64_t n_cols, int32_t T,
                               int32_t n_heads, const int32_t* positions, const int32_t* slots,
                               const float* rope_cos, const float* rope_sin, int32_t rope_len,
                               const int32_t* block_tables, int64_t table_stride, int32_t max_blocks,
                               const fs_kv_layout* kv, void* q_out, int64_t q_stride, void* stream);

/* Gather every block of every row's table in table order: paged.py:80-81.
 * k_out, v_out: contiguous [B, n_kv_heads, max_blocks*block_size, head_dim]. */
int fs_paged_gather(const fs_kv_layout* kv, const int32_t* block_tables, int64_t table_stride, int32_t B,
                    int32_t max_blocks, void* k_out, void* v_out, void* stream);

/* ---------------------------------------------------------------------------------------------- */
/* Attention                                                                                        */
/* ---------------------------------------------------------------------------------------------- */

/* Causal GQA attention of each row's T queries over its paged keys/values.
 * Replaces the gather of paged.py:80-81 plus model.py:70-76 (repeat_interleave, key <= query-position
 * mask, scaled_dot_product_attention). q/out element (b, t, h, d) at base + b*s_b + t*s_t + h*s_h + d.
 * Query head h reads KV head h / (n_heads / n_kv_heads) (model.py:70-71). Query (b, t) sees the keys
 * at positions 0..positions[b*T+t] (model.py:75). workspace: at least
 * fs_paged_attention_workspace_size(...) bytes, 256-byte aligned, any contents. */
int fs_paged_attention(const void* q, int64_t q_sb, int64_t q_st, int64_t q_sh, const fs_kv_layout* kv,
                       const int32_t* block_tables, int64_t table_stride, int32_t max_blocks,
                       const int32_t* positions, int32_t B, int32_t T, int32_t n_heads, float scale,
                       void* out, int64_t o_sb, int64_t o_st, int64_t o_sh, void* workspace,
                       int64_t workspace_bytes, void* stream);

/* fs_paged_attention over packed sequences (varlen prefill): sequence s owns tokens
 * cu_seqlens[s] .. cu_seqlens[s+1]-1 of q and out (element (token, h, d) at base + token*s_t + h*s_h + d),
 * at most T of them; positions is [S, T], its first cu_seqlens[s+1]-cu_seqlens[s] entries of row s
 * the tokens' positions and the rest -1. Rows of q/out past the sequences' tokens are not touched.
 * Each query's result is bit-identical to fs_paged_attention's for the same query, keys and position.
 * Replaces model.py:70-76 over paged.py:80-81 for a prefill (T = prompt length, engine.py:80-95) of
 * several prompts at once. workspace: fs_paged_attention_workspace_size(S, T, ...). */
/* Keys per chunk of the MFMA attention path (FS_ATTN_SPLIT, default 16384), fixed for the life of the
 * process: a query at position p reads chunks 0 .. p / split and, past the first, its output is merged
 * from per-chunk partials. No counterpart in the reference (it gathers every key); for callers and
 * benchmarks that report how a workload is split. */
int32_t fs_paged_attention_split(void);

int fs_paged_attention_varlen(const void* q, int64_t q_st, int64_t q_sh, const fs_kv_layout* kv,
                              const int32_t* block_tables, int64_t table_stride, int32_t max_blocks,
                              const int32_t* positions, const int32_t* cu_seqlens, int32_t S, int32_t T,
                              int32_t n_heads, float scale, void* out, int64_t o_st, int64_t o_sh, void* workspace,
                              int64_t workspace_bytes, void* stream);

int64_t fs_paged_attention_workspace_size(int32_t B, int32_t T, int32_t n_heads, int32_t head_dim,
                                          int32_t max_blocks, int32_t block_size);

/* fs_paged_attention / fs_paged_attention_varlen for the second and later layers of one forward step:
 * every layer of a step attends with the same positions and tables (model.py:69-76 per Block, under one
 * engine step), so the work plan the first layer's call left in the workspace is taken as it is. The
 * plan is recomputed anyway unless the previous call on this host thread used the same workspace,
 * positions (and cu_seqlens), stream, B (S), T, n_heads and output alignment; the caller guarantees
 * that the positions still hold the values that call saw. Same arguments and results otherwise. */
int fs_paged_attention_reuse_plan(const void* q, int64_t q_sb, int64_t q_st, int64_t q_sh, const fs_kv_layout* kv,
                                  const int32_t* block_tables, int64_t table_stride, int32_t max_blocks,
                                  const int32_t* positions, int32_t B, int32_t T, int32_t n_heads, float scale,
                                  void* out, int64_t o_sb, int64_t o_st, int64_t o_sh, void* workspace,
                                  int64_t workspace_bytes, void* stream);
int fs_paged_attention_varlen_reuse_plan(const void* q, int64_t q_st, int64_t q_sh, const fs_kv_layout* kv,
                                         const int32_t* block_tables, int64_t table_stride, int32_t max_blocks,
                                         const int32_t* positions, const int32_t* cu_seqlens, int32_t S,
                                         int32_t T, int32_t n_heads, float scale, void* out, int64_t o_st,
                                         int64_t o_sh, void* workspace, int64_t workspace_bytes, void* stream);

/* ---------------------------------------------------------------------------------------------- */
/* Dense ops of the decoder (model.py)                                                              */
/* ---------------------------------------------------------------------------------------------- */

/* C[M,N] = A[M,K] . B[N,K]^T (+ R[M,N]) in the dtype, f32 accumulation, one rounding of the product
 * and, with R, a second rounding of the sum (nn.Linear then `x + ...`: model.py:77, 93, 105-106,
 * 119-120). Rows may be strided; columns are contiguous. A row of C does not depend on M (the
 * k-order, including any split of K, is a function of N and K only). workspace: at least
 * fs_gemm_workspace_size(M, N, K, dtype) bytes for this call's M, 16-byte aligned, any contents (may
 * be NULL when that size is 0); calls that share a workspace must be ordered on one stream. */
int fs_gemm(const void* A, int64_t lda, const void* B, int64_t ldb, void* C, int64_t ldc, const void* R,
            int64_t ldr, int64_t M, int64_t N, int64_t K, int32_t dtype, void* workspace,
            int64_t workspace_bytes, void* stream);

/* Workspace bytes fs_gemm needs for this M: splits * M * N * 4 for a shape that splits K, except that
 * long batches (fs_gemm_serial) need none. The size therefore does not grow monotonically with M: a
 * caller that keeps one workspace for calls of several M must query each M it uses (or the largest M
 * for which fs_gemm_serial is 0) and keep the largest answer. */
int64_t fs_gemm_workspace_size(int64_t M, int64_t N, int64_t K, int32_t dtype);

/* How many ways fs_gemm splits K for an (N, K) bf16 product (1: not split). A function of N and K only. */
int32_t fs_gemm_splits(int64_t N, int64_t K, int32_t dtype);

/* 1 when fs_gemm runs a split shape's K ranges one after the other inside each workgroup (large M:
 * same arithmetic, same bits, no f32 partials, fs_gemm_workspace_size 0), else 0. Such shapes are
 * cheaper through fs_gemm than through fs_gemm_partials. Internal tuning, no counterpart in the
 * reference. */
int32_t fs_gemm_serial(int64_t M, int64_t N, int64_t K, int32_t dtype);

/* The first half of a split-K fs_gemm: the f32 partial products of each K range, partials[s][M][N]
 * (s = 0 .. fs_gemm_splits(N, K) - 1), each the sum over its K range in increasing k. For consumers
 * that add them themselves (fs_splitk_add_rmsnorm). bf16, K % 64 == 0, N % 4 == 0, only for shapes
 * that split. Replaces the same nn.Linear calls as fs_gemm. */
int fs_gemm_partials(const void* A, int64_t lda, const void* B, int64_t ldb, int64_t M, int64_t N, int64_t K,
                     int32_t dtype, void* partials, int64_t partials_bytes, void* stream);

/* The LM head (model.py:137-138) with the softmax statistics of its logits (sampling.py:13) as a
 * by-product, so that sampling and acceptance need not read the logits back to normalise them.
 * C = A . B^T as fs_gemm (bf16, K % 64 == 0, 16-byte aligned rows, no residual), and for every row m
 * and every column block p of the kernel's tiling, stats[m * stats_ld + p] = {max of y, sum of
 * exp(y - max), max of x, first index of that max} over the block's stored (bf16) values x, with
 * y = x / temperature[m], a true float32 division as in sampling.py:13 (temperature NULL, 1 or 0:
 * y = x; at 0 only the argmax is meaningful). nparts must equal fs_gemm_row_stats_parts(M, N, K)
 * (0: the shape has no such kernel). No counterpart in the reference: it computes
 * softmax(logits.float() / T) from the stored logits. */
int fs_gemm_row_stats(const void* A, int64_t lda, const void* B, int64_t ldb, void* C, int64_t ldc, int64_t M,
                      int64_t N, int64_t K, const float* temperature, void* stats, int64_t stats_ld,
                      int64_t nparts, void* stream);

int64_t fs_gemm_row_stats_parts(int64_t M, int64_t N, int64_t K);

/* The end of a split-K projection fused with the residual add and RMSNorm that follow it
 * (model.py:105-106 then model.py:29-31): x = round(sum of parts[s] in increasing s), then
 * x_out = round(x + residual) and y = rmsnorm(x_out) * weight, exactly as fs_gemm with that residual
 * followed by fs_add_rmsnorm on its output. parts: splits * M * N f32 (fs_gemm_partials). 16-bit
 * dtypes, N % 8 == 0, N <= 8192, 16-byte aligned rows. */
int fs_splitk_add_rmsnorm(const float* parts, int32_t splits, const void* residual, int64_t ldr, void* x_out,
                          int64_t ldxo, const void* weight, void* y, int64_t ldy, int64_t M, int64_t N, float eps,
                          int32_t dtype, void* stream);

/* Merge fs_gemm_row_stats' per-block statistics (row m's nparts records at parts + m * parts_ld)
 * into one record per row, in a fixed order: row m goes to out[(m / group) * gstride + m % group +
 * offset] (records of 16 bytes: max, sum, argmax value, argmax index). With group = K+1,
 * gstride = 2K+1 the target's verify rows land where fs_spec_accept_stats expects them; with the K
 * draft steps' records interleaved per sequence (row b*K + i) and group = K, gstride = 2K+1,
 * offset = K+1 the draft rows do. */
int fs_row_stats_merge(const void* parts, int64_t parts_ld, int64_t nparts, int64_t M, void* out, int32_t group,
                       int64_t gstride, int64_t offset, void* stream);

/* RMSNorm of model.py:29-31, optionally after a residual add (model.py:105-106):
 * if delta != NULL: x_out = x + delta (rounded to the dtype) is written, then normed.
 * y = ((x32 * rsqrt(mean(x32^2) + eps)) rounded to the dtype) * weight, rounded to the dtype. */
int fs_add_rmsnorm(const void* x, int64_t ldx, const void* delta, int64_t ldd, void* x_out, int64_t ldxo,
                   const void* weight, void* y, int64_t ldy, int64_t M, int64_t N, float eps,
                   int32_t dtype, void* stream);

/* SwiGLU gate: h = silu(gu[:, :F]) * gu[:, F:2F], each op rounded to the dtype (model.py:93). */
int fs_silu_mul(const void* gu, int64_t ldgu, void* h, int64_t ldh, int64_t M, int64_t F, int32_t dtype,
                void* stream);

/* The gate|up projection and the SwiGLU gate in one kernel: h = silu(A . B[:F]^T) * (A . B[F:2F]^T)
 * with B the [gate; up] weight (2F rows of K), each product rounded to bf16 as fs_gemm stores it and
 * the gate then as fs_silu_mul computes it; bit-identical to fs_gemm followed by fs_silu_mul, without
 * writing the 2F-wide products. Replaces SwiGLU.forward's w_gate/w_up linears and silu * (model.py:93).
 * bf16, K % 64 == 0, 16-byte aligned rows, F even, and a shape whose GEMM does not split K
 * (fs_gemm_splits(2F, K, bf16) == 1). */
int fs_gemm_swiglu(const void* A, int64_t lda, const void* B, int64_t ldb, void* h, int64_t ldh, int64_t M,
                   int64_t F, int64_t K, int32_t dtype, void* stream);

/* Embedding lookup (model.py:134-135): out[m] = weight[ids[m]]; ids int64. */
int fs_embedding(const int64_t* ids, int64_t M, const void* weight, int64_t d_model, int64_t vocab,
                 void* out, int64_t ldo, int32_t dtype, void* stream);

/* ---------------------------------------------------------------------------------------------- */
/* Sampling and acceptance                                                                          */
/* ---------------------------------------------------------------------------------------------- */

/* probs_from_logits (sampling.py:9-13) for R rows of V: temperature > 0 gives
 * softmax(f32(logits) / temperature) in f32 (out_dtype must be FS_F32); temperature == 0 gives the
 * one-hot of the first argmax in the logits dtype (out_dtype == dtype). */
int fs_probs_from_logits(const void* logits, int64_t ld, int64_t R, int64_t V, float temperature,
                         int32_t dtype, void* out, int64_t ldo, int32_t out_dtype, void* workspace,
                         int64_t workspace_bytes, void* stream);

/* sample (sampling.py:16-21) and the draft draw of speculative.py:61-62, for R rows.
 * Temperature of row r: temperature[r] (device f32 [R]) or, if temperature is NULL, temperature_all.
 * T == 0 -> first argmax of the logits; else argmax_v( p_v / E[r, v] ) with p = softmax(logits / T)
 * (torch.multinomial(p, 1) == argmax(p / Exp(1) noise), first index on ties).
 * E == NULL makes every row take the argmax. tokens_out: int64 [R]; if tokens_out32 is not NULL the
 * tokens are also written there as int32 with stride ld_tok32. */
int fs_sample_logits(const void* logits, int64_t ld, int64_t R, int64_t V, const float* temperature,
                     float temperature_all, const float* E, int64_t ldE, int32_t dtype, int64_t* tokens_out,
                     int32_t* tokens_out32, int64_t ld_tok32, void* workspace, int64_t workspace_bytes,
                     void* stream);

int64_t fs_sampling_workspace_size(int64_t R, int64_t V);

/* Batched speculative acceptance: probs_from_logits + verify_draft (speculative.py:20-33) for B
 * sequences in one stream-ordered call, no host round trip.
 *   tgt: [B, K+1, V] target logits (row (b,i) at tgt + b*tgt_sb + i*tgt_si)
 *   dft: [B, K, V] draft logits (same convention)
 *   draft_tokens int32 [B, K]; k_eff int32 [B] (<= K, proposals of sequence b);
 *   temperature f32 [B]; u f32 [B, K] uniforms; E f32 [B, V] Exp(1) noise for the one final draw.
 * For i < k_eff[b]: ratio = p_i(x_i) / q_i(x_i) if q_i(x_i) > 0 else 1; accept while u[b,i] < min(1, ratio).
 * At the first rejection j the extra token is argmax_v( w_v / E_v ) with w = r / sum(r),
 * r = max(p_j - q_j, 0) (w = p_j if sum(r) == 0); if all are accepted, w = p_{k_eff}.
 * Outputs: out_tokens int32 [B, K+1] (accepted proposals, then the extra token, then -1),
 * n_accepted int32 [B]. If seq_len != NULL it is the device-side rollback: on entry seq_len[b] is
 * the number of cached tokens before the verify window, on exit cached + 1 + n_accepted
 * (speculative.py:77).
 * Probabilities are p_v = exp(x_v/T - M) * (1/S) (x_v/T a true float32 division, M the row's max of
 * x/T, S the sum of exp(x/T - M)): the order torch's softmax forms them (sampling.py:13). One function
 * computes them for the test, the residual and the draws.
 * Optional debug outputs (all three or none, f32): p_x [B, K] and q_x [B, K] receive p_i(x_i) and
 * q_i(x_i) of the proposals the test evaluates (speculative.py:26): the proposals are tested 64 at a
 * time, so every i < min(k_eff, 64), and past 64 the batches of 64 up to the one holding the first
 * rejection; entries of proposals not evaluated, and of proposal ids outside [0, V), are left
 * untouched. res_sum [B] the sum of the residual max(p_j - q_j, 0) at the first rejection j
 * (speculative.py:30), 0 when every proposal was accepted or the row is greedy. They let a caller
 * measure how near a decision was to a tie.
 * The call is four kernel launches (statistics, steps, chunks of the draws, draws; three with the
 * statistics given) that pass records through the workspace; each launch reads only what an earlier
 * one of the same call wrote, so the workspace needs no initial contents. Calls that share a
 * workspace must not overlap (order them on one stream). */
int fs_spec_accept(const void* tgt, int64_t tgt_sb, int64_t tgt_si, const void* dft, int64_t dft_sb,
                   int64_t dft_si, int32_t B, int32_t K, int64_t V, int32_t dtype, const int32_t* draft_tokens,
                   const int32_t* k_eff, const float* temperature, const float* u, const float* E,
                   int64_t ldE, int32_t* out_tokens, int32_t* n_accepted, int32_t* seq_len, float* p_x,
                   float* q_x, float* res_sum, void* workspace, int64_t workspace_bytes, void* stream);

/* fs_spec_accept with the rows' softmax statistics given (row_stats: [B][2K+1] records of
 * fs_row_stats_merge at the rows' temperatures, target rows 0..K then draft rows; 16-byte aligned): the
 * vocab-wide statistics pass is skipped. Replaces the same seam as fs_spec_accept (speculative.py:20-33
 * with probs_from_logits), for callers whose LM head produced the statistics (fs_gemm_row_stats). */
int fs_spec_accept_stats(const void* tgt, int64_t tgt_sb, int64_t tgt_si, const void* dft, int64_t dft_sb,
                         int64_t dft_si, int32_t B, int32_t K, int64_t V, int32_t dtype, const int32_t* draft_tokens,
                         const int32_t* k_eff, const float* temperature, const float* u, const float* E,
                         int64_t ldE, const void* row_stats, int32_t* out_tokens, int32_t* n_accepted,
                         int32_t* seq_len, float* p_x, float* q_x, float* res_sum, void* workspace,
                         int64_t workspace_bytes, void* stream);

/* fs_spec_accept (row_stats NULL) or fs_spec_accept_stats (row_stats given) without a workspace
 * argument and without any allocation: the scratch is a fixed 4 MiB device array of the library, one
 * per GPU, held until the process ends (its address is looked up once per device, on that device's
 * first call). No counterpart in the reference; it is for callers that cannot allocate device memory
 * (code under HIP graph capture, serving loops and harnesses that forbid allocation). Shapes whose
 * scratch exceeds 4 MiB (fs_spec_accept_workspace_size(B, K, V) > 4 MiB; batch 512 with k = 8 and a
 * 128256-token vocabulary fits) are refused with FS_ERR_ARG before anything is launched. Every call on
 * one GPU shares that GPU's scratch, so calls that overlap on one device (different streams, or host
 * threads) race; calls ordered on one stream do not. No debug outputs. The first call on a device
 * looks the array up (a host API call); it must not be made while `stream` is being captured into a
 * HIP graph (it then fails with FS_ERR_ARG): make one call before capturing. */
int fs_spec_accept_noalloc(const void* tgt, int64_t tgt_sb, int64_t tgt_si, const void* dft, int64_t dft_sb,
                           int64_t dft_si, int32_t B, int32_t K, int64_t V, int32_t dtype, const int32_t* draft_tokens,
                           const int32_t* k_eff, const float* temperature, const float* u, const float* E,
                           int64_t ldE, const void* row_stats, int32_t* out_tokens, int32_t* n_accepted,
                           int32_t* seq_len, void* stream);

/* The round-to-round bookkeeping of speculative.py:71-85 (emit the accepted tokens and the extra,
 * advance the cache length, stop at the token limit) for B rows at once, on the device, so that the
 * next round can be queued before the host has read this round's tokens. res: the acceptance's
 * [B, res_ld] int32 rows (n_accepted a, then a+1 committed tokens). Per row: n += a+1, budget -= a+1
 * (budget = min(max_new - generated, max_seq_len - n)), done once budget <= 0 or a committed token
 * equals eos[row] (-1: none); then the next round's inputs as a host would stage them: ids [B,2]
 * (prev, last) int64, last [B] int64, k_eff [B] = min(k, budget-1), pos0 [B,2], posd [k-first, B]
 * (draft step i at n-1+i while i < k_eff), posv [B, k+1] (n-1+t for t <= k_eff); done rows get
 * k_eff 0 and -1 positions. first: 1 when draft step 0 feeds the (prev, last) pair at pos0, 0 when
 * it feeds `last` alone (a draft on the target's cache). */
int fs_spec_advance(const int32_t* res, int64_t res_ld, int32_t B, int32_t k, int32_t first, int32_t* n,
                    int32_t* budget, const int32_t* eos, int32_t* done, int64_t* ids, int64_t* last, int32_t* keff,
                    int32_t* pos0, int32_t* posd, int32_t* posv, void* stream);

/* verify_draft (speculative.py:20-33) on probabilities instead of logits: p [K+1, V] rows at
 * p + i*ldp, q [K, V]; one sequence, K proposals; p and q in `dtype` (f32 from a softmax, or the
 * logits dtype for one-hot rows). Same outputs as fs_spec_accept with B = 1. */
int fs_verify_probs(const void* p, int64_t ldp, const void* q, int64_t ldq, int32_t K, int64_t V,
                    int32_t dtype, const int32_t* draft_tokens, const float* u, const float* E,
                    int32_t* out_tokens, int32_t* n_accepted, void* workspace, int64_t workspace_bytes,
                    void* stream);

/* Workspace of fs_spec_accept / fs_verify_probs (256-byte aligned, any contents). */
int64_t fs_spec_accept_workspace_size(int32_t B, int32_t K, int64_t V);

/* ---------------------------------------------------------------------------------------------- */
/* Keyed random numbers                                                                             */
/* ---------------------------------------------------------------------------------------------- */
#define FS_RNG_UNIFORM 0
#define FS_RNG_EXP 1

/* Per-request random streams for batched speculation in the Engine (engine.py:41, 126-133 draw
 * from one shared generator in running-row order instead; this replaces those draws for the
 * speculative engine, the per-request RNG keyed by (request, position) of the batched Engine).
 * out[s*ld_slot + b*ld_row + j] for s < n_slots, b < B, j < n is the variate of (keys[b],
 * slot0 + s, j): Philox4x32-10 with key keys[b] and counter (j/2, slot, 0, 0); kind FS_RNG_UNIFORM:
 * u = (w >> 8) * 2^-24 in [0, 1) (torch.rand's float32 grid, speculative.py:27); FS_RNG_EXP: Exp(1)
 * E = -log1p(-t), t uniform in (0, 1) with 2^-23 relative resolution down to 2^-33, never 0 (the
 * noise of multinomial as argmax(w / E), sampling.py:21, speculative.py:32-33, 62). At most 65535
 * rows x slots per call. */
int fs_keyed_noise(const uint64_t* keys, int32_t B, int32_t slot0, int32_t n_slots, int64_t n, int32_t kind,
                   float* out, int64_t ld_row, int64_t ld_slot, void* stream);

#ifdef __cplusplus
}
#endif

#endif /* FORGESERVE_AMD_H */
