/*
 * mla.h -- C ABI of libmla_amd.so, the MI355X (gfx950) absorbed-MLA layer.
 *
 * The library replaces the reference's CUDA extension (pgangwar-ucsd/mla-cuda,
 * mla_kernels.cu).  Its two fused entry points are the reference's pybind surface
 * (mla_kernels.cu:1688-1693); the per-step entry points expose each of the nine kernels
 * of that file on its own, so each step can be checked and profiled alone.
 *
 * Conventions shared by every entry point
 *   - All tensor arguments are DEVICE pointers to dense row-major storage with the shapes
 *     given in the comments; every pointer must be 16-byte aligned.
 *   - `dtype` names the storage type of the layer's inputs and outputs.  Intermediates that
 *     the reference keeps in its accumulate dtype (mla_kernels.cu:115-120) are float32
 *     here ("acc" below): q_lat_acc, q_raw, scores, m/l/alpha, row_sum, ctx -- float64
 *     under MLA_DTYPE_F64, which the two fused entry points (and their ragged and
 *     no-workspace variants) take; every other entry point refuses it with
 *     MLA_ERR_UNSUPPORTED.
 *   - Work is enqueued on `stream` (NULL = the null stream); no entry point synchronises
 *     the host, none allocates device memory.  Scratch memory comes from the caller through
 *     `workspace` / `workspace_bytes`, sized by the matching *_workspace_bytes() query.
 *   - Return value: MLA_OK, or an mla_status_t error code with a message available from
 *     mla_last_error() on the calling thread.  Arguments are validated before any HIP call,
 *     so a rejected call has no side effect on the device.
 *   - Calls that share a workspace must be ordered on one stream.
 */
#ifndef MLA_AMD_MLA_H_
#define MLA_AMD_MLA_H_

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* The HIP runtime's own stream handle type (hip_runtime_api.h declares the same). */
typedef struct ihipStream_t* hipStream_t;

typedef enum mla_dtype {
    MLA_DTYPE_F32 = 0,   /* float32 storage, float32 MFMA (v_mfma_f32_32x32x2_f32)       */
    MLA_DTYPE_BF16 = 1,  /* bfloat16 storage, float32 accumulation on bf16 MFMA          */
    MLA_DTYPE_F16 = 2,   /* float16 storage, float32 accumulation on fp16 MFMA            */
    MLA_DTYPE_F64 = 3,   /* float64 storage and intermediates, double MFMA
                            (v_mfma_f64_16x16x4_f64): the reference's double dispatch,
                            mla_kernels.cu:674, 1561.  mla_q_absorbed(_ragged) and
                            mla_attention(_noalloc) only                                 */
} mla_dtype_t;

typedef enum mla_status {
    MLA_OK = 0,
    MLA_ERR_INVALID_ARGUMENT = 1,  /* shape, pointer, alignment or value out of range   */
    MLA_ERR_UNSUPPORTED = 2,       /* valid request this build does not implement       */
    MLA_ERR_WORKSPACE = 3,         /* workspace missing or smaller than the query says  */
    MLA_ERR_HIP = 4,               /* a HIP runtime call or kernel launch failed        */
} mla_status_t;

/* Layer dimensions.  Reference values (DeepSeek-V3, exhaustive_benchmark_suite.py:30-49):
 * hidden 7168, q_lora 1536, heads 128, nope 128, rope 64, kv_rank 512, v 128. */
typedef struct mla_dims {
    int32_t batch;    /* B                                   */
    int32_t sq;       /* query tokens per sequence           */
    int32_t sk;       /* cached keys per sequence            */
    int32_t hidden;   /* model width                         */
    int32_t q_lora;   /* Q latent rank                       */
    int32_t heads;    /* H                                   */
    int32_t nope;     /* per-head non-rotary q/k width       */
    int32_t rope;     /* per-head rotary width (even)        */
    int32_t kv_rank;  /* latent cache width R                */
    int32_t v;        /* per-head value width                */
} mla_dims_t;

/* Thread-local message describing the most recent failed call ("" if none). */
const char* mla_last_error(void);
/* Library version string. */
const char* mla_version(void);
/* Keys covered by one softmax partial of the scores step (128): the m/l/alpha row length
 * is ceil(sk / mla_score_tile()). */
int32_t mla_score_tile(void);
/* Row stride, in elements, of the `scores` buffer for a given sk (sk rounded up to 32). */
int32_t mla_score_ld(int32_t sk);

/* ======================================================================================
 * Fused entry points -- the reference's boundary
 * ==================================================================================== */

/* Q path, steps 2a1 -> 2a-n -> 2a2 -> 2b -> 2c.
 * Replaces mla_custom_cuda.q_absorbed / launch_q_absorbed (mla_kernels.cu:599-767).
 *   x          [B, Sq, hidden]                 dtype
 *   W_q_a      [hidden, q_lora]                dtype
 *   q_norm_w   [q_lora]                        dtype  RMSNorm gain
 *   W_q_b      [q_lora, H*(nope+rope)]         dtype
 *   W_uk       [H, nope, kv_rank]              dtype
 *   positions  [Sq]                            int64  absolute position of each query
 *   inv_freq   [rope/2]                        RoPE inverse frequencies 1/10000^(2i/rope),
 *                                              computed by the caller in float32 (float64
 *                                              under MLA_DTYPE_F64), the accumulate dtype
 *                                              the reference evaluates them in
 *   q_absorbed [B, Sq, H, kv_rank]             dtype  (out)
 *   q_rope     [B, Sq, H, rope]                dtype  (out)
 */
size_t mla_q_absorbed_workspace_bytes(mla_dtype_t dtype, const mla_dims_t* dims);
int mla_q_absorbed(mla_dtype_t dtype, const mla_dims_t* dims,
                   const void* x, const void* W_q_a, const void* q_norm_w,
                   const void* W_q_b, const void* W_uk, const int64_t* positions,
                   const void* inv_freq, double eps,
                   void* q_absorbed, void* q_rope,
                   void* workspace, size_t workspace_bytes, hipStream_t stream);

/* Attention, steps 3a -> 3b -> 3c -> 3d.
 * Replaces mla_custom_cuda.mla_attention / launch_mla_attention (mla_kernels.cu:1479-1682).
 *   q_absorbed [B, Sq, H, kv_rank], q_rope [B, Sq, H, rope]          dtype
 *   c_kv       [B, Sk, kv_rank],    pe_cache [B, Sk, rope]           dtype
 *   W_uv       [H, v, kv_rank]                                      dtype
 *   out        [B, Sq, H, v]                                        dtype (out)
 *   scale      softmax DIVISOR (the reference passes sqrt(nope+rope))
 *   causal     0: every key visible; 1: key j visible to query i iff j <= Sk - Sq + i
 *              (not in the reference; used for chunked prefill)
 * At kv_rank 512 / rope 64 this runs 3a+3b+3c as one fused pass (mla_attn_ctx), whose
 * workspace holds no score matrix; MLA_ATTENTION_PATH=split selects the per-step kernels.
 * Under MLA_DTYPE_F64 it runs the reference's decomposition in double (scores
 * [B*Sq*H, Sk] in the workspace, a row softmax, ctx, then 3d).
 * The variable is read by the size query and by the call: a caller that changes it in
 * between gets MLA_ERR_WORKSPACE when the workspace is too small.
 */
size_t mla_attention_workspace_bytes(mla_dtype_t dtype, const mla_dims_t* dims, int causal);
int mla_attention(mla_dtype_t dtype, const mla_dims_t* dims,
                  const void* q_absorbed, const void* q_rope, const void* c_kv,
                  const void* pe_cache, const void* W_uv, double scale, int causal,
                  void* out, void* workspace, size_t workspace_bytes, hipStream_t stream);

/* mla_attention without a workspace argument, for callers that cannot allocate device
 * memory (code under HIP graph capture, tight serving loops, harnesses that forbid
 * allocation).  No counterpart in the reference.  The scratch memory is a fixed device array
 * of the library, MLA_ATTENTION_NOALLOC_MAX_BYTES (64 MiB) per GPU, held from the library's
 * load until the process ends: it covers decode (Sq = 1) at B <= 128 for any Sk.
 * A shape whose mla_attention_workspace_bytes() exceeds it is rejected with
 * MLA_ERR_WORKSPACE.  The call allocates nothing and runs the same kernels as mla_attention
 * (same results, bit for bit).  All calls on one GPU share the array: calls that overlap on
 * one GPU (several streams or host threads) race and must be serialised by the caller. */
#define MLA_ATTENTION_NOALLOC_MAX_BYTES ((size_t)64 << 20)
int mla_attention_noalloc(mla_dtype_t dtype, const mla_dims_t* dims,
                          const void* q_absorbed, const void* q_rope, const void* c_kv,
                          const void* pe_cache, const void* W_uv, double scale, int causal,
                          void* out, hipStream_t stream);

/* Attention over an fp8 KV cache (the cache-format row of the hot path's next steps; the
 * reference keeps the cache in the query dtype, mla_kernels.cu:1489, 847-848).
 *   c_kv_fp8 [B, Sk, kv_rank], pe_fp8 [B, Sk, rope]   uint8: OCP float8 e4m3 codes
 *            (torch.float8_e4m3fn) of value / kv_scale, one scale for both
 *   q_absorbed, q_rope, W_uv, out                    bf16 (dtype must be MLA_DTYPE_BF16)
 * Result: mla_attention on the decoded cache (code * kv_scale), at bf16 accuracy.  The fused
 * pass decodes the rows in LDS (e4m3 -> bf16 is exact) and applies kv_scale to the scores and
 * the output.  kv_rank 512 and rope 64 only (MLA_ERR_UNSUPPORTED otherwise); the cache moves
 * half the bytes of a bf16 cache. */
size_t mla_attention_fp8kv_workspace_bytes(mla_dtype_t dtype, const mla_dims_t* dims,
                                           int causal);
int mla_attention_fp8kv(mla_dtype_t dtype, const mla_dims_t* dims, const void* q_absorbed,
                        const void* q_rope, const void* c_kv_fp8, const void* pe_fp8,
                        float kv_scale, const void* W_uv, double scale, int causal, void* out,
                        void* workspace, size_t workspace_bytes, hipStream_t stream);
/* The fp8 cache's decoder on its own: out[i] = e4m3 code[i] * scale (float32), through the
 * same conversion the attention uses. */
int mla_fp8_dequantize(const void* codes, int64_t n, float scale, float* out, hipStream_t stream);

/* Attention over a long key range without materialising the [B*Sq*H, Sk] score matrix:
 * keys are processed in chunks of `key_chunk` (a multiple of mla_score_tile(); 0 = choose
 * so the per-chunk score buffer stays <= 1 GiB).  Each chunk runs 3a -> 3b -> 3c into a
 * bounded buffer and is merged into running (max, sum, unnormalised ctx) state with the
 * online-softmax rescale; 3d runs once at the end.  Same arguments and result as
 * mla_attention (not in the reference, which always materialises the scores,
 * mla_kernels.cu:1526-1529; at B=4, Sq=128, Sk=32768 that matrix alone is 8.6 GB). */
size_t mla_attention_streaming_workspace_bytes(mla_dtype_t dtype, const mla_dims_t* dims,
                                               int causal, int32_t key_chunk);
int mla_attention_streaming(mla_dtype_t dtype, const mla_dims_t* dims,
                            const void* q_absorbed, const void* q_rope, const void* c_kv,
                            const void* pe_cache, const void* W_uv, double scale, int causal,
                            int32_t key_chunk, void* out, void* workspace,
                            size_t workspace_bytes, hipStream_t stream);

/* ======================================================================================
 * Per-step entry points (no reference counterpart: the reference fuses them behind the
 * two calls above).  dims fields a step does not use are ignored.
 * ==================================================================================== */

/* 2a1 / 2a2: C[M, N] (float32) = A[M, K] @ W[K, N]; A and W in dtype.
 * The reference's q_raw_gemm_kernel (mla_kernels.cu:233-366). */
size_t mla_gemm_workspace_bytes(mla_dtype_t dtype, int32_t M, int32_t N, int32_t K);
int mla_gemm(mla_dtype_t dtype, const void* A, const void* W, float* C,
             int32_t M, int32_t N, int32_t K,
             void* workspace, size_t workspace_bytes, hipStream_t stream);

/* 2a-n: out[M, N] (dtype) = in[M, N] * rsqrt(mean(in^2) + eps) * gain[N];
 * in float32, gain dtype.  The reference's q_lat_norm_kernel (mla_kernels.cu:377-420). */
int mla_rmsnorm(mla_dtype_t dtype, const float* in, const void* gain, void* out,
                int32_t M, int32_t N, double eps, hipStream_t stream);

/* 2b: q_rope[B, Sq, H, rope] (dtype) = RoPE of q_raw[b*Sq+s, h*(nope+rope)+nope : +rope]
 * (q_raw float32 [B*Sq, H*(nope+rope)]) at positions[s].
 * The reference's q_rope_kernel (mla_kernels.cu:425-466). */
int mla_rope(mla_dtype_t dtype, const mla_dims_t* dims, const float* q_raw,
             const int64_t* positions, const float* inv_freq, void* q_rope,
             hipStream_t stream);

/* 2c: q_absorbed[b, s, h, :] (dtype) = q_raw[b*Sq+s, h*(nope+rope) : +nope] @ W_uk[h].
 * The reference's q_absorb_kernel (mla_kernels.cu:474-596). */
int mla_absorb(mla_dtype_t dtype, const mla_dims_t* dims, const float* q_raw,
               const void* W_uk, void* q_absorbed, hipStream_t stream);

/* 3a: for every row f = (b*Sq + s)*H + h and key k < Sk:
 *   t = (q_absorbed[f]·c_kv[b,k] + q_rope[f]·pe_cache[b,k]) / scale
 * and for each block j of mla_score_tile() keys: m_part[f, j] = max of t over the block's
 * visible keys, scores[f, k] = exp(t - m_part[f, j]) (0 where masked or k >= Sk, up to
 * ld_scores), l_part[f, j] = sum of scores over the block.  scores float32
 * [B*Sq*H, ld_scores] with ld_scores >= mla_score_ld(Sk); m_part, l_part float32
 * [B*Sq*H, ceil(Sk/tile)].  The reference's mla_scores_kernel (mla_kernels.cu:808-1033). */
int mla_scores(mla_dtype_t dtype, const mla_dims_t* dims,
               const void* q_absorbed, const void* q_rope, const void* c_kv,
               const void* pe_cache, double scale, int causal,
               float* scores, int32_t ld_scores, float* m_part, float* l_part,
               hipStream_t stream);

/* 3b: per row: M = max_j m_part[row, j]; alpha[row, j] = exp(m_part[row, j] - M)
 * (exactly 1 where equal); row_sum[row] = sum_j l_part[row, j] * alpha[row, j].
 * All float32.  The reference's mla_combine_kernel (mla_kernels.cu:1036-1081). */
int mla_combine(const float* m_part, const float* l_part, float* alpha, float* row_sum,
                int32_t rows, int32_t n_partials, hipStream_t stream);

/* 3c: ctx[b, s, h, :] (float32) = sum_k scores[f, k] * alpha[f, k / tile] * c_kv[b, k, :]
 * -- the unnormalised attention numerator.  scores/alpha float32, c_kv dtype.
 * The reference's mla_ctx_kernel (mla_kernels.cu:1088-1326). */
size_t mla_ctx_workspace_bytes(mla_dtype_t dtype, const mla_dims_t* dims);
int mla_ctx(mla_dtype_t dtype, const mla_dims_t* dims, const float* scores,
            int32_t ld_scores, const float* alpha, const void* c_kv, float* ctx,
            void* workspace, size_t workspace_bytes, hipStream_t stream);

/* 3a + 3b + 3c as one pass over the cache (16-bit or float32 with kv_rank = 512 and
 * rope = 64 only; MLA_ERR_UNSUPPORTED otherwise): ctx [B*Sq*H, kv_rank] and row_sum
 * [B*Sq*H], float32, such that ctx[f] / row_sum[f] = sum_k softmax_k(t[f, :]) c_kv[b, k]
 * -- what mla_ctx and mla_combine produce, up to one positive factor per row shared by
 * ctx[f] and row_sum[f] (the kernels keep their own per-row reference maximum).
 * mla_attention runs this at those widths.
 * Fuses the reference's mla_scores_kernel, mla_combine_kernel and mla_ctx_kernel
 * (mla_kernels.cu:808-1326). */
size_t mla_attn_ctx_workspace_bytes(mla_dtype_t dtype, const mla_dims_t* dims, int causal);
int mla_attn_ctx(mla_dtype_t dtype, const mla_dims_t* dims, const void* q_absorbed,
                 const void* q_rope, const void* c_kv, const void* pe_cache, double scale,
                 int causal, float* ctx, float* row_sum, void* workspace,
                 size_t workspace_bytes, hipStream_t stream);

/* 3d: out[b, s, h, :] (dtype) = (ctx[b, s, h, :] / row_sum[f]) @ W_uv[h]^T;
 * ctx/row_sum float32, W_uv dtype [H, v, kv_rank].
 * The reference's mla_output_smem_kernel (mla_kernels.cu:1339-1476). */
size_t mla_out_workspace_bytes(mla_dtype_t dtype, const mla_dims_t* dims);
int mla_out(mla_dtype_t dtype, const mla_dims_t* dims, const float* ctx,
            const float* row_sum, const void* W_uv, void* out,
            void* workspace, size_t workspace_bytes, hipStream_t stream);

/* ======================================================================================
 * Neighbours of the path: the caller's weight prep before it, the KV-cache write beside
 * it, and the output projection after it.  None is in the reference; the reference names
 * the weight split its callers repeat per call (exhaustive_benchmark_suite.py:261-265,
 * 320, 334) and wkv_a's cache write (exhaustive_benchmark_suite.py:188-196).
 * ==================================================================================== */

/* Weight prep, once at load: split wkv_b [H, nope + v, kv_rank] into contiguous
 * W_uk [H, nope, kv_rank] = wkv_b[:, :nope, :] and W_uv [H, v, kv_rank] = wkv_b[:, nope:, :]
 * (the copies the reference's callers make with .contiguous() on every call).  Uses
 * dims->heads, nope, v, kv_rank.  Bit-exact copy. */
int mla_split_wkv_b(mla_dtype_t dtype, const mla_dims_t* dims, const void* wkv_b,
                    void* W_uk, void* W_uv, hipStream_t stream);

/* KV-cache append for dims->sq new tokens of each of dims->batch sequences, as DeepSeek-V3
 * writes its absorbed-layout cache (deepseek-ai/DeepSeek-V3 inference/model.py, MLA.forward):
 *   kv = x @ W_kv_a                                  x [B, Sq, hidden], W_kv_a [hidden, kv_rank + rope]
 *   c_kv[b, start_row + s, :]     = RMSNorm(kv[b, s, :kv_rank]) * kv_norm_w     (eps)
 *   pe_cache[b, start_row + s, :] = RoPE(kv[b, s, kv_rank:], positions[s])       (interleaved pairs)
 * with the same RMSNorm and RoPE arithmetic as mla_q_absorbed (inv_freq as there).
 * c_kv [B, cache_rows, kv_rank] and pe_cache [B, cache_rows, rope] are updated in place;
 * rows outside [start_row, start_row + Sq) are untouched.  start_row + Sq <= cache_rows. */
size_t mla_kv_append_workspace_bytes(mla_dtype_t dtype, const mla_dims_t* dims);
int mla_kv_append(mla_dtype_t dtype, const mla_dims_t* dims, const void* x, const void* W_kv_a,
                  const void* kv_norm_w, const int64_t* positions, const float* inv_freq,
                  double eps, int32_t start_row, int32_t cache_rows, void* c_kv,
                  void* pe_cache, void* workspace, size_t workspace_bytes,
                  hipStream_t stream);

/* ---- Ragged, paged KV cache (the reference has one dense [B, Sk, kv_rank] cache with one
 * Sk for the whole batch and query positions shared by the batch, mla_kernels.cu:1489,
 * 847-848, 449).  Keys live in a pool of pages:
 *   c_kv_pages [num_pages, page_size, kv_rank], pe_pages [num_pages, page_size, rope]
 *   block_table [B, max_pages] int32: sequence b's keys [j*page_size, (j+1)*page_size)
 *               are page block_table[b*max_pages + j] of the pool
 *   seq_lens    [B] int32: keys of sequence b, clamped to [0, max_pages*page_size]; a
 *               sequence without keys (or, with causal, a query that sees none) gives
 *               zero output rows, as a softmax over no keys does in the reference's
 *               formulation
 * page_size is a multiple of 64; dims->sk = max_pages * page_size (the table's key span).
 * Both tables are device memory, read by the kernels (no host synchronisation). */

/* mla_q_absorbed with per-sequence positions: positions [B, Sq] (int64, row b = sequence b's
 * absolute query positions) instead of one [Sq] row shared by the batch.  Same workspace as
 * mla_q_absorbed. */
int mla_q_absorbed_ragged(mla_dtype_t dtype, const mla_dims_t* dims, const void* x,
                          const void* W_q_a, const void* q_norm_w, const void* W_q_b,
                          const void* W_uk, const int64_t* positions, const void* inv_freq,
                          double eps, void* q_absorbed, void* q_rope, void* workspace,
                          size_t workspace_bytes, hipStream_t stream);

/* Attention over the paged cache: sequence b attends to its first seq_lens[b] keys; with
 * causal, key j is visible to query i iff j <= seq_lens[b] - Sq + i (seq_lens[b] >= Sq).
 * Same queries, W_uv, scale and output as mla_attention, and like it the fused 3a+3b+3c
 * pass at kv_rank 512 / rope 64 (MLA_ATTENTION_PATH=split: the per-step kernels).  The
 * fused pass cuts the sequences into key chunks from a work list it builds on the device
 * from seq_lens (the total key count spread over the CUs; equal lengths take the dense
 * split), so the workspace is larger than mla_attention's by the list and its partial
 * slots. */
size_t mla_attention_paged_workspace_bytes(mla_dtype_t dtype, const mla_dims_t* dims,
                                           int causal, int32_t page_size);
int mla_attention_paged(mla_dtype_t dtype, const mla_dims_t* dims, const void* q_absorbed,
                        const void* q_rope, const void* c_kv_pages, const void* pe_pages,
                        const int32_t* block_table, const int32_t* seq_lens, int32_t page_size,
                        const void* W_uv, double scale, int causal, void* out, void* workspace,
                        size_t workspace_bytes, hipStream_t stream);

/* Attention over a paged fp8 cache: mla_attention_paged's pools, block table, seq_lens and
 * causal rule, with the pools holding mla_attention_fp8kv's e4m3 codes.  It combines two
 * cache formats that the reference has neither of (one dense cache in the query dtype,
 * mla_kernels.cu:1489, 847-848).
 *   c_kv_pages_fp8 [num_pages, page_size, kv_rank], pe_pages_fp8 [.., rope]   uint8 codes
 *                  of value / kv_scale, one scale for both pools
 *   q_absorbed, q_rope, W_uv, out                                          bf16
 * dtype must be MLA_DTYPE_BF16; kv_rank 512 and rope 64 only; page_size a positive multiple
 * of 64 and dims->sk = max_pages * page_size.  The fused pass runs on the work list that
 * mla_attention_paged builds. */
size_t mla_attention_paged_fp8kv_workspace_bytes(mla_dtype_t dtype, const mla_dims_t* dims,
                                                 int causal, int32_t page_size);
int mla_attention_paged_fp8kv(mla_dtype_t dtype, const mla_dims_t* dims, const void* q_absorbed,
                              const void* q_rope, const void* c_kv_pages_fp8,
                              const void* pe_pages_fp8, const int32_t* block_table,
                              const int32_t* seq_lens, int32_t page_size, float kv_scale,
                              const void* W_uv, double scale, int causal, void* out,
                              void* workspace, size_t workspace_bytes, hipStream_t stream);

/* The work list that mla_attention_paged's fused pass builds on the device from seq_lens,
 * written to `work_list` for inspection (a per-step view of that kernel; no reference
 * counterpart).  int32 layout: [0] item count, [1] keys per chunk, first partial slot [B],
 * chunk count [B], then the items {b, c} (chunk c of sequence b covers keys [c*chunk,
 * min((c+1)*chunk, seq_lens[b]))): the full-length chunks first, then the shorter last
 * chunks, longest first.  Uses dims->batch, sq, heads and sk (= max_pages * page_size);
 * dtype selects the key block (16 keys for float32, 32 for bf16 and float16).
 * mla_attention_work_list_ints() gives the list's length in ints (0 if dims are invalid). */
int32_t mla_attention_work_list_ints(mla_dtype_t dtype, const mla_dims_t* dims);
int mla_attention_work_list(mla_dtype_t dtype, const mla_dims_t* dims, const int32_t* seq_lens,
                            int32_t* work_list, int32_t ints, hipStream_t stream);

/* KV-cache append into the paged cache: as mla_kv_append, but token (b, s) is written to
 * logical slot positions[b*Sq + s] of sequence b (positions [B, Sq], int64): pool row
 * block_table[b*max_pages + slot/page_size]*page_size + slot%page_size.  Slots outside
 * [0, max_pages*page_size) are skipped.  Uses dims->batch, sq, hidden, kv_rank, rope, sk
 * (= max_pages * page_size).  Same workspace as mla_kv_append. */
int mla_kv_append_paged(mla_dtype_t dtype, const mla_dims_t* dims, const void* x,
                        const void* W_kv_a, const void* kv_norm_w, const int64_t* positions,
                        const float* inv_freq, double eps, const int32_t* block_table,
                        int32_t page_size, void* c_kv_pages, void* pe_pages, void* workspace,
                        size_t workspace_bytes, hipStream_t stream);

/* Output projection wo: out [B*Sq, hidden] = attn [B*Sq, H*v] @ W_o [H*v, hidden], all in
 * dtype (fp32 accumulation).  attn is mla_attention's output [B, Sq, H, v]. */
size_t mla_o_proj_workspace_bytes(mla_dtype_t dtype, const mla_dims_t* dims);
int mla_o_proj(mla_dtype_t dtype, const mla_dims_t* dims, const void* attn, const void* W_o,
               void* out, void* workspace, size_t workspace_bytes, hipStream_t stream);

#ifdef __cplusplus
}  /* extern "C" */
#endif

#endif  /* MLA_AMD_MLA_H_ */
