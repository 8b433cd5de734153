// Host-side launch interface of the gfx950 kernels (internal to libmla_amd.so).
// Every launcher assumes its arguments were validated by the C ABI layer (abi.cpp).
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

namespace mla {

// ---------------------------------------------------------------- batched MFMA GEMM
// C[g][m][n] = sum_k opA(A)[g][m][k] * opB(B)[g][k][n]   (fp32 accumulate; fp32, bf16 or
// fp16 MFMA as GemmProblem::half / f16 say)
//   A[g][m][k]  at A + g*sAg + m*lda + k
//   B (NN)      at B + g*sBg + k*ldb + n      B (NT) at B + g*sBg + n*ldb + k
//   C[g][m][n]  at C + g*sCg + m*ldc + n
// A modes: kAPlain; kARowRecip (row m of batch g scaled by 1/rs[m*rs_m + g*rs_g]);
//          kAAlpha (A[g][m][k] scaled by alpha[(g*M + m)*alpha_ld + k/alpha_tile]).
enum AMode { kAPlain = 0, kARowRecip = 1, kAAlpha = 2 };
enum OutType { kOutF32 = 0, kOutBF16 = 1, kOutF16 = 2 };   // the codes Store16<> takes

// 2a2's fused epilogue (16-bit weight-streaming plans with split 1 only): instead of the
// fp32 product C [M, H*(nope+rope)], the nope columns of every head go to q_nope
// [M, H, nope] and the rope columns, rotated, to q_rope [M, H, rope], both rounded once to
// the storage format -- the rounding 2c and 2b apply to the same fp32 values.  The rotation
// of row m, pair i takes cos_sin[2 (m * rope/2 + i)] and the sin after it, the table the
// 2a-n launch writes (RopeTable).  nope and rope are multiples of 32, rope <= 64.
// With w_uk set the epilogue also does 2c: each head's 16-bit q_nope tile stays in LDS and
// is multiplied by W_uk[h] ([H, nope, kv] contiguous) into q_abs [M, H, kv] (storage
// format), and q_nope is not written.  That needs the 128 x 4 plan, nope = 128, rope = 64,
// an even H and kv a multiple of 128 up to 512 (qup_supported).
struct QUpEpilogue {
    void* q_nope = nullptr;
    void* q_rope = nullptr;
    const float* cos_sin = nullptr;
    int H = 0, nope = 0, rope = 0;
    const void* w_uk = nullptr;
    void* q_abs = nullptr;
    int kv = 0;
};

// Optional output of the 2a-n launch for that epilogue: row m's cos and sin of the angles
// pos(m) * inv_freq[i], i < half, with pos(m) = positions[m] (per_batch) or
// positions[m % Sq] -- the angles and the sincosf of 2b.
struct RopeTable {
    float* cos_sin = nullptr;
    const int64_t* positions = nullptr;
    const float* inv_freq = nullptr;
    int half = 0, Sq = 1;
    bool per_batch = false;
};

struct GemmProblem {
    const void* A = nullptr; int64_t lda = 0, sAg = 0;
    const void* B = nullptr; int64_t ldb = 0, sBg = 0;
    void* C = nullptr;        int64_t ldc = 0, sCg = 0;
    int M = 0, N = 0, K = 0, G = 1;
    bool b_nt = false;
    bool half = false;   // B (weights / cache) and the MFMA are 16-bit (else fp32)
    bool f16 = false;    // the 16-bit format is fp16 (else bfloat16)
    bool a_f32 = true;   // A is fp32 in global memory (else the storage dtype)
    AMode amode = kAPlain;
    const float* rs = nullptr; int64_t rs_m = 0, rs_g = 0;
    const float* alpha = nullptr; int alpha_ld = 0, alpha_tile = 1;
    OutType out_type = kOutF32;
    // optional: per-group K limit k_len[g] (<= K), and a paged NN B operand -- K row k of
    // group g is pool row b_pages[g*max_pages + k/page_size]*page_size + k%page_size of B
    // (sBg unused; page_size a multiple of 64; only the alpha-scaled NN form)
    const int* k_len = nullptr;
    const int* b_pages = nullptr;
    int page_size = 0, max_pages = 0;
    const QUpEpilogue* qup = nullptr;   // weight-streaming plans only (launch_wgemm)
    // fp32 tiled plans with one K split: 2b in 2a2's epilogue (q_rope, cos_sin, H, nope,
    // rope of the struct; the nope columns still go to C)
    const QUpEpilogue* rope_epi = nullptr;
};

// Tile/split plan chosen for a problem (pure function of the shape; see plan_gemm).
struct GemmPlan {
    int bm = 128, bn = 128;   // workgroup tile
    int split = 1;            // K slices
    int k_chunk = 0;          // K elements per slice (multiple of 32)
    int tiles_per_wg = 1;     // > 1: persistent grid of ceil(tiles / tiles_per_wg) workgroups
    size_t workspace_bytes = 0;  // fp32 partials when split > 1
    bool wgemm = false;       // the weight-streaming engine (wgemm.hip): bm 128, bn 64 / 128
    int stages = 4;           // its LDS ring depth
};

GemmPlan plan_gemm(const GemmProblem& p);
// Weight-streaming engine: 16-bit A and B, NN, plain A, N % bn == 0, K % 64 == 0; fp32
// output, or split-K partials (any output type: the reduction converts).
// (shape conditions only, so that plans and workspace sizes depend on the shape alone; the
// operand pointers must also be 16-byte aligned -- wgemm_aligned -- or the launch takes the
// tiled engine with the same plan)
bool wgemm_supported(const GemmProblem& p, int bn, int split);
// The fused 2a2 epilogue applies to a problem that wgemm_supported takes with split 1 (and
// with w_uk set, on the plan's 128 x 4 tile only).
bool qup_supported(const GemmProblem& p, const QUpEpilogue& q, const GemmPlan& plan);
bool wgemm_aligned(const GemmProblem& p);
hipError_t launch_wgemm(const GemmProblem& p, const GemmPlan& plan, float* partials,
                        hipStream_t stream);
hipError_t launch_gemm(const GemmProblem& p, const GemmPlan& plan, void* workspace,
                       hipStream_t stream);
// Split-K slices only (plan.split > 1): fp32 partials [split][G][M][N] into `partials`,
// left for the consumer to sum (2a-n sums 2a1's partials while it normalises).
hipError_t launch_gemm_partials(const GemmProblem& p, const GemmPlan& plan, float* partials,
                                hipStream_t stream);

// ---------------------------------------------------------------- row kernels
// 2a-n: out[m][:] = sum_s in[s][m][:] * rsqrt(mean((sum_s in)^2) + eps) * gain
hipError_t launch_rmsnorm(const float* in, int nsplit, int64_t split_stride,
                          const void* gain, void* out, OutType out_type, int M, int N,
                          float eps, hipStream_t stream, const RopeTable& rope_table = {});
// 2b
// positions [Sq] shared by the batch, or [B*Sq] per sequence (pos_per_batch)
// With nope_out, q_raw is 2a2's split-K partials ([nsplit][B*Sq][H*(nope+rope)],
// split_stride floats apart): the kernel sums them in split order, writes the nope columns
// to nope_out (same layout as q_raw) and rotates the summed rope columns.
hipError_t launch_rope(const float* q_raw, const int64_t* positions, const float* inv_freq,
                       void* q_rope, OutType out_type, int B, int Sq, int H, int nope,
                       int rope, hipStream_t stream, bool pos_per_batch = false, int nsplit = 1,
                       int64_t split_stride = 0, float* nope_out = nullptr);
// 2b + 2c for decode-sized fp32 batches (B*Sq <= kQSmallRows, nope 128, kv 512, even
// rope <= 64): from 2a2's output or its split-K partials (q_parts, nsplit of them,
// split_stride floats apart, [B*Sq][H*(nope+rope)] each), the rotated q_rope [B*Sq][H][rope]
// (rope_kernel's arithmetic, the same bits) and q_abs [B*Sq][H][kv] = q_nope @ W_uk[h]
// (W_uk [H][nope][kv]) on the VALU, W_uk streamed once.  Pointers 16-byte aligned; at most
// kQSmallMaxSplit partials.
constexpr int kQSmallRows = 8;
constexpr int kQSmallMaxSplit = 8;
hipError_t launch_q_small(const float* q_parts, int nsplit, int64_t split_stride,
                          const int64_t* positions, const float* inv_freq, const float* W_uk,
                          float* q_rope, float* q_abs, int B, int Sq, int H, int nope, int rope,
                          int kv, bool pos_per_batch, hipStream_t stream);
// 3b (row_max may be null; when given it receives M = max_j m_part[row, j])
hipError_t launch_combine(const float* m_part, const float* l_part, float* alpha,
                          float* row_sum, float* row_max, int rows, int P, hipStream_t stream);
// Streaming merge of one key chunk into the running softmax state (online softmax):
//   M' = max(M, Mc); a = exp(M - M'), b = exp(Mc - M');
//   ctx = ctx*a + ctx_c*b;  L = L*a + Lc*b;  M = M'      (first chunk: plain copy)
hipError_t launch_stream_merge(float* ctx, float* run_max, float* run_sum, const float* ctx_c,
                               const float* max_c, const float* sum_c, int rows, int R,
                               bool first, hipStream_t stream);

// KV-cache append: in = x @ W_kv_a rows [B*Sq][R + D] (or nsplit split-K partials);
// c_kv[b][start_row + s] = RMSNorm(row[:R]) * gain (as launch_rmsnorm),
// pe[b][start_row + s] = RoPE(row[R:], positions[s]) (as launch_rope).
// Paged form (block_table given): token (b, s) goes to logical slot positions[b*Sq + s]
// (pos_per_batch) of sequence b, i.e. pool row table[b][slot/page_size]*page_size +
// slot%page_size; slots outside the table are skipped.
hipError_t launch_kv_append(const float* in, int nsplit, int64_t split_stride, const void* gain,
                            const int64_t* positions, const float* inv_freq, void* c_kv,
                            void* pe, OutType out_type, int B, int Sq, int R, int D,
                            int start_row, int cache_rows, float eps, hipStream_t stream,
                            bool pos_per_batch = false, const int* block_table = nullptr,
                            int page_size = 0, int max_pages = 0);
// Split each group of rows_a + rows_b rows (row_bytes each) of src into dst_a / dst_b.
// out[i] = e4m3 code[i] * scale (the fused attention's own fp8 -> bf16 conversion, then fp32)
hipError_t launch_fp8_dequant(const void* codes, int64_t n, float scale, float* out,
                              hipStream_t stream);
hipError_t launch_split_rows(const void* src, void* dst_a, void* dst_b, int64_t groups,
                             int rows_a, int rows_b, int64_t row_bytes, hipStream_t stream);

// ---------------------------------------------------------------- 3a scores
struct ScoresProblem {
    const void* qa = nullptr;    // [B*Sq*H, R]   storage dtype
    const void* qr = nullptr;    // [B*Sq*H, D]
    const void* ckv = nullptr;   // [B, Sk, R]
    const void* pe = nullptr;    // [B, Sk, D]
    bool half = false;           // storage / MFMA dtype 16-bit (else fp32)
    bool f16 = false;            // the 16-bit format is fp16 (else bfloat16)
    float* p = nullptr;          // [B*Sq*H, ld_p]
    float* m_part = nullptr;     // [B*Sq*H, P]
    float* l_part = nullptr;
    int B = 0, Sq = 0, Sk = 0, H = 0, R = 0, D = 0, ld_p = 0, P = 0;
    int64_t key_stride = 0;      // rows between batches of ckv / pe (>= Sk; Sk_total when chunked)
    int key_offset = 0;          // absolute index of key 0 (causal rule uses absolute keys)
    int sk_total = 0;            // keys in the whole sequence (causal rule)
    float inv_scale = 1.f;
    bool causal = false;
    // ragged / paged keys (optional): per-batch key counts (<= Sk) and a block table
    // [B][max_pages] of page_size-row pages of ckv / pe (page_size a multiple of 64)
    const int* seq_lens = nullptr;
    const int* block_table = nullptr;
    int page_size = 0, max_pages = 0;
};
hipError_t launch_scores(const ScoresProblem& p, hipStream_t stream);

constexpr int kScoreTile = 128;  // keys per softmax partial (one 3a workgroup's key tile)

// ---------------------------------------------------------------- 3a+3b+3c fused
// One pass over the cache per key split: ctx [rows, R] (unnormalised) and row_sum [rows]
// for 3d, as 3c and 3b produce them.  16-bit or fp32 storage (or an fp8 cache with bf16
// queries), R = 512, D = 64 only.
struct FlashProblem {
    bool half = true;            // storage dtype 16-bit (else fp32)
    bool f16 = false;            // the 16-bit format is fp16 (else bfloat16)
    const void* qa = nullptr;    // [B*Sq*H, R]
    const void* qr = nullptr;    // [B*Sq*H, D]
    const void* ckv = nullptr;   // [B, key_stride, R]
    const void* pe = nullptr;    // [B, key_stride, D]
    int B = 0, Sq = 0, Sk = 0, H = 0, R = 0, D = 0;
    int64_t key_stride = 0;      // key rows between batches (0: Sk)
    float scale = 1.f;           // divisor of the scores
    bool causal = false;
    // ragged / paged keys (optional): batch b has min(seq_lens[b], Sk) keys; with a block
    // table, ckv / pe are pools of pages of page_size rows (a multiple of 64, Sk a multiple
    // of it) and key k of batch b is row k % page_size of page block_table[b*Sk/page_size
    // + k/page_size]
    const int32_t* seq_lens = nullptr;
    const int32_t* block_table = nullptr;
    int page_size = 0;
    bool ragged = false;         // plan for per-batch key counts (a size query sets this
                                 // without seq_lens; a launch with it needs seq_lens)
    bool want_list = false;      // plan the balanced work list even where a small fp32
                                 // batch would run the key-split waves (list inspection)
    // fp8 cache (bf16 queries only): ckv / pe hold OCP e4m3 codes of value / kv_scale,
    // one byte per element (rows of R and D bytes)
    bool fp8_kv = false;
    float kv_scale = 1.f;
};
struct FlashPlan {
    bool wave = false;           // fp32 pass on 16-row workgroups of key-split waves
    int row_tiles = 1;           // row tiles per batch (64 rows; 16 with `wave`)
    int n_split = 1;             // key splits (one workgroup each)
    int keys_per_split = 0;      // multiple of the key block
    bool balanced = false;       // ragged keys: a device-built work list of key chunks
    int max_items = 0;           // its largest item count (grid = max_items * row_tiles)
    size_t partial_bytes = 0;    // scratch: split partials (and the work list)
};
bool flash_supported(const FlashProblem& p);
FlashPlan plan_flash(const FlashProblem& p);
// merge = false leaves a split pass's partials unmerged (flash_partials() locates them)
// for a consumer that folds the merge in (launch_out_small).
hipError_t launch_flash(const FlashProblem& p, const FlashPlan& plan, float* ctx, float* row_sum,
                        float* partials, hipStream_t stream, bool merge = true,
                        void* ctx16 = nullptr);
// ctx16 (launch_flash): a dense unsplit 16-bit or fp8-cache pass on the default kernels can
// write ctx already normalised by its row sum and rounded to the storage format
// ([rows][R], the values 3d's A staging would form), instead of ctx and row_sum.
// MLA_CTX16=0 turns this off.
bool flash_ctx16_ok(const FlashProblem& p, const FlashPlan& plan);
// Where a dense (not balanced) pass leaves its state: n_split > 1 -> partial rows o
// [n_split][rows][R], log2-domain references m and row sums l [n_split][rows] (slot
// s * B * rows_b + row); n_split == 1 -> ctx / row_sum themselves.
struct FlashPartials { const float* o; const float* m; const float* l; int n_split; };
FlashPartials flash_partials(const FlashProblem& p, const FlashPlan& plan, const float* partials);
// 3d for decode-sized fp32 batches (B*Sq <= kOutSmallRows, R = 512), with the fused
// attention's split merge folded in: out[B*Sq][H][V] from the pass's state (fp.n_split > 1:
// partials, else ctx / row_sum) and W_uv [H][V][R].
constexpr int kOutSmallRows = 8;
constexpr int kOutSmallMaxSplit = 64;
// Where it pays (measured, attention with 3d at Sk = 4989): both workgroups of a head read
// the head's B*Sq*n_split partial rows beside the W_uv stream.  With a merge it is taken up
// to B*Sq = 4 and 128 such rows (B=1: 43.1 against 49.1 us, B=2 54.1 / 60.2, B=4 87.6 /
// 88.3); at B=8 (16 splits) the merge kernel and the 3d GEMM are faster (128.9 against
// 132.1 us), so B*Sq = 5 .. 8 take it after the merge kernel, on the merged ctx / row_sum
// (B=8: 128.7 against 129.4 us for the merge kernel and the GEMM; B=5: 97.8 / 100.4).
constexpr int kOutSmallMergeRows = 128;
constexpr int kOutSmallMergeM = 4;
hipError_t launch_out_small(const FlashPartials& fp, const float* ctx, const float* row_sum,
                            const float* W_uv, float* out, int B, int Sq, int H, int R, int V,
                            hipStream_t stream);
// The work list alone (plan.balanced, seq_lens given): wl receives flash_worklist_ints()
// ints, laid out as worklist.h describes.
int flash_worklist_ints(const FlashProblem& p, const FlashPlan& plan);
hipError_t launch_flash_worklist(const FlashProblem& p, const FlashPlan& plan, int* wl,
                                 hipStream_t stream);

// ---------------------------------------------------------------- float64 path (f64.hip)
// C[g] = alpha * A[g] . op(B[g]) + beta * C[g] in double on the double MFMA (beta 0: C is
// not read):  A[g][m][k] at A + g*sA + m*lda + k;  B (NN) at B + g*sB + k*ldb + n,
// B (NT, b_nt) at B + g*sB + n*ldb + k;  C[g][m][n] at C + g*sC + m*ldc + n.
struct Gemm64Problem {
    const double* A = nullptr; int64_t lda = 0, sA = 0;
    const double* B = nullptr; int64_t ldb = 0, sB = 0;
    double* C = nullptr;       int64_t ldc = 0, sC = 0;
    int M = 0, N = 0, K = 0, G = 1;
    bool b_nt = false;
    double alpha = 1.0, beta = 0.0;
};
hipError_t launch_gemm64(const Gemm64Problem& p, hipStream_t stream);
// 2a-n in place on x [M][N]: x = (x / sqrt(mean(x^2) + eps)) * gain
hipError_t launch_rmsnorm64(double* x, const double* gain, int M, int N, double eps,
                            hipStream_t stream);
// 2b: q_rope [B*Sq][H][rope] from q_raw [B*Sq][H*(nope+rope)], positions [Sq] (or [B*Sq]
// with per_batch), inv_freq [rope/2]
hipError_t launch_rope64(const double* q_raw, const int64_t* pos, const double* inv_freq,
                         double* q_rope, int B, int Sq, int H, int nope, int rope,
                         bool per_batch, hipStream_t stream);
// in place on S [rows][Sk] (row = (b*Sq + s)*H + h): softmax over the visible keys of
// S / scale, zeros where masked
hipError_t launch_softmax64(double* S, int rows, int Sk, int Sq, int H, double scale,
                            bool causal, hipStream_t stream);

}  // namespace mla
