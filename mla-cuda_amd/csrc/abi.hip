// extern "C" surface of libmla_amd.so (declared in include/mla/mla.h).
//
// Every entry point validates its arguments completely -- dims, pointers, alignment,
// workspace size, dtype -- before the first HIP call, so a rejected call leaves the
// device untouched and the validation is testable on a machine without a GPU.  Kernel
// grids are planned from the shapes alone (plan_gemm / fixed 3a tiles), so the
// *_workspace_bytes() queries and the launches always agree.

#include <algorithm>
#include <cmath>
#include <cstdarg>
#include <cstdio>
#include <cstdlib>
#include <cstring>
#include <mutex>
#include <string>

#include "../../include/mla/mla.h"
#include "kernels.h"

using namespace mla;

namespace {

thread_local std::string g_last_error;

int fail(int status, const char* fmt, ...) {
    char buf[512];
    va_list ap;
    va_start(ap, fmt);
    vsnprintf(buf, sizeof(buf), fmt, ap);
    va_end(ap);
    g_last_error = buf;
    return status;
}

int ok() {
    g_last_error.clear();
    return MLA_OK;
}

int hip_fail(hipError_t e, const char* what) {
    return fail(MLA_ERR_HIP, "%s: %s", what, hipGetErrorString(e));
}

#define MLA_TRY_HIP(expr, what)                         \
    do {                                                \
        hipError_t e_ = (expr);                         \
        if (e_ != hipSuccess) return hip_fail(e_, what); \
    } while (0)

constexpr size_t kAlign = 256;
size_t align_up(size_t x) { return (x + kAlign - 1) / kAlign * kAlign; }
int cdiv(int a, int b) { return (a + b - 1) / b; }

bool aligned16(const void* p) { return (reinterpret_cast<uintptr_t>(p) & 15u) == 0; }

int check_ptr(const void* p, const char* name) {
    if (!p) return fail(MLA_ERR_INVALID_ARGUMENT, "%s must not be NULL", name);
    if (!aligned16(p)) return fail(MLA_ERR_INVALID_ARGUMENT, "%s must be 16-byte aligned", name);
    return MLA_OK;
}

#define MLA_CHECK(expr)            \
    do {                           \
        int st_ = (expr);          \
        if (st_ != MLA_OK) return st_; \
    } while (0)

int check_dtype(mla_dtype_t dt) {
    if (dt == MLA_DTYPE_F32 || dt == MLA_DTYPE_BF16 || dt == MLA_DTYPE_F16) return MLA_OK;
    if (dt == MLA_DTYPE_F64)
        return fail(MLA_ERR_UNSUPPORTED, "float64 is taken by mla_q_absorbed, "
                    "mla_q_absorbed_ragged, mla_attention and mla_attention_noalloc only");
    return fail(MLA_ERR_INVALID_ARGUMENT, "unknown dtype %d", (int)dt);
}

// 16-bit storage (bf16 or fp16); the kernels take the format as a second flag
bool is_half(mla_dtype_t dt) { return dt == MLA_DTYPE_BF16 || dt == MLA_DTYPE_F16; }
bool is_f16(mla_dtype_t dt) { return dt == MLA_DTYPE_F16; }
OutType storage_out(mla_dtype_t dt) {
    return dt == MLA_DTYPE_BF16 ? kOutBF16 : dt == MLA_DTYPE_F16 ? kOutF16 : kOutF32;
}
const char* dtype_name(mla_dtype_t dt) {
    return dt == MLA_DTYPE_BF16 ? "bf16" : dt == MLA_DTYPE_F16 ? "fp16" : "fp32";
}

// Row lengths of storage-dtype tensors must be whole 16-byte chunks: 4 fp32 / 8 16-bit.
int check_row(mla_dtype_t dt, int v, const char* name) {
    // float64 has its own shape rules (check_f64_*); every path that reaches here is one
    // that does not take it
    if (dt == MLA_DTYPE_F64) return check_dtype(dt);
    const int q = is_half(dt) ? 8 : 4;
    if (v <= 0 || v % q != 0)
        return fail(MLA_ERR_INVALID_ARGUMENT, "%s must be a positive multiple of %d for %s (got %d)",
                    name, q, dtype_name(dt), v);
    return MLA_OK;
}

int check_pos(int64_t v, const char* name) {
    if (v <= 0) return fail(MLA_ERR_INVALID_ARGUMENT, "%s must be positive (got %lld)", name,
                            (long long)v);
    return MLA_OK;
}

int check_mult4(int v, const char* name) {
    if (v <= 0 || v % 4 != 0)
        return fail(MLA_ERR_INVALID_ARGUMENT, "%s must be a positive multiple of 4 (got %d)",
                    name, v);
    return MLA_OK;
}

// Upper bound for any row count / flattened index the kernels form in 32-bit ints.
constexpr int64_t kMaxI32 = 0x7fffffffLL;

int check_q_dims(mla_dtype_t dt, const mla_dims_t* d) {
    if (!d) return fail(MLA_ERR_INVALID_ARGUMENT, "dims must not be NULL");
    MLA_CHECK(check_pos(d->batch, "dims.batch"));
    MLA_CHECK(check_pos(d->sq, "dims.sq"));
    MLA_CHECK(check_pos(d->heads, "dims.heads"));
    MLA_CHECK(check_row(dt, d->hidden, "dims.hidden"));
    MLA_CHECK(check_row(dt, d->q_lora, "dims.q_lora"));
    MLA_CHECK(check_row(dt, d->nope, "dims.nope"));
    MLA_CHECK(check_row(dt, d->rope, "dims.rope"));
    MLA_CHECK(check_row(dt, d->kv_rank, "dims.kv_rank"));
    if (d->rope > 512) return fail(MLA_ERR_INVALID_ARGUMENT, "dims.rope must be <= 512");
    const int64_t bq = (int64_t)d->batch * d->sq;
    if (bq * d->heads * (int64_t)(d->nope + d->rope) > kMaxI32 ||
        bq * d->heads * (int64_t)d->kv_rank > (int64_t)1 << 40)
        return fail(MLA_ERR_INVALID_ARGUMENT, "batch*sq*heads too large");
    return MLA_OK;
}

// The fields the work list reads: batch, sq, heads and sk (the block table's key span).
int check_work_list_dims(const mla_dims_t* d) {
    if (!d) return fail(MLA_ERR_INVALID_ARGUMENT, "dims must not be NULL");
    MLA_CHECK(check_pos(d->batch, "dims.batch"));
    MLA_CHECK(check_pos(d->sq, "dims.sq"));
    MLA_CHECK(check_pos(d->sk, "dims.sk"));
    MLA_CHECK(check_pos(d->heads, "dims.heads"));
    if ((int64_t)d->sq * d->heads > kMaxI32 / 2 || (int64_t)d->sk > kMaxI32 / 1024)
        return fail(MLA_ERR_INVALID_ARGUMENT, "sq*heads or sk too large");
    return MLA_OK;
}

// The fields the 2b / 2c steps read: batch, sq, heads, nope, rope (+ kv_rank for 2c).
int check_qraw_dims(mla_dtype_t dt, const mla_dims_t* d, bool absorb) {
    if (!d) return fail(MLA_ERR_INVALID_ARGUMENT, "dims must not be NULL");
    MLA_CHECK(check_pos(d->batch, "dims.batch"));
    MLA_CHECK(check_pos(d->sq, "dims.sq"));
    MLA_CHECK(check_pos(d->heads, "dims.heads"));
    MLA_CHECK(check_row(dt, d->nope, "dims.nope"));
    MLA_CHECK(check_row(dt, d->rope, "dims.rope"));
    if (d->rope > 512) return fail(MLA_ERR_INVALID_ARGUMENT, "dims.rope must be <= 512");
    if (absorb) MLA_CHECK(check_row(dt, d->kv_rank, "dims.kv_rank"));
    if ((int64_t)d->batch * d->sq * d->heads * (int64_t)(d->nope + d->rope) > kMaxI32)
        return fail(MLA_ERR_INVALID_ARGUMENT, "batch*sq*heads too large");
    return MLA_OK;
}

// 3c reads batch, sq, sk, heads, kv_rank; 3d reads batch, sq, heads, kv_rank, v.
int check_ctx_dims(mla_dtype_t dt, const mla_dims_t* d) {
    if (!d) return fail(MLA_ERR_INVALID_ARGUMENT, "dims must not be NULL");
    MLA_CHECK(check_pos(d->batch, "dims.batch"));
    MLA_CHECK(check_pos(d->sq, "dims.sq"));
    MLA_CHECK(check_pos(d->sk, "dims.sk"));
    MLA_CHECK(check_pos(d->heads, "dims.heads"));
    MLA_CHECK(check_row(dt, d->kv_rank, "dims.kv_rank"));
    if ((int64_t)d->batch * d->sq * d->heads > kMaxI32 / 2)
        return fail(MLA_ERR_INVALID_ARGUMENT, "batch*sq*heads too large");
    if ((int64_t)d->sk > kMaxI32 / 1024) return fail(MLA_ERR_INVALID_ARGUMENT, "sk too large");
    return MLA_OK;
}

int check_out_dims(mla_dtype_t dt, const mla_dims_t* d) {
    if (!d) return fail(MLA_ERR_INVALID_ARGUMENT, "dims must not be NULL");
    MLA_CHECK(check_pos(d->batch, "dims.batch"));
    MLA_CHECK(check_pos(d->sq, "dims.sq"));
    MLA_CHECK(check_pos(d->heads, "dims.heads"));
    MLA_CHECK(check_row(dt, d->kv_rank, "dims.kv_rank"));
    MLA_CHECK(check_mult4(d->v, "dims.v"));
    if ((int64_t)d->batch * d->sq * d->heads > kMaxI32 / 2)
        return fail(MLA_ERR_INVALID_ARGUMENT, "batch*sq*heads too large");
    return MLA_OK;
}

int check_attn_dims(mla_dtype_t dt, const mla_dims_t* d, int causal) {
    if (!d) return fail(MLA_ERR_INVALID_ARGUMENT, "dims must not be NULL");
    MLA_CHECK(check_pos(d->batch, "dims.batch"));
    MLA_CHECK(check_pos(d->sq, "dims.sq"));
    MLA_CHECK(check_pos(d->sk, "dims.sk"));
    MLA_CHECK(check_pos(d->heads, "dims.heads"));
    MLA_CHECK(check_row(dt, d->rope, "dims.rope"));
    MLA_CHECK(check_row(dt, d->kv_rank, "dims.kv_rank"));
    MLA_CHECK(check_mult4(d->v, "dims.v"));
    if (causal && d->sk < d->sq)
        return fail(MLA_ERR_INVALID_ARGUMENT,
                    "causal attention needs sk >= sq (got sk=%d, sq=%d)", d->sk, d->sq);
    const int64_t rows = (int64_t)d->batch * d->sq * d->heads;
    if (rows > kMaxI32 / 2) return fail(MLA_ERR_INVALID_ARGUMENT, "batch*sq*heads too large");
    if ((int64_t)d->sk > kMaxI32 / 1024)
        return fail(MLA_ERR_INVALID_ARGUMENT, "sk too large (%d)", d->sk);
    return MLA_OK;
}

int check_ws(void* ws, size_t have, size_t need) {
    if (need == 0) return MLA_OK;
    if (!ws) return fail(MLA_ERR_WORKSPACE, "workspace is NULL but %zu bytes are required", need);
    if (have < need)
        return fail(MLA_ERR_WORKSPACE, "workspace too small: %zu bytes given, %zu required", have,
                    need);
    if ((reinterpret_cast<uintptr_t>(ws) & (kAlign - 1)) != 0)
        return fail(MLA_ERR_WORKSPACE, "workspace must be %zu-byte aligned", kAlign);
    return MLA_OK;
}

// ------------------------------------------------------------------ problem builders

GemmProblem q_down_problem(mla_dtype_t dt, const mla_dims_t* d, const void* x, const void* W,
                           float* C) {
    GemmProblem p;
    p.half = is_half(dt); p.f16 = is_f16(dt); p.a_f32 = !is_half(dt);
    p.A = x; p.lda = d->hidden;
    p.B = W; p.ldb = d->q_lora;
    p.C = C; p.ldc = d->q_lora;
    p.M = d->batch * d->sq; p.N = d->q_lora; p.K = d->hidden;
    return p;
}

GemmProblem q_up_problem(mla_dtype_t dt, const mla_dims_t* d, const void* q_lat, const void* W,
                         float* C) {
    const int n = d->heads * (d->nope + d->rope);
    GemmProblem p;
    p.half = is_half(dt); p.f16 = is_f16(dt); p.a_f32 = !is_half(dt);
    p.A = q_lat; p.lda = d->q_lora;
    p.B = W; p.ldb = n;
    p.C = C; p.ldc = n;
    p.M = d->batch * d->sq; p.N = n; p.K = d->q_lora;
    return p;
}

// A is q_raw's nope columns (fp32, [B*Sq, H*(nope+rope)]), or with nope16 the 16-bit
// q_nope [B*Sq, H, nope] that 2a2's fused epilogue writes.
GemmProblem absorb_problem(mla_dtype_t dt, const mla_dims_t* d, const void* q_raw,
                           const void* W_uk, void* q_abs, bool nope16 = false) {
    const int qk = d->nope + d->rope;
    GemmProblem p;
    p.half = is_half(dt); p.f16 = is_f16(dt); p.a_f32 = !nope16; p.out_type = storage_out(dt);
    p.A = q_raw; p.lda = (int64_t)d->heads * (nope16 ? d->nope : qk); p.sAg = nope16 ? d->nope : qk;
    p.B = W_uk; p.ldb = d->kv_rank; p.sBg = (int64_t)d->nope * d->kv_rank;
    p.C = q_abs; p.ldc = (int64_t)d->heads * d->kv_rank; p.sCg = d->kv_rank;
    p.M = d->batch * d->sq; p.N = d->kv_rank; p.K = d->nope; p.G = d->heads;
    return p;
}

GemmProblem ctx_problem(mla_dtype_t dt, const mla_dims_t* d, const float* p_scores, int ld_p,
                        const float* alpha, const void* c_kv, float* ctx) {
    const int rows_b = d->sq * d->heads;
    GemmProblem p;
    p.half = is_half(dt); p.f16 = is_f16(dt); p.a_f32 = true;
    p.A = p_scores; p.lda = ld_p; p.sAg = (int64_t)rows_b * ld_p;
    p.B = c_kv; p.ldb = d->kv_rank; p.sBg = (int64_t)d->sk * d->kv_rank;
    p.C = ctx; p.ldc = d->kv_rank; p.sCg = (int64_t)rows_b * d->kv_rank;
    p.M = rows_b; p.N = d->kv_rank; p.K = d->sk; p.G = d->batch;
    p.amode = kAAlpha; p.alpha = alpha; p.alpha_ld = cdiv(d->sk, kScoreTile);
    p.alpha_tile = kScoreTile;
    return p;
}

GemmProblem out_problem(mla_dtype_t dt, const mla_dims_t* d, const float* ctx,
                        const float* row_sum, const void* W_uv, void* out) {
    GemmProblem p;
    p.half = is_half(dt); p.f16 = is_f16(dt); p.a_f32 = true; p.out_type = storage_out(dt);
    p.A = ctx; p.lda = (int64_t)d->heads * d->kv_rank; p.sAg = d->kv_rank;
    p.B = W_uv; p.ldb = d->kv_rank; p.sBg = (int64_t)d->v * d->kv_rank; p.b_nt = true;
    p.C = out; p.ldc = (int64_t)d->heads * d->v; p.sCg = d->v;
    p.M = d->batch * d->sq; p.N = d->v; p.K = d->kv_rank; p.G = d->heads;
    p.amode = kARowRecip; p.rs = row_sum; p.rs_m = d->heads; p.rs_g = 1;
    return p;
}

// 3d from the fused pass's normalised 16-bit ctx (flash_ctx16_ok): A is that ctx
// [B*Sq, H*kv_rank] in the storage format, no row scale.
GemmProblem out_problem16(mla_dtype_t dt, const mla_dims_t* d, const void* ctx16,
                          const void* W_uv, void* out) {
    GemmProblem p = out_problem(dt, d, nullptr, nullptr, W_uv, out);
    p.A = ctx16; p.a_f32 = false; p.amode = kAPlain; p.rs = nullptr;
    return p;
}

// ------------------------------------------------------------------ workspace layouts

struct QLayout {
    GemmPlan down, up, absorb;
    bool fused;   // 2a2 writes q_nope and the rotated q_rope itself (no 2b launch)
    bool fused_2c;  // ... and 2c too (no 2c launch, no q_nope), when the pointers allow
    bool rope_epi;  // fp32: 2a2 on the tiled engine rotates q_rope in its epilogue (no 2b)
    size_t off_lat_acc, off_lat, off_raw, off_up_ws, off_abs_ws, off_rope_tab, total;
};

// 2a2's fused epilogue (wgemm.hip) for a 16-bit weight-streaming 2a2 plan without split-K;
// MLA_QUP_FUSE=0 keeps the separate 2b launch (a comparison aid: both give the same bits).
bool qup_fused(mla_dtype_t dt, const mla_dims_t* d, const GemmPlan& up) {
    const char* env = getenv("MLA_QUP_FUSE");
    if (env && strcmp(env, "0") == 0) return false;
    return is_half(dt) && up.wgemm && up.split == 1 && up.bn <= 128 && d->nope % 32 == 0 &&
           d->rope % 32 == 0 &&
           d->rope > 0 && d->rope <= 64;
}

// 2a2's fused epilogue with 2c as well (wgemm.hip, qup_supported): one head's nope columns
// per 128-column tile of the 128 x 4 plan; MLA_QUP_ABSORB=0 keeps the 2c launch (a
// comparison aid: both give the same bits).
bool qup_fused_2c(mla_dtype_t dt, const mla_dims_t* d, const GemmPlan& up) {
    const char* env = getenv("MLA_QUP_ABSORB");
    if (env && strcmp(env, "0") == 0) return false;
    return qup_fused(dt, d, up) && up.bn == 128 && up.stages == 4 && d->nope == 128 &&
           d->rope == 64 && d->heads % 2 == 0 && d->kv_rank % 128 == 0 && d->kv_rank <= 512;
}

// 2b + 2c as one VALU kernel at decode-sized fp32 batches (rowops.hip, launch_q_small);
// MLA_Q_SMALL=0 keeps the 2b launch and the MFMA 2c.
bool q_small_ok(mla_dtype_t dt, const mla_dims_t* d, const GemmPlan& up, const void* W_uk,
                const void* q_abs, const void* q_rope) {
    const char* env = getenv("MLA_Q_SMALL");
    if (env && strcmp(env, "0") == 0) return false;
    return dt == MLA_DTYPE_F32 && (int64_t)d->batch * d->sq <= kQSmallRows &&
           std::max(1, up.split) <= kQSmallMaxSplit && d->nope == 128 &&
           d->kv_rank == 512 && d->rope % 2 == 0 && d->rope <= 64 &&
           (reinterpret_cast<uintptr_t>(W_uk) & 15) == 0 &&
           (reinterpret_cast<uintptr_t>(q_abs) & 15) == 0 &&
           (reinterpret_cast<uintptr_t>(q_rope) & 7) == 0;
}

// fp32 2a2 in one K split on the tiled engine does 2b in its epilogue (gemm.hip, ROPE
// kernels), on tiles whose waves hold one 32x32 block each (64x64, 32x128, 128x32).  With
// more blocks per wave, a later block's cos / sin loads queue behind the earlier block's
// stores on the one memory counter: M = 512 on 128x128 tiles measured 563 us against
// 487 us with the RoPE launch, while B = 128 on 64x64 tiles gains ~3 us.
// MLA_ROPE_EPI=0 keeps the RoPE launch (a comparison aid: both give the same bits).
bool rope_epi_ok(mla_dtype_t dt, const mla_dims_t* d, const GemmPlan& up) {
    const char* env = getenv("MLA_ROPE_EPI");
    if (env && strcmp(env, "0") == 0) return false;
    const bool one_block = (up.bm == 64 && up.bn == 64) || (up.bm == 32 && up.bn == 128) ||
                           (up.bm == 128 && up.bn == 32);
    return dt == MLA_DTYPE_F32 && !up.wgemm && up.split == 1 && up.tiles_per_wg == 1 &&
           one_block && d->nope % 32 == 0 && d->rope % 32 == 0 && d->rope / 2 <= 256;
}

QLayout q_layout(mla_dtype_t dt, const mla_dims_t* d) {
    QLayout L;
    const size_t bq = (size_t)d->batch * d->sq;
    const size_t n_raw = (size_t)d->heads * (d->nope + d->rope);
    L.down = plan_gemm(q_down_problem(dt, d, nullptr, nullptr, nullptr));
    L.up = plan_gemm(q_up_problem(dt, d, nullptr, nullptr, nullptr));
    L.fused = qup_fused(dt, d, L.up);
    L.fused_2c = L.fused && qup_fused_2c(dt, d, L.up);
    L.rope_epi = rope_epi_ok(dt, d, L.up);
    L.absorb = plan_gemm(absorb_problem(dt, d, nullptr, nullptr, nullptr, L.fused));
    size_t o = 0;
    L.off_lat_acc = o;  // 2a1 output or its split partials (summed by the norm kernel)
    o = align_up(o + (size_t)L.down.split * bq * d->q_lora * sizeof(float));
    L.off_lat = o;
    o = align_up(o + bq * d->q_lora * sizeof(float));
    L.off_raw = o;
    o = align_up(o + bq * n_raw * sizeof(float));
    L.off_up_ws = o;
    o = align_up(o + L.up.workspace_bytes);
    L.off_abs_ws = o;
    o = align_up(o + L.absorb.workspace_bytes);
    L.off_rope_tab = o;   // 2a-n's RoPE angle table for the fused epilogue
    if (L.fused || L.rope_epi) o = align_up(o + bq * (size_t)d->rope * sizeof(float));
    L.total = o;
    return L;
}

// 3a+3b+3c as one fused pass over the cache (flash.hip), for 16-bit and fp32 storage at the
// DeepSeek-V3 widths.  MLA_ATTENTION_PATH=split selects the per-step kernels instead.
FlashProblem flash_problem(mla_dtype_t dt, const mla_dims_t* d, const void* qa, const void* qr,
                           const void* ckv, const void* pe, double scale, int causal) {
    FlashProblem p;
    p.half = is_half(dt); p.f16 = is_f16(dt);
    p.qa = qa; p.qr = qr; p.ckv = ckv; p.pe = pe;
    p.B = d->batch; p.Sq = d->sq; p.Sk = d->sk; p.H = d->heads; p.R = d->kv_rank;
    p.D = d->rope; p.key_stride = d->sk;
    p.scale = (float)scale;
    p.causal = causal != 0;
    return p;
}

bool flash_eligible(mla_dtype_t dt, const mla_dims_t* d) {
    // per-lane 32-bit buffer offsets: a batch's query rows and key rows (R elements each)
    constexpr int64_t kRange = 0x7fffffff;
    const int64_t row_bytes = 512 * (is_half(dt) ? 2 : 4);
    if ((int64_t)d->sq * d->heads * row_bytes >= kRange || (int64_t)d->sk * row_bytes >= kRange)
        return false;
    return flash_supported(flash_problem(dt, d, nullptr, nullptr, nullptr, nullptr, 1.0, 0));
}

bool use_flash(mla_dtype_t dt, const mla_dims_t* d) {
    const char* e = std::getenv("MLA_ATTENTION_PATH");
    if (e && std::strcmp(e, "split") == 0) return false;
    return flash_eligible(dt, d);
}

struct AttnLayout {
    bool fused = false;   // the path this layout is for
    bool ctx16 = false;   // fused: the pass writes the normalised 16-bit ctx for 3d
    int ld_p, P;
    GemmPlan ctx, out;
    FlashPlan flash;
    size_t off_p, off_m, off_l, off_alpha, off_rowsum, off_ctx, off_ctx_ws, off_out_ws, off_part,
        total;
};

// The workspace of the attention path a call takes (use_flash: read per call, so a caller
// that changes MLA_ATTENTION_PATH between the size query and the call gets
// MLA_ERR_WORKSPACE, never an overrun).  Fused: ctx, row_sum, the split partials and 3d's
// workspace -- no score matrix; `ragged` (the paged entry points) sizes the partials for
// the work list that balances per-sequence key counts.  Per-step: scores, tile partials,
// alpha, row_sum, ctx and the 3c / 3d workspaces.
AttnLayout attn_layout(mla_dtype_t dt, const mla_dims_t* d, bool ragged = false) {
    AttnLayout L;
    const size_t rows = (size_t)d->batch * d->sq * d->heads;
    L.ld_p = mla_score_ld(d->sk);
    L.P = cdiv(d->sk, kScoreTile);
    L.out = plan_gemm(out_problem(dt, d, nullptr, nullptr, nullptr, nullptr));
    size_t o = 0;
    L.fused = use_flash(dt, d);
    if (L.fused) {
        FlashProblem fp = flash_problem(dt, d, nullptr, nullptr, nullptr, nullptr, 1.0, 0);
        fp.ragged = ragged;
        L.flash = plan_flash(fp);
        L.ctx16 = flash_ctx16_ok(fp, L.flash);
        if (L.ctx16) L.out = plan_gemm(out_problem16(dt, d, nullptr, nullptr, nullptr));
        L.off_p = L.off_m = L.off_l = L.off_alpha = L.off_ctx_ws = 0;
        L.off_rowsum = o; o = align_up(o + rows * sizeof(float));
        L.off_ctx = o;    o = align_up(o + rows * d->kv_rank * sizeof(float));
        L.off_out_ws = o; o = align_up(o + L.out.workspace_bytes);
        L.off_part = o;   o = align_up(o + L.flash.partial_bytes);
        L.total = o;
        return L;
    }
    L.ctx = plan_gemm(ctx_problem(dt, d, nullptr, L.ld_p, nullptr, nullptr, nullptr));
    L.off_p = o;      o = align_up(o + rows * L.ld_p * sizeof(float));
    L.off_m = o;      o = align_up(o + rows * L.P * sizeof(float));
    L.off_l = o;      o = align_up(o + rows * L.P * sizeof(float));
    L.off_alpha = o;  o = align_up(o + rows * L.P * sizeof(float));
    L.off_rowsum = o; o = align_up(o + rows * sizeof(float));
    L.off_ctx = o;    o = align_up(o + rows * d->kv_rank * sizeof(float));
    L.off_ctx_ws = o; o = align_up(o + L.ctx.workspace_bytes);
    L.off_out_ws = o; o = align_up(o + L.out.workspace_bytes);
    L.off_part = 0;
    L.total = o;
    return L;
}

struct StreamLayout {
    int chunk;  // keys per chunk
    GemmPlan out;
    size_t off_p, off_m, off_l, off_alpha, off_sum_c, off_max_c, off_ctx_c, off_ctx, off_run_max,
        off_run_sum, off_ctx_ws, off_out_ws, total;
};

// Chunk choice for streaming attention: the largest multiple of the score tile whose fp32
// score buffer stays within 1 GiB (at least one tile; at most the whole key range).
int stream_chunk(const mla_dims_t* d, int32_t key_chunk) {
    const int64_t rows = (int64_t)d->batch * d->sq * d->heads;
    const int full = cdiv(d->sk, kScoreTile) * kScoreTile;
    int c = key_chunk;
    if (c == 0) {
        const int64_t fit = ((int64_t)1 << 30) / (rows * 4) / kScoreTile * kScoreTile;
        c = (int)std::max<int64_t>(kScoreTile, std::min<int64_t>(fit, full));
    }
    return std::min(c, full);
}

StreamLayout stream_layout(mla_dtype_t dt, const mla_dims_t* d, int32_t key_chunk) {
    StreamLayout L;
    const size_t rows = (size_t)d->batch * d->sq * d->heads;
    L.chunk = stream_chunk(d, key_chunk);
    const int P = cdiv(L.chunk, kScoreTile);
    // the 3c plan depends on the chunk length: take the larger workspace of a full chunk
    // and of the (possibly shorter) last one
    size_t ctx_ws = 0;
    for (int kc : {L.chunk, d->sk - (cdiv(d->sk, L.chunk) - 1) * L.chunk}) {
        mla_dims_t dc = *d;
        dc.sk = kc;
        GemmProblem cp = ctx_problem(dt, &dc, nullptr, mla_score_ld(kc), nullptr, nullptr, nullptr);
        ctx_ws = std::max(ctx_ws, plan_gemm(cp).workspace_bytes);
    }
    L.out = plan_gemm(out_problem(dt, d, nullptr, nullptr, nullptr, nullptr));
    size_t o = 0;
    L.off_p = o;       o = align_up(o + rows * mla_score_ld(L.chunk) * sizeof(float));
    L.off_m = o;       o = align_up(o + rows * P * sizeof(float));
    L.off_l = o;       o = align_up(o + rows * P * sizeof(float));
    L.off_alpha = o;   o = align_up(o + rows * P * sizeof(float));
    L.off_sum_c = o;   o = align_up(o + rows * sizeof(float));
    L.off_max_c = o;   o = align_up(o + rows * sizeof(float));
    L.off_ctx_c = o;   o = align_up(o + rows * d->kv_rank * sizeof(float));
    L.off_ctx = o;     o = align_up(o + rows * d->kv_rank * sizeof(float));
    L.off_run_max = o; o = align_up(o + rows * sizeof(float));
    L.off_run_sum = o; o = align_up(o + rows * sizeof(float));
    L.off_ctx_ws = o;  o = align_up(o + ctx_ws);
    L.off_out_ws = o;  o = align_up(o + L.out.workspace_bytes);
    L.total = o;
    return L;
}

template <typename T> T* at(void* base, size_t off) {
    return reinterpret_cast<T*>(static_cast<char*>(base) + off);
}

// ------------------------------------------------------------------ step bodies

int run_scores(mla_dtype_t dt, const mla_dims_t* d, const void* qa, const void* qr, const void* ckv,
               const void* pe, double scale, int causal, float* p, int ld_p, float* m_part,
               float* l_part, hipStream_t stream, int64_t key_stride = 0, int key_offset = 0,
               int sk_total = 0, const int* seq_lens = nullptr, const int* block_table = nullptr,
               int page_size = 0) {
    ScoresProblem sp;
    sp.qa = qa; sp.qr = qr; sp.ckv = ckv; sp.pe = pe;
    sp.half = is_half(dt); sp.f16 = is_f16(dt);
    sp.p = p; sp.m_part = m_part; sp.l_part = l_part;
    sp.B = d->batch; sp.Sq = d->sq; sp.Sk = d->sk; sp.H = d->heads;
    sp.R = d->kv_rank; sp.D = d->rope; sp.ld_p = ld_p; sp.P = cdiv(d->sk, kScoreTile);
    sp.inv_scale = 1.0f / (float)scale;
    sp.causal = causal != 0;
    sp.key_stride = key_stride; sp.key_offset = key_offset; sp.sk_total = sk_total;
    sp.seq_lens = seq_lens; sp.block_table = block_table; sp.page_size = page_size;
    sp.max_pages = page_size > 0 ? d->sk / page_size : 0;
    MLA_TRY_HIP(launch_scores(sp, stream), "scores kernel launch");
    return MLA_OK;
}

int check_scale(double scale) {
    if (!(scale > 0.0) || !std::isfinite(scale))
        return fail(MLA_ERR_INVALID_ARGUMENT, "scale must be a positive finite divisor");
    return MLA_OK;
}

// ------------------------------------------------------------------ neighbours of the path

// wkv_b split reads heads, nope, v, kv_rank.
int check_split_dims(mla_dtype_t dt, const mla_dims_t* d) {
    if (!d) return fail(MLA_ERR_INVALID_ARGUMENT, "dims must not be NULL");
    MLA_CHECK(check_pos(d->heads, "dims.heads"));
    MLA_CHECK(check_pos(d->nope, "dims.nope"));
    MLA_CHECK(check_pos(d->v, "dims.v"));
    MLA_CHECK(check_row(dt, d->kv_rank, "dims.kv_rank"));
    if ((int64_t)d->heads * (d->nope + d->v) * (int64_t)d->kv_rank > ((int64_t)1 << 40))
        return fail(MLA_ERR_INVALID_ARGUMENT, "wkv_b too large");
    return MLA_OK;
}

// KV append reads batch, sq, hidden, kv_rank, rope.
int check_kv_dims(mla_dtype_t dt, const mla_dims_t* d) {
    if (!d) return fail(MLA_ERR_INVALID_ARGUMENT, "dims must not be NULL");
    MLA_CHECK(check_pos(d->batch, "dims.batch"));
    MLA_CHECK(check_pos(d->sq, "dims.sq"));
    MLA_CHECK(check_row(dt, d->hidden, "dims.hidden"));
    MLA_CHECK(check_row(dt, d->kv_rank, "dims.kv_rank"));
    MLA_CHECK(check_row(dt, d->rope, "dims.rope"));
    if ((int64_t)d->batch * d->sq * (int64_t)(d->kv_rank + d->rope) > kMaxI32 ||
        (int64_t)d->batch * d->sq * (int64_t)d->hidden > kMaxI32)
        return fail(MLA_ERR_INVALID_ARGUMENT, "batch*sq too large");
    return MLA_OK;
}

// wo reads batch, sq, heads, v, hidden.
int check_oproj_dims(mla_dtype_t dt, const mla_dims_t* d) {
    if (!d) return fail(MLA_ERR_INVALID_ARGUMENT, "dims must not be NULL");
    MLA_CHECK(check_pos(d->batch, "dims.batch"));
    MLA_CHECK(check_pos(d->sq, "dims.sq"));
    MLA_CHECK(check_pos(d->heads, "dims.heads"));
    MLA_CHECK(check_row(dt, d->v, "dims.v"));
    MLA_CHECK(check_row(dt, d->hidden, "dims.hidden"));
    const int64_t bq = (int64_t)d->batch * d->sq;
    if (bq * d->heads * (int64_t)d->v > kMaxI32 || bq * (int64_t)d->hidden > kMaxI32 ||
        (int64_t)d->heads * d->v > kMaxI32 / 8)
        return fail(MLA_ERR_INVALID_ARGUMENT, "batch*sq*heads*v too large");
    return MLA_OK;
}

GemmProblem kv_problem(mla_dtype_t dt, const mla_dims_t* d, const void* x, const void* W,
                       float* C) {
    const int n = d->kv_rank + d->rope;
    GemmProblem p;
    p.half = is_half(dt); p.f16 = is_f16(dt); p.a_f32 = !is_half(dt);
    p.A = x; p.lda = d->hidden;
    p.B = W; p.ldb = n;
    p.C = C; p.ldc = n;
    p.M = d->batch * d->sq; p.N = n; p.K = d->hidden;
    return p;
}

GemmProblem oproj_problem(mla_dtype_t dt, const mla_dims_t* d, const void* attn, const void* W,
                          void* out) {
    const int k = d->heads * d->v;
    GemmProblem p;
    p.half = is_half(dt); p.f16 = is_f16(dt); p.a_f32 = !is_half(dt); p.out_type = storage_out(dt);
    p.A = attn; p.lda = k;
    p.B = W; p.ldb = d->hidden;
    p.C = out; p.ldc = d->hidden;
    p.M = d->batch * d->sq; p.N = d->hidden; p.K = k;
    return p;
}

// x @ W_kv_a lands in one fp32 buffer: the product itself, or its split-K partials for the
// append kernel to sum.
size_t kv_ws_bytes(mla_dtype_t dt, const mla_dims_t* d, GemmPlan* plan_out) {
    const GemmPlan plan = plan_gemm(kv_problem(dt, d, nullptr, nullptr, nullptr));
    if (plan_out) *plan_out = plan;
    return align_up((size_t)std::max(1, plan.split) * d->batch * d->sq *
                    (size_t)(d->kv_rank + d->rope) * sizeof(float));
}

int q_absorbed_f64(const mla_dims_t* d, const void* x, const void* W_q_a, const void* q_norm_w,
                   const void* W_q_b, const void* W_uk, const int64_t* positions,
                   const void* inv_freq, double eps, void* q_absorbed, void* q_rope,
                   void* workspace, size_t workspace_bytes, hipStream_t stream,
                   bool pos_per_batch);

int q_absorbed_impl(mla_dtype_t dtype, const mla_dims_t* dims, const void* x, const void* W_q_a,
                   const void* q_norm_w, const void* W_q_b, const void* W_uk,
                   const int64_t* positions, const void* inv_freq_tab, double eps,
                   void* q_absorbed, void* q_rope, void* workspace, size_t workspace_bytes,
                   hipStream_t stream, bool pos_per_batch) {
    if (dtype == MLA_DTYPE_F64)
        return q_absorbed_f64(dims, x, W_q_a, q_norm_w, W_q_b, W_uk, positions, inv_freq_tab,
                              eps, q_absorbed, q_rope, workspace, workspace_bytes, stream,
                              pos_per_batch);
    const float* inv_freq = static_cast<const float*>(inv_freq_tab);
    MLA_CHECK(check_dtype(dtype));
    MLA_CHECK(check_q_dims(dtype, dims));
    MLA_CHECK(check_ptr(x, "x"));
    MLA_CHECK(check_ptr(W_q_a, "W_q_a"));
    MLA_CHECK(check_ptr(q_norm_w, "q_norm_w"));
    MLA_CHECK(check_ptr(W_q_b, "W_q_b"));
    MLA_CHECK(check_ptr(W_uk, "W_uk"));
    MLA_CHECK(check_ptr(positions, "positions"));
    MLA_CHECK(check_ptr(inv_freq, "inv_freq"));
    MLA_CHECK(check_ptr(q_absorbed, "q_absorbed"));
    MLA_CHECK(check_ptr(q_rope, "q_rope"));
    if (!(eps >= 0.0) || !std::isfinite(eps))
        return fail(MLA_ERR_INVALID_ARGUMENT, "eps must be finite and >= 0");
    const QLayout L = q_layout(dtype, dims);
    MLA_CHECK(check_ws(workspace, workspace_bytes, L.total));

    const int bq = dims->batch * dims->sq;
    float* lat_acc = at<float>(workspace, L.off_lat_acc);
    void* lat = at<void>(workspace, L.off_lat);  // storage dtype
    float* raw = at<float>(workspace, L.off_raw);

    // 2a1: split-K partials land in lat_acc[split][bq][q_lora]; 2a-n sums them.
    GemmProblem down = q_down_problem(dtype, dims, x, W_q_a, lat_acc);
    GemmPlan down_plan = L.down;
    int nsplit = 1;
    if (down_plan.split > 1) {
        nsplit = down_plan.split;
        down_plan.workspace_bytes = 0;
        MLA_TRY_HIP(launch_gemm_partials(down, down_plan, lat_acc, stream), "2a1 launch");
    } else {
        MLA_TRY_HIP(launch_gemm(down, down_plan, nullptr, stream), "2a1 launch");
    }
    // 2a-n (with a fused 2b, also the rows' RoPE cos / sin table)
    const bool small = q_small_ok(dtype, dims, L.up, W_uk, q_absorbed, q_rope);
    const bool rope_epi = L.rope_epi && !small;
    RopeTable rt;
    if (L.fused || rope_epi) {
        rt.cos_sin = at<float>(workspace, L.off_rope_tab);
        rt.positions = positions; rt.inv_freq = inv_freq; rt.half = dims->rope / 2;
        rt.Sq = dims->sq; rt.per_batch = pos_per_batch;
    }
    MLA_TRY_HIP(launch_rmsnorm(lat_acc, nsplit, (int64_t)bq * dims->q_lora, q_norm_w, lat,
                               storage_out(dtype), bq, dims->q_lora, (float)eps, stream, rt),
                "2a-n launch");
    // 2a2, then 2b.  A split-K 2a2 leaves its partials in its workspace and the RoPE kernel
    // sums them (the nope columns into raw for 2c): no reduction launch.  With the fused
    // epilogue 2a2 writes the 16-bit q_nope (into raw's space) and q_rope itself.
    GemmProblem up = q_up_problem(dtype, dims, lat, W_q_b, raw);
    if (L.fused) {
        QUpEpilogue qe;
        qe.q_nope = raw; qe.q_rope = q_rope; qe.cos_sin = rt.cos_sin;
        qe.H = dims->heads; qe.nope = dims->nope; qe.rope = dims->rope;
        up.qup = &qe;
        up.C = nullptr;
        if (L.fused_2c && (reinterpret_cast<uintptr_t>(W_uk) & 15) == 0 &&
            (reinterpret_cast<uintptr_t>(q_absorbed) & 3) == 0) {
            qe.w_uk = W_uk; qe.q_abs = q_absorbed; qe.kv = dims->kv_rank;
            MLA_TRY_HIP(launch_gemm(up, L.up, at<void>(workspace, L.off_up_ws), stream),
                        "2a2 + 2b + 2c launch");
            return ok();
        }
        MLA_TRY_HIP(launch_gemm(up, L.up, at<void>(workspace, L.off_up_ws), stream),
                    "2a2 + 2b launch");
        GemmProblem ab = absorb_problem(dtype, dims, raw, W_uk, q_absorbed, true);
        MLA_TRY_HIP(launch_gemm(ab, L.absorb, at<void>(workspace, L.off_abs_ws), stream),
                    "2c launch");
        return ok();
    }
    if (L.up.split > 1) {
        float* up_parts = at<float>(workspace, L.off_up_ws);
        MLA_TRY_HIP(launch_gemm_partials(up, L.up, up_parts, stream), "2a2 launch");
        if (small) {
            MLA_TRY_HIP(launch_q_small(up_parts, L.up.split,
                                       (int64_t)bq * dims->heads * (dims->nope + dims->rope),
                                       positions, inv_freq, static_cast<const float*>(W_uk),
                                       static_cast<float*>(q_rope),
                                       static_cast<float*>(q_absorbed), dims->batch, dims->sq,
                                       dims->heads, dims->nope, dims->rope, dims->kv_rank,
                                       pos_per_batch, stream),
                        "2b + 2c launch");
            return ok();
        }
        MLA_TRY_HIP(launch_rope(up_parts, positions, inv_freq, q_rope, storage_out(dtype),
                                dims->batch, dims->sq, dims->heads, dims->nope, dims->rope,
                                stream, pos_per_batch, L.up.split,
                                (int64_t)bq * dims->heads * (dims->nope + dims->rope), raw),
                    "2b launch");
    } else if (rope_epi) {
        QUpEpilogue re;
        re.q_rope = q_rope; re.cos_sin = rt.cos_sin;
        re.H = dims->heads; re.nope = dims->nope; re.rope = dims->rope;
        up.rope_epi = &re;
        MLA_TRY_HIP(launch_gemm(up, L.up, at<void>(workspace, L.off_up_ws), stream),
                    "2a2 + 2b launch");
    } else {
        MLA_TRY_HIP(launch_gemm(up, L.up, at<void>(workspace, L.off_up_ws), stream), "2a2 launch");
        if (small) {
            MLA_TRY_HIP(launch_q_small(raw, 1, 0, positions, inv_freq,
                                       static_cast<const float*>(W_uk),
                                       static_cast<float*>(q_rope),
                                       static_cast<float*>(q_absorbed), dims->batch, dims->sq,
                                       dims->heads, dims->nope, dims->rope, dims->kv_rank,
                                       pos_per_batch, stream),
                        "2b + 2c launch");
            return ok();
        }
        MLA_TRY_HIP(launch_rope(raw, positions, inv_freq, q_rope, storage_out(dtype), dims->batch,
                                dims->sq, dims->heads, dims->nope, dims->rope, stream,
                                pos_per_batch),
                    "2b launch");
    }
    // 2c
    GemmProblem ab = absorb_problem(dtype, dims, raw, W_uk, q_absorbed);
    MLA_TRY_HIP(launch_gemm(ab, L.absorb, at<void>(workspace, L.off_abs_ws), stream),
                "2c launch");
    return ok();
}

// Paged cache: page_size a positive multiple of 64 that divides dims->sk (the table span).
int check_pages(const mla_dims_t* d, int32_t page_size) {
    if (page_size <= 0 || page_size % 64 != 0)
        return fail(MLA_ERR_INVALID_ARGUMENT, "page_size must be a positive multiple of 64 (got %d)",
                    page_size);
    if (d->sk <= 0 || d->sk % page_size != 0)
        return fail(MLA_ERR_INVALID_ARGUMENT,
                    "dims.sk must be max_pages * page_size, a positive multiple of page_size "
                    "(got sk=%d, page_size=%d)", d->sk, page_size);
    return MLA_OK;
}

// KV append: x @ W_kv_a into the workspace, then the fused norm / RoPE / scatter kernel.
// Dense: rows start_row + s of a [B, cache_rows] cache.  Paged (block_table): the rows of
// slots positions[b*Sq + s] through the table.
int kv_append_impl(mla_dtype_t dtype, const mla_dims_t* dims, const void* x, const void* W_kv_a,
                   const void* kv_norm_w, const int64_t* positions, const float* inv_freq,
                   double eps, int32_t start_row, int32_t cache_rows, const int32_t* block_table,
                   int32_t page_size, void* c_kv, void* pe_cache, void* workspace,
                   size_t workspace_bytes, hipStream_t stream) {
    MLA_CHECK(check_dtype(dtype));
    MLA_CHECK(check_kv_dims(dtype, dims));
    MLA_CHECK(check_ptr(x, "x"));
    MLA_CHECK(check_ptr(W_kv_a, "W_kv_a"));
    MLA_CHECK(check_ptr(kv_norm_w, "kv_norm_w"));
    MLA_CHECK(check_ptr(positions, "positions"));
    MLA_CHECK(check_ptr(inv_freq, "inv_freq"));
    MLA_CHECK(check_ptr(c_kv, block_table ? "c_kv_pages" : "c_kv"));
    MLA_CHECK(check_ptr(pe_cache, block_table ? "pe_pages" : "pe_cache"));
    if (!(eps >= 0.0) || !std::isfinite(eps))
        return fail(MLA_ERR_INVALID_ARGUMENT, "eps must be finite and >= 0");
    int max_pages = 0;
    if (block_table) {
        MLA_CHECK(check_pages(dims, page_size));
        max_pages = dims->sk / page_size;
    } else {
        if (cache_rows <= 0 || start_row < 0 || (int64_t)start_row + dims->sq > cache_rows)
            return fail(MLA_ERR_INVALID_ARGUMENT,
                        "cache rows [start_row, start_row + sq) = [%d, %lld) must lie in [0, %d)",
                        start_row, (long long)start_row + dims->sq, cache_rows);
        if ((int64_t)dims->batch * cache_rows * (int64_t)dims->kv_rank > ((int64_t)1 << 40))
            return fail(MLA_ERR_INVALID_ARGUMENT, "cache too large");
    }
    GemmPlan plan;
    const size_t need = kv_ws_bytes(dtype, dims, &plan);
    MLA_CHECK(check_ws(workspace, workspace_bytes, need));

    const int bq = dims->batch * dims->sq;
    const int n = dims->kv_rank + dims->rope;
    float* acc = at<float>(workspace, 0);
    GemmProblem gp = kv_problem(dtype, dims, x, W_kv_a, acc);
    int nsplit = 1;
    if (plan.split > 1) {
        nsplit = plan.split;
        plan.workspace_bytes = 0;
        MLA_TRY_HIP(launch_gemm_partials(gp, plan, acc, stream), "kv GEMM launch");
    } else {
        MLA_TRY_HIP(launch_gemm(gp, plan, nullptr, stream), "kv GEMM launch");
    }
    MLA_TRY_HIP(launch_kv_append(acc, nsplit, (int64_t)bq * n, kv_norm_w, positions, inv_freq,
                                 c_kv, pe_cache, storage_out(dtype), dims->batch, dims->sq,
                                 dims->kv_rank, dims->rope, start_row, cache_rows, (float)eps,
                                 stream, block_table != nullptr, block_table, page_size,
                                 max_pages),
                "kv append launch");
    return ok();
}

// ------------------------------------------------------------------ allocation-free attention
//
// mla_attention_noalloc takes its workspace from `scratch`, a device array of this file,
// instead of a caller buffer.  Each GPU holds its own copy of the array (at its own
// address) from the library's load until the process ends.  In host code `scratch` is a
// host-side stand-in for the symbol: its device address comes from hipGetSymbolAddress,
// looked up once per device with that device current, and only that address is handed to
// the kernels.  Every call on one GPU shares the array, so calls that overlap on one GPU
// (two streams, two host threads) race; the kernels write every scratch byte they read
// before reading it, so nothing needs clearing between calls.
constexpr size_t kScratchBytes = MLA_ATTENTION_NOALLOC_MAX_BYTES;
static __device__ __align__(256) uint8_t scratch[kScratchBytes];

constexpr int kMaxDevices = 64;
std::mutex g_scratch_mu;
void* g_scratch_ptr[kMaxDevices] = {};

// The scratch address on the device that `stream` belongs to (the current device for the
// null stream).
int scratch_for_stream(hipStream_t stream, void** out) {
    int cur = 0, dev = 0;
    MLA_TRY_HIP(hipGetDevice(&cur), "hipGetDevice");
    dev = cur;
    if (stream) MLA_TRY_HIP(hipStreamGetDevice(stream, &dev), "hipStreamGetDevice");
    if (dev < 0 || dev >= kMaxDevices)
        return fail(MLA_ERR_UNSUPPORTED, "device %d is beyond the %d devices the scratch table "
                    "covers", dev, kMaxDevices);
    std::lock_guard<std::mutex> lock(g_scratch_mu);
    if (!g_scratch_ptr[dev]) {
        // The first call on a device may come while the caller captures `stream` into a
        // graph.  The lookup enqueues nothing, but it can load the code object, which
        // strict capture modes refuse; this thread runs it in relaxed mode and restores
        // the caller's mode afterwards.
        hipStreamCaptureMode mode = hipStreamCaptureModeRelaxed;
        MLA_TRY_HIP(hipThreadExchangeStreamCaptureMode(&mode), "capture mode (relax)");
        hipError_t e = hipSuccess;
        void* p = nullptr;
        if (dev != cur) e = hipSetDevice(dev);
        if (e == hipSuccess) e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
        const hipError_t e_back = dev != cur ? hipSetDevice(cur) : hipSuccess;
        const hipError_t e_mode = hipThreadExchangeStreamCaptureMode(&mode);
        if (e != hipSuccess) return hip_fail(e, "scratch symbol lookup");
        if (e_back != hipSuccess) return hip_fail(e_back, "hipSetDevice (restore)");
        if (e_mode != hipSuccess) return hip_fail(e_mode, "capture mode (restore)");
        if (!p) return fail(MLA_ERR_HIP, "scratch symbol lookup returned NULL");
        g_scratch_ptr[dev] = p;
    }
    *out = g_scratch_ptr[dev];
    return MLA_OK;
}

// ------------------------------------------------------------------ float64 (f64.hip)
//
// The reference's double dispatch (mla_kernels.cu:674, 1561) with double intermediates
// (:118-120): the per-step decomposition in double on the double-MFMA GEMM.  Shapes only
// need to be positive (rope even); the grids put M / 64 in y and the batch in z, which
// bounds those at 65535.

int check_f64_grid(int64_t m, int64_t g, const char* what) {
    if ((m + 63) / 64 > 65535 || g > 65535)
        return fail(MLA_ERR_UNSUPPORTED, "float64 %s: %lld rows in %lld groups is past the "
                    "grid's limits (65535 row tiles of 64, 65535 groups)", what, (long long)m,
                    (long long)g);
    return MLA_OK;
}

int check_f64_q_dims(const mla_dims_t* d) {
    if (!d) return fail(MLA_ERR_INVALID_ARGUMENT, "dims must not be NULL");
    MLA_CHECK(check_pos(d->batch, "dims.batch"));
    MLA_CHECK(check_pos(d->sq, "dims.sq"));
    MLA_CHECK(check_pos(d->heads, "dims.heads"));
    MLA_CHECK(check_pos(d->hidden, "dims.hidden"));
    MLA_CHECK(check_pos(d->q_lora, "dims.q_lora"));
    MLA_CHECK(check_pos(d->nope, "dims.nope"));
    MLA_CHECK(check_pos(d->kv_rank, "dims.kv_rank"));
    if (d->rope <= 0 || d->rope % 2 != 0)
        return fail(MLA_ERR_INVALID_ARGUMENT, "dims.rope must be positive and even (got %d)",
                    d->rope);
    const int64_t bq = (int64_t)d->batch * d->sq;
    if (bq * d->heads * (int64_t)(d->nope + d->rope) > kMaxI32)
        return fail(MLA_ERR_INVALID_ARGUMENT, "batch*sq*heads too large");
    return check_f64_grid(bq, d->heads, "Q path");
}

int check_f64_attn_dims(const mla_dims_t* d, int causal) {
    if (!d) return fail(MLA_ERR_INVALID_ARGUMENT, "dims must not be NULL");
    MLA_CHECK(check_pos(d->batch, "dims.batch"));
    MLA_CHECK(check_pos(d->sq, "dims.sq"));
    MLA_CHECK(check_pos(d->sk, "dims.sk"));
    MLA_CHECK(check_pos(d->heads, "dims.heads"));
    MLA_CHECK(check_pos(d->rope, "dims.rope"));
    MLA_CHECK(check_pos(d->kv_rank, "dims.kv_rank"));
    MLA_CHECK(check_pos(d->v, "dims.v"));
    if (causal && d->sk < d->sq)
        return fail(MLA_ERR_INVALID_ARGUMENT,
                    "causal attention needs sk >= sq (got sk=%d, sq=%d)", d->sk, d->sq);
    const int64_t rows_b = (int64_t)d->sq * d->heads;
    if (rows_b * d->batch > kMaxI32 / 2)
        return fail(MLA_ERR_INVALID_ARGUMENT, "batch*sq*heads too large");
    MLA_CHECK(check_f64_grid(rows_b, d->batch, "scores"));
    return check_f64_grid((int64_t)d->batch * d->sq, d->heads, "output");
}

struct QLayout64 { size_t off_lat, off_raw, total; };
QLayout64 q_layout64(const mla_dims_t* d) {
    QLayout64 L;
    const size_t bq = (size_t)d->batch * d->sq;
    size_t o = 0;
    L.off_lat = o; o = align_up(o + bq * d->q_lora * sizeof(double));
    L.off_raw = o; o = align_up(o + bq * d->heads * (size_t)(d->nope + d->rope) * sizeof(double));
    L.total = o;
    return L;
}

struct AttnLayout64 { size_t off_s, off_ctx, total; };
AttnLayout64 attn_layout64(const mla_dims_t* d) {
    AttnLayout64 L;
    const size_t rows = (size_t)d->batch * d->sq * d->heads;
    size_t o = 0;
    L.off_s = o;   o = align_up(o + rows * (size_t)d->sk * sizeof(double));
    L.off_ctx = o; o = align_up(o + rows * (size_t)d->kv_rank * sizeof(double));
    L.total = o;
    return L;
}

// 2a1 -> 2a-n -> 2a2 -> 2b -> 2c in double; inv_freq is a double table
int q_absorbed_f64(const mla_dims_t* d, const void* x, const void* W_q_a, const void* q_norm_w,
                   const void* W_q_b, const void* W_uk, const int64_t* positions,
                   const void* inv_freq, double eps, void* q_absorbed, void* q_rope,
                   void* workspace, size_t workspace_bytes, hipStream_t stream,
                   bool pos_per_batch) {
    MLA_CHECK(check_f64_q_dims(d));
    MLA_CHECK(check_ptr(x, "x"));
    MLA_CHECK(check_ptr(W_q_a, "W_q_a"));
    MLA_CHECK(check_ptr(q_norm_w, "q_norm_w"));
    MLA_CHECK(check_ptr(W_q_b, "W_q_b"));
    MLA_CHECK(check_ptr(W_uk, "W_uk"));
    MLA_CHECK(check_ptr(positions, "positions"));
    MLA_CHECK(check_ptr(inv_freq, "inv_freq"));
    MLA_CHECK(check_ptr(q_absorbed, "q_absorbed"));
    MLA_CHECK(check_ptr(q_rope, "q_rope"));
    if (!(eps >= 0.0) || !std::isfinite(eps))
        return fail(MLA_ERR_INVALID_ARGUMENT, "eps must be finite and >= 0");
    const QLayout64 L = q_layout64(d);
    MLA_CHECK(check_ws(workspace, workspace_bytes, L.total));
    double* lat = at<double>(workspace, L.off_lat);
    double* raw = at<double>(workspace, L.off_raw);
    const int bq = d->batch * d->sq;
    const int qk = d->nope + d->rope;
    const int64_t n_raw = (int64_t)d->heads * qk;
    // 2a1: lat [bq, q_lora] = x [bq, hidden] . W_q_a [hidden, q_lora]
    Gemm64Problem p;
    p.A = static_cast<const double*>(x); p.lda = d->hidden;
    p.B = static_cast<const double*>(W_q_a); p.ldb = d->q_lora;
    p.C = lat; p.ldc = d->q_lora;
    p.M = bq; p.N = d->q_lora; p.K = d->hidden;
    MLA_TRY_HIP(launch_gemm64(p, stream), "2a1 launch (f64)");
    // 2a-n, in place
    MLA_TRY_HIP(launch_rmsnorm64(lat, static_cast<const double*>(q_norm_w), bq, d->q_lora, eps,
                                 stream), "2a-n launch (f64)");
    // 2a2: raw [bq, H*(nope+rope)] = lat . W_q_b
    p = Gemm64Problem();
    p.A = lat; p.lda = d->q_lora;
    p.B = static_cast<const double*>(W_q_b); p.ldb = n_raw;
    p.C = raw; p.ldc = n_raw;
    p.M = bq; p.N = (int)n_raw; p.K = d->q_lora;
    MLA_TRY_HIP(launch_gemm64(p, stream), "2a2 launch (f64)");
    // 2b
    MLA_TRY_HIP(launch_rope64(raw, positions, static_cast<const double*>(inv_freq),
                              static_cast<double*>(q_rope), d->batch, d->sq, d->heads, d->nope,
                              d->rope, pos_per_batch, stream), "2b launch (f64)");
    // 2c, one group per head: q_absorbed[m, h, :] = raw[m, h*qk : h*qk+nope] . W_uk[h]
    p = Gemm64Problem();
    p.A = raw; p.lda = n_raw; p.sA = qk;
    p.B = static_cast<const double*>(W_uk); p.ldb = d->kv_rank; p.sB = (int64_t)d->nope * d->kv_rank;
    p.C = static_cast<double*>(q_absorbed); p.ldc = (int64_t)d->heads * d->kv_rank;
    p.sC = d->kv_rank;
    p.M = bq; p.N = d->kv_rank; p.K = d->nope; p.G = d->heads;
    MLA_TRY_HIP(launch_gemm64(p, stream), "2c launch (f64)");
    return ok();
}

// 3a -> softmax -> 3c -> 3d in double
int attention_f64(const mla_dims_t* d, const void* q_absorbed, const void* q_rope,
                  const void* c_kv, const void* pe_cache, const void* W_uv, double scale,
                  int causal, void* out, void* workspace, size_t workspace_bytes,
                  hipStream_t stream) {
    MLA_CHECK(check_f64_attn_dims(d, causal));
    MLA_CHECK(check_scale(scale));
    MLA_CHECK(check_ptr(q_absorbed, "q_absorbed"));
    MLA_CHECK(check_ptr(q_rope, "q_rope"));
    MLA_CHECK(check_ptr(c_kv, "c_kv"));
    MLA_CHECK(check_ptr(pe_cache, "pe_cache"));
    MLA_CHECK(check_ptr(W_uv, "W_uv"));
    MLA_CHECK(check_ptr(out, "out"));
    const AttnLayout64 L = attn_layout64(d);
    MLA_CHECK(check_ws(workspace, workspace_bytes, L.total));
    double* S = at<double>(workspace, L.off_s);
    double* ctx = at<double>(workspace, L.off_ctx);
    const int rows_b = d->sq * d->heads;
    const int64_t R = d->kv_rank, Dr = d->rope, Sk = d->sk;
    const double* ckv = static_cast<const double*>(c_kv);
    // 3a: S[b] = q_absorbed[b] . c_kv[b]^T, then += q_rope[b] . pe[b]^T  ([rows_b, Sk])
    Gemm64Problem p;
    p.A = static_cast<const double*>(q_absorbed); p.lda = R; p.sA = rows_b * R;
    p.B = ckv; p.ldb = R; p.sB = Sk * R; p.b_nt = true;
    p.C = S; p.ldc = Sk; p.sC = rows_b * Sk;
    p.M = rows_b; p.N = d->sk; p.K = d->kv_rank; p.G = d->batch;
    MLA_TRY_HIP(launch_gemm64(p, stream), "3a launch (f64)");
    p.A = static_cast<const double*>(q_rope); p.lda = Dr; p.sA = rows_b * Dr;
    p.B = static_cast<const double*>(pe_cache); p.ldb = Dr; p.sB = Sk * Dr;
    p.K = d->rope; p.beta = 1.0;
    MLA_TRY_HIP(launch_gemm64(p, stream), "3a rope launch (f64)");
    // 3b: softmax of S / scale over each row's visible keys
    MLA_TRY_HIP(launch_softmax64(S, d->batch * rows_b, d->sk, d->sq, d->heads, scale,
                                 causal != 0, stream), "softmax launch (f64)");
    // 3c: ctx[b] = P[b] . c_kv[b]  ([rows_b, R])
    p = Gemm64Problem();
    p.A = S; p.lda = Sk; p.sA = rows_b * Sk;
    p.B = ckv; p.ldb = R; p.sB = Sk * R;
    p.C = ctx; p.ldc = R; p.sC = rows_b * R;
    p.M = rows_b; p.N = d->kv_rank; p.K = d->sk; p.G = d->batch;
    MLA_TRY_HIP(launch_gemm64(p, stream), "3c launch (f64)");
    // 3d, one group per head: out[m, h, :] = ctx[m, h, :] . W_uv[h]^T
    p = Gemm64Problem();
    p.A = ctx; p.lda = (int64_t)d->heads * R; p.sA = R;
    p.B = static_cast<const double*>(W_uv); p.ldb = R; p.sB = (int64_t)d->v * R; p.b_nt = true;
    p.C = static_cast<double*>(out); p.ldc = (int64_t)d->heads * d->v; p.sC = d->v;
    p.M = d->batch * d->sq; p.N = d->v; p.K = d->kv_rank; p.G = d->heads;
    MLA_TRY_HIP(launch_gemm64(p, stream), "3d launch (f64)");
    return ok();
}

// fp8 KV cache (mla_attention_fp8kv)

struct Fp8Layout {
    FlashPlan flash;
    GemmPlan out;
    bool ctx16 = false;   // the pass writes the normalised bf16 ctx for 3d
    size_t off_rowsum, off_ctx, off_out_ws, off_part, total;
};

FlashProblem fp8_problem(const mla_dims_t* d, const void* qa, const void* qr, const void* ckv,
                         const void* pe, float kv_scale, double scale, int causal) {
    FlashProblem p = flash_problem(MLA_DTYPE_BF16, d, qa, qr, ckv, pe, scale, causal);
    p.fp8_kv = true;
    p.kv_scale = kv_scale;
    return p;
}

// ragged: the paged pool's plan (the balanced work list and its partial slots)
Fp8Layout fp8_layout(const mla_dims_t* d, bool ragged = false) {
    Fp8Layout L;
    const size_t rows = (size_t)d->batch * d->sq * d->heads;
    FlashProblem fp = fp8_problem(d, nullptr, nullptr, nullptr, nullptr, 1.f, 1.0, 0);
    fp.ragged = ragged;
    L.flash = plan_flash(fp);
    L.ctx16 = flash_ctx16_ok(fp, L.flash);
    L.out = L.ctx16 ? plan_gemm(out_problem16(MLA_DTYPE_BF16, d, nullptr, nullptr, nullptr))
                    : plan_gemm(out_problem(MLA_DTYPE_BF16, d, nullptr, nullptr, nullptr, nullptr));
    size_t o = 0;
    L.off_rowsum = o; o = align_up(o + rows * sizeof(float));
    L.off_ctx = o;    o = align_up(o + rows * d->kv_rank * sizeof(float));
    L.off_out_ws = o; o = align_up(o + L.out.workspace_bytes);
    L.off_part = o;   o = align_up(o + L.flash.partial_bytes);
    L.total = o;
    return L;
}

int check_fp8_attn(mla_dtype_t dtype, const mla_dims_t* dims, int causal, float kv_scale) {
    if (dtype != MLA_DTYPE_BF16)
        return fail(MLA_ERR_UNSUPPORTED, "an fp8 cache is read with bf16 queries (dtype %d)",
                    (int)dtype);
    MLA_CHECK(check_attn_dims(dtype, dims, causal));
    if (!(kv_scale > 0.f) || !std::isfinite(kv_scale))
        return fail(MLA_ERR_INVALID_ARGUMENT, "kv_scale must be positive and finite");
    // the cache rows are bytes: the fused pass reads whole 16-byte chunks
    if (dims->kv_rank % 16 != 0 || dims->rope % 16 != 0)
        return fail(MLA_ERR_INVALID_ARGUMENT, "fp8 cache rows must be multiples of 16 bytes");
    if (!flash_supported(fp8_problem(dims, nullptr, nullptr, nullptr, nullptr, kv_scale, 1.0, causal)))
        return fail(MLA_ERR_UNSUPPORTED, "an fp8 cache needs kv_rank 512 and rope 64");
    // the fused pass forms 32-bit per-lane buffer offsets within one sequence: its query
    // rows (bf16, 1 KiB each) and its dense cache rows (one byte per element) must span less
    // than 2^31 bytes -- the bound flash_eligible puts on the 16-bit path, which has the
    // per-step path to fall back on; the fp8 cache has none
    constexpr int64_t kRange = 0x7fffffff;
    if ((int64_t)dims->sq * dims->heads * dims->kv_rank * 2 >= kRange ||
        (int64_t)dims->sk * dims->kv_rank >= kRange)
        return fail(MLA_ERR_UNSUPPORTED, "an fp8-cache call needs Sq * heads * kv_rank * 2 and "
                    "Sk * kv_rank below 2^31 bytes (Sq %d, heads %d, Sk %d)", dims->sq,
                    dims->heads, dims->sk);
    return MLA_OK;
}

// fp32 decode-sized batches on the fused path: 3d with the split merge folded in, where it
// measured faster (B=1, Sk=4989: attention with 3d 43.1 against 49.1 us; B=2, 3: 56.8 / 74.8
// against 60.4 / 77.4 us; B=4, Sk=512: 36.0 against 37.7 us; B=4, Sk=4989 with 32 splits:
// 99.0 against 91.3 us, so not there)
// Returns 1 for out_small_kernel with the merge folded in (or an unsplit pass), 2 for the
// merge kernel followed by out_small_kernel on the merged ctx / row_sum (the other split
// passes up to B*Sq = 8: 0.5-2.7 us ahead of the merge kernel and the 3d GEMM at B = 5..8,
// Sk = 512..16384), 0 for the 3d GEMM.
int out_small_mode(mla_dtype_t dtype, const mla_dims_t* d, const FlashPlan& plan) {
    const char* env = std::getenv("MLA_OUT_SMALL");
    if (env && env[0] == '0') return 0;
    const int64_t M = (int64_t)d->batch * d->sq;
    if (is_half(dtype) || plan.balanced || M > kOutSmallRows || d->kv_rank != 512) return 0;
    if (plan.n_split <= 1) return 1;
    if (plan.n_split <= kOutSmallMaxSplit && M * plan.n_split <= kOutSmallMergeRows &&
        M <= kOutSmallMergeM)
        return 1;
    return 2;
}

}  // namespace

// ====================================================================== C ABI
// The library is built with -fvisibility=hidden; only this block is exported.

#pragma GCC visibility push(default)
extern "C" {

const char* mla_last_error(void) { return g_last_error.c_str(); }
const char* mla_version(void) { return "mla_amd 0.1.0 (gfx950)"; }
int32_t mla_score_tile(void) { return kScoreTile; }
int32_t mla_score_ld(int32_t sk) { return sk <= 0 ? 0 : ((sk + 31) / 32) * 32; }

size_t mla_gemm_workspace_bytes(mla_dtype_t dtype, int32_t M, int32_t N, int32_t K) {
    if (M <= 0 || N <= 0 || K <= 0 || check_dtype(dtype) != MLA_OK) return 0;
    GemmProblem p;   // mla_gemm's problem, without the pointers
    p.lda = K; p.ldb = N; p.ldc = N;
    p.M = M; p.N = N; p.K = K;
    p.half = is_half(dtype); p.f16 = is_f16(dtype); p.a_f32 = !is_half(dtype);
    return plan_gemm(p).workspace_bytes;
}

int mla_gemm(mla_dtype_t dtype, const void* A, const void* W, float* C, int32_t M, int32_t N,
             int32_t K, void* workspace, size_t workspace_bytes, hipStream_t stream) {
    MLA_CHECK(check_dtype(dtype));
    MLA_CHECK(check_pos(M, "M"));
    MLA_CHECK(check_row(dtype, N, "N"));
    MLA_CHECK(check_row(dtype, K, "K"));
    MLA_CHECK(check_ptr(A, "A"));
    MLA_CHECK(check_ptr(W, "W"));
    MLA_CHECK(check_ptr(C, "C"));
    GemmProblem p;
    p.A = A; p.lda = K;
    p.B = W; p.ldb = N;
    p.half = is_half(dtype); p.f16 = is_f16(dtype); p.a_f32 = !is_half(dtype);
    p.C = C; p.ldc = N;
    p.M = M; p.N = N; p.K = K;
    const GemmPlan plan = plan_gemm(p);
    MLA_CHECK(check_ws(workspace, workspace_bytes, plan.workspace_bytes));
    MLA_TRY_HIP(launch_gemm(p, plan, workspace, stream), "gemm launch");
    return ok();
}

int mla_rmsnorm(mla_dtype_t dtype, const float* in, const void* gain, void* out, int32_t M,
                int32_t N, double eps, hipStream_t stream) {
    MLA_CHECK(check_dtype(dtype));
    MLA_CHECK(check_pos(M, "M"));
    MLA_CHECK(check_mult4(N, "N"));
    MLA_CHECK(check_ptr(in, "in"));
    MLA_CHECK(check_ptr(gain, "gain"));
    MLA_CHECK(check_ptr(out, "out"));
    if (!(eps >= 0.0) || !std::isfinite(eps))
        return fail(MLA_ERR_INVALID_ARGUMENT, "eps must be finite and >= 0");
    MLA_TRY_HIP(launch_rmsnorm(in, 1, 0, gain, out, storage_out(dtype), M, N, (float)eps, stream),
                "rmsnorm launch");
    return ok();
}

int mla_rope(mla_dtype_t dtype, const mla_dims_t* dims, const float* q_raw,
             const int64_t* positions, const float* inv_freq, void* q_rope,
             hipStream_t stream) {
    MLA_CHECK(check_dtype(dtype));
    MLA_CHECK(check_qraw_dims(dtype, dims, false));
    MLA_CHECK(check_ptr(q_raw, "q_raw"));
    MLA_CHECK(check_ptr(positions, "positions"));
    MLA_CHECK(check_ptr(inv_freq, "inv_freq"));
    MLA_CHECK(check_ptr(q_rope, "q_rope"));
    MLA_TRY_HIP(launch_rope(q_raw, positions, inv_freq, q_rope, storage_out(dtype), dims->batch,
                            dims->sq, dims->heads, dims->nope, dims->rope, stream),
                "rope launch");
    return ok();
}

int mla_absorb(mla_dtype_t dtype, const mla_dims_t* dims, const float* q_raw,
               const void* W_uk, void* q_absorbed, hipStream_t stream) {
    MLA_CHECK(check_dtype(dtype));
    MLA_CHECK(check_qraw_dims(dtype, dims, true));
    MLA_CHECK(check_ptr(q_raw, "q_raw"));
    MLA_CHECK(check_ptr(W_uk, "W_uk"));
    MLA_CHECK(check_ptr(q_absorbed, "q_absorbed"));
    GemmProblem p = absorb_problem(dtype, dims, q_raw, W_uk, q_absorbed);
    const GemmPlan plan = plan_gemm(p);
    if (plan.workspace_bytes)
        return fail(MLA_ERR_UNSUPPORTED, "absorb at this shape needs split-K; use mla_q_absorbed");
    MLA_TRY_HIP(launch_gemm(p, plan, nullptr, stream), "absorb launch");
    return ok();
}

int mla_scores(mla_dtype_t dtype, const mla_dims_t* dims, const void* q_absorbed,
               const void* q_rope, const void* c_kv, const void* pe_cache, double scale,
               int causal, float* scores, int32_t ld_scores, float* m_part, float* l_part,
               hipStream_t stream) {
    MLA_CHECK(check_dtype(dtype));
    MLA_CHECK(check_attn_dims(dtype, dims, causal));
    MLA_CHECK(check_scale(scale));
    MLA_CHECK(check_ptr(q_absorbed, "q_absorbed"));
    MLA_CHECK(check_ptr(q_rope, "q_rope"));
    MLA_CHECK(check_ptr(c_kv, "c_kv"));
    MLA_CHECK(check_ptr(pe_cache, "pe_cache"));
    MLA_CHECK(check_ptr(scores, "scores"));
    MLA_CHECK(check_ptr(m_part, "m_part"));
    MLA_CHECK(check_ptr(l_part, "l_part"));
    if (ld_scores < mla_score_ld(dims->sk) || ld_scores % 4 != 0)
        return fail(MLA_ERR_INVALID_ARGUMENT,
                    "ld_scores must be a multiple of 4 and >= mla_score_ld(sk)=%d (got %d)",
                    mla_score_ld(dims->sk), ld_scores);
    MLA_CHECK(run_scores(dtype, dims, q_absorbed, q_rope, c_kv, pe_cache, scale, causal, scores,
                         ld_scores, m_part, l_part, stream));
    return ok();
}

int mla_combine(const float* m_part, const float* l_part, float* alpha, float* row_sum,
                int32_t rows, int32_t n_partials, hipStream_t stream) {
    MLA_CHECK(check_pos(rows, "rows"));
    MLA_CHECK(check_pos(n_partials, "n_partials"));
    MLA_CHECK(check_ptr(m_part, "m_part"));
    MLA_CHECK(check_ptr(l_part, "l_part"));
    MLA_CHECK(check_ptr(alpha, "alpha"));
    MLA_CHECK(check_ptr(row_sum, "row_sum"));
    MLA_TRY_HIP(launch_combine(m_part, l_part, alpha, row_sum, nullptr, rows, n_partials, stream),
                "combine launch");
    return ok();
}

size_t mla_ctx_workspace_bytes(mla_dtype_t dtype, const mla_dims_t* dims) {
    if (!dims || check_ctx_dims(dtype, dims) != MLA_OK) return 0;
    return plan_gemm(ctx_problem(dtype, dims, nullptr, mla_score_ld(dims->sk), nullptr, nullptr,
                                 nullptr)).workspace_bytes;
}

int mla_ctx(mla_dtype_t dtype, const mla_dims_t* dims, const float* scores, int32_t ld_scores,
            const float* alpha, const void* c_kv, float* ctx, void* workspace,
            size_t workspace_bytes, hipStream_t stream) {
    MLA_CHECK(check_dtype(dtype));
    MLA_CHECK(check_ctx_dims(dtype, dims));
    MLA_CHECK(check_ptr(scores, "scores"));
    MLA_CHECK(check_ptr(alpha, "alpha"));
    MLA_CHECK(check_ptr(c_kv, "c_kv"));
    MLA_CHECK(check_ptr(ctx, "ctx"));
    if (ld_scores < mla_score_ld(dims->sk) || ld_scores % 4 != 0)
        return fail(MLA_ERR_INVALID_ARGUMENT,
                    "ld_scores must be a multiple of 4 and >= mla_score_ld(sk)=%d (got %d)",
                    mla_score_ld(dims->sk), ld_scores);
    GemmProblem p = ctx_problem(dtype, dims, scores, ld_scores, alpha, c_kv, ctx);
    const GemmPlan plan = plan_gemm(p);
    MLA_CHECK(check_ws(workspace, workspace_bytes, plan.workspace_bytes));
    MLA_TRY_HIP(launch_gemm(p, plan, workspace, stream), "ctx launch");
    return ok();
}

size_t mla_attn_ctx_workspace_bytes(mla_dtype_t dtype, const mla_dims_t* dims, int causal) {
    if (!dims || check_attn_dims(dtype, dims, causal) != MLA_OK) return 0;
    if (!flash_eligible(dtype, dims)) return 0;
    return align_up(plan_flash(flash_problem(dtype, dims, nullptr, nullptr, nullptr, nullptr, 1.0,
                                             causal)).partial_bytes);
}

int mla_attn_ctx(mla_dtype_t dtype, const mla_dims_t* dims, const void* q_absorbed,
                 const void* q_rope, const void* c_kv, const void* pe_cache, double scale,
                 int causal, float* ctx, float* row_sum, void* workspace,
                 size_t workspace_bytes, hipStream_t stream) {
    MLA_CHECK(check_dtype(dtype));
    MLA_CHECK(check_attn_dims(dtype, dims, causal));
    MLA_CHECK(check_scale(scale));
    if (!flash_eligible(dtype, dims))
        return fail(MLA_ERR_UNSUPPORTED,
                    "fused attention needs kv_rank 512 and rope 64 (got %d, %d)",
                    dims->kv_rank, dims->rope);
    MLA_CHECK(check_ptr(q_absorbed, "q_absorbed"));
    MLA_CHECK(check_ptr(q_rope, "q_rope"));
    MLA_CHECK(check_ptr(c_kv, "c_kv"));
    MLA_CHECK(check_ptr(pe_cache, "pe_cache"));
    MLA_CHECK(check_ptr(ctx, "ctx"));
    MLA_CHECK(check_ptr(row_sum, "row_sum"));
    const FlashProblem fp =
        flash_problem(dtype, dims, q_absorbed, q_rope, c_kv, pe_cache, scale, causal);
    const FlashPlan plan = plan_flash(fp);
    MLA_CHECK(check_ws(workspace, workspace_bytes, align_up(plan.partial_bytes)));
    MLA_TRY_HIP(launch_flash(fp, plan, ctx, row_sum, static_cast<float*>(workspace), stream),
                "fused attention launch");
    return ok();
}

size_t mla_out_workspace_bytes(mla_dtype_t dtype, const mla_dims_t* dims) {
    if (!dims || check_out_dims(dtype, dims) != MLA_OK) return 0;
    return plan_gemm(out_problem(dtype, dims, nullptr, nullptr, nullptr, nullptr)).workspace_bytes;
}

int mla_out(mla_dtype_t dtype, const mla_dims_t* dims, const float* ctx, const float* row_sum,
            const void* W_uv, void* out, void* workspace, size_t workspace_bytes,
            hipStream_t stream) {
    MLA_CHECK(check_dtype(dtype));
    MLA_CHECK(check_out_dims(dtype, dims));
    MLA_CHECK(check_ptr(ctx, "ctx"));
    MLA_CHECK(check_ptr(row_sum, "row_sum"));
    MLA_CHECK(check_ptr(W_uv, "W_uv"));
    MLA_CHECK(check_ptr(out, "out"));
    GemmProblem p = out_problem(dtype, dims, ctx, row_sum, W_uv, out);
    const GemmPlan plan = plan_gemm(p);
    MLA_CHECK(check_ws(workspace, workspace_bytes, plan.workspace_bytes));
    MLA_TRY_HIP(launch_gemm(p, plan, workspace, stream), "out launch");
    return ok();
}

size_t mla_q_absorbed_workspace_bytes(mla_dtype_t dtype, const mla_dims_t* dims) {
    if (dtype == MLA_DTYPE_F64)
        return dims && check_f64_q_dims(dims) == MLA_OK ? q_layout64(dims).total : 0;
    if (!dims || check_q_dims(dtype, dims) != MLA_OK) return 0;
    return q_layout(dtype, dims).total;
}

int mla_q_absorbed(mla_dtype_t dtype, const mla_dims_t* dims, const void* x, const void* W_q_a,
                   const void* q_norm_w, const void* W_q_b, const void* W_uk,
                   const int64_t* positions, const void* inv_freq, double eps,
                   void* q_absorbed, void* q_rope, void* workspace, size_t workspace_bytes,
                   hipStream_t stream) {
    return q_absorbed_impl(dtype, dims, x, W_q_a, q_norm_w, W_q_b, W_uk, positions, inv_freq, eps,
                           q_absorbed, q_rope, workspace, workspace_bytes, stream, false);
}

int mla_q_absorbed_ragged(mla_dtype_t dtype, const mla_dims_t* dims, const void* x,
                          const void* W_q_a, const void* q_norm_w, const void* W_q_b,
                          const void* W_uk, const int64_t* positions, const void* inv_freq,
                          double eps, void* q_absorbed, void* q_rope, void* workspace,
                          size_t workspace_bytes, hipStream_t stream) {
    return q_absorbed_impl(dtype, dims, x, W_q_a, q_norm_w, W_q_b, W_uk, positions, inv_freq, eps,
                           q_absorbed, q_rope, workspace, workspace_bytes, stream, true);
}

size_t mla_attention_workspace_bytes(mla_dtype_t dtype, const mla_dims_t* dims, int causal) {
    if (dtype == MLA_DTYPE_F64)
        return dims && check_f64_attn_dims(dims, causal) == MLA_OK ? attn_layout64(dims).total : 0;
    if (!dims || check_attn_dims(dtype, dims, causal) != MLA_OK) return 0;
    return attn_layout(dtype, dims).total;
}

int mla_attention(mla_dtype_t dtype, const mla_dims_t* dims, const void* q_absorbed,
                  const void* q_rope, const void* c_kv, const void* pe_cache, const void* W_uv,
                  double scale, int causal, void* out, void* workspace, size_t workspace_bytes,
                  hipStream_t stream) {
    if (dtype == MLA_DTYPE_F64)
        return attention_f64(dims, q_absorbed, q_rope, c_kv, pe_cache, W_uv, scale, causal, out,
                             workspace, workspace_bytes, stream);
    MLA_CHECK(check_dtype(dtype));
    MLA_CHECK(check_attn_dims(dtype, dims, causal));
    MLA_CHECK(check_scale(scale));
    MLA_CHECK(check_ptr(q_absorbed, "q_absorbed"));
    MLA_CHECK(check_ptr(q_rope, "q_rope"));
    MLA_CHECK(check_ptr(c_kv, "c_kv"));
    MLA_CHECK(check_ptr(pe_cache, "pe_cache"));
    MLA_CHECK(check_ptr(W_uv, "W_uv"));
    MLA_CHECK(check_ptr(out, "out"));
    const AttnLayout L = attn_layout(dtype, dims);
    MLA_CHECK(check_ws(workspace, workspace_bytes, L.total));

    float* p = at<float>(workspace, L.off_p);
    float* m = at<float>(workspace, L.off_m);
    float* l = at<float>(workspace, L.off_l);
    float* alpha = at<float>(workspace, L.off_alpha);
    float* row_sum = at<float>(workspace, L.off_rowsum);
    float* ctx = at<float>(workspace, L.off_ctx);
    const int rows = dims->batch * dims->sq * dims->heads;

    if (L.fused) {
        // 3a+3b+3c fused, then 3d.  Decode-sized fp32 batches take 3d on a kernel that also
        // does the pass's split merge (MLA_OUT_SMALL=0: the merge kernel and the GEMM).
        const FlashProblem fp = flash_problem(dtype, dims, q_absorbed, q_rope, c_kv, pe_cache,
                                              scale, causal);
        float* part = at<float>(workspace, L.off_part);
        if (const int osm = out_small_mode(dtype, dims, L.flash)) {
            MLA_TRY_HIP(launch_flash(fp, L.flash, ctx, row_sum, part, stream, osm == 2),
                        "fused attention launch");
            const FlashPartials merged = {nullptr, nullptr, nullptr, 1};
            MLA_TRY_HIP(launch_out_small(osm == 2 ? merged : flash_partials(fp, L.flash, part),
                                         ctx, row_sum,
                                         static_cast<const float*>(W_uv),
                                         static_cast<float*>(out), dims->batch, dims->sq,
                                         dims->heads, dims->kv_rank, dims->v, stream),
                        "3d launch");
            return ok();
        }
        if (L.ctx16) {   // the pass writes ctx / row_sum already divided, in 16 bits
            MLA_TRY_HIP(launch_flash(fp, L.flash, ctx, row_sum, part, stream, true, ctx),
                        "fused attention launch");
            GemmProblem op = out_problem16(dtype, dims, ctx, W_uv, out);
            MLA_TRY_HIP(launch_gemm(op, L.out, at<void>(workspace, L.off_out_ws), stream),
                        "3d launch");
            return ok();
        }
        MLA_TRY_HIP(launch_flash(fp, L.flash, ctx, row_sum, part, stream), "fused attention launch");
        GemmProblem op = out_problem(dtype, dims, ctx, row_sum, W_uv, out);
        MLA_TRY_HIP(launch_gemm(op, L.out, at<void>(workspace, L.off_out_ws), stream),
                    "3d launch");
        return ok();
    }

    // 3a
    MLA_CHECK(run_scores(dtype, dims, q_absorbed, q_rope, c_kv, pe_cache, scale, causal, p, L.ld_p, m,
                         l, stream));
    // 3b
    MLA_TRY_HIP(launch_combine(m, l, alpha, row_sum, nullptr, rows, L.P, stream), "3b launch");
    // 3c
    GemmProblem cp = ctx_problem(dtype, dims, p, L.ld_p, alpha, c_kv, ctx);
    MLA_TRY_HIP(launch_gemm(cp, L.ctx, at<void>(workspace, L.off_ctx_ws), stream), "3c launch");
    // 3d
    GemmProblem op = out_problem(dtype, dims, ctx, row_sum, W_uv, out);
    MLA_TRY_HIP(launch_gemm(op, L.out, at<void>(workspace, L.off_out_ws), stream), "3d launch");
    return ok();
}

// ------------------------------------------------------------------ fp8 KV cache

size_t mla_attention_fp8kv_workspace_bytes(mla_dtype_t dtype, const mla_dims_t* dims, int causal) {
    if (!dims || check_fp8_attn(dtype, dims, causal, 1.f) != MLA_OK) return 0;
    return fp8_layout(dims).total;
}

int mla_attention_fp8kv(mla_dtype_t dtype, const mla_dims_t* dims, const void* q_absorbed,
                        const void* q_rope, const void* c_kv_fp8, const void* pe_fp8,
                        float kv_scale, const void* W_uv, double scale, int causal, void* out,
                        void* workspace, size_t workspace_bytes, hipStream_t stream) {
    MLA_CHECK(check_fp8_attn(dtype, dims, causal, kv_scale));
    MLA_CHECK(check_scale(scale));
    MLA_CHECK(check_ptr(q_absorbed, "q_absorbed"));
    MLA_CHECK(check_ptr(q_rope, "q_rope"));
    MLA_CHECK(check_ptr(c_kv_fp8, "c_kv_fp8"));
    MLA_CHECK(check_ptr(pe_fp8, "pe_fp8"));
    MLA_CHECK(check_ptr(W_uv, "W_uv"));
    MLA_CHECK(check_ptr(out, "out"));
    const Fp8Layout L = fp8_layout(dims);
    MLA_CHECK(check_ws(workspace, workspace_bytes, L.total));
    float* row_sum = at<float>(workspace, L.off_rowsum);
    float* ctx = at<float>(workspace, L.off_ctx);
    const FlashProblem fp = fp8_problem(dims, q_absorbed, q_rope, c_kv_fp8, pe_fp8, kv_scale,
                                        scale, causal);
    MLA_TRY_HIP(launch_flash(fp, L.flash, ctx, row_sum, at<float>(workspace, L.off_part), stream,
                             true, L.ctx16 ? ctx : nullptr),
                "fp8-cache attention launch");
    GemmProblem op = L.ctx16 ? out_problem16(MLA_DTYPE_BF16, dims, ctx, W_uv, out)
                             : out_problem(MLA_DTYPE_BF16, dims, ctx, row_sum, W_uv, out);
    MLA_TRY_HIP(launch_gemm(op, L.out, at<void>(workspace, L.off_out_ws), stream), "3d launch");
    return ok();
}

size_t mla_attention_paged_fp8kv_workspace_bytes(mla_dtype_t dtype, const mla_dims_t* dims,
                                                 int causal, int32_t page_size) {
    if (!dims || check_fp8_attn(dtype, dims, causal, 1.f) != MLA_OK ||
        check_pages(dims, page_size) != MLA_OK)
        return 0;
    return fp8_layout(dims, true).total;
}

int mla_attention_paged_fp8kv(mla_dtype_t dtype, const mla_dims_t* dims, const void* q_absorbed,
                              const void* q_rope, const void* c_kv_pages_fp8,
                              const void* pe_pages_fp8, const int32_t* block_table,
                              const int32_t* seq_lens, int32_t page_size, float kv_scale,
                              const void* W_uv, double scale, int causal, void* out,
                              void* workspace, size_t workspace_bytes, hipStream_t stream) {
    MLA_CHECK(check_fp8_attn(dtype, dims, causal, kv_scale));
    MLA_CHECK(check_pages(dims, page_size));
    MLA_CHECK(check_scale(scale));
    MLA_CHECK(check_ptr(q_absorbed, "q_absorbed"));
    MLA_CHECK(check_ptr(q_rope, "q_rope"));
    MLA_CHECK(check_ptr(c_kv_pages_fp8, "c_kv_pages_fp8"));
    MLA_CHECK(check_ptr(pe_pages_fp8, "pe_pages_fp8"));
    MLA_CHECK(check_ptr(block_table, "block_table"));
    MLA_CHECK(check_ptr(seq_lens, "seq_lens"));
    MLA_CHECK(check_ptr(W_uv, "W_uv"));
    MLA_CHECK(check_ptr(out, "out"));
    const Fp8Layout L = fp8_layout(dims, true);
    MLA_CHECK(check_ws(workspace, workspace_bytes, L.total));
    float* row_sum = at<float>(workspace, L.off_rowsum);
    float* ctx = at<float>(workspace, L.off_ctx);
    // the fp8 pass over the pages (each sequence to its own length, the key chunks balanced
    // by the device-built work list, merged into ctx / row_sum), then 3d
    FlashProblem fp = fp8_problem(dims, q_absorbed, q_rope, c_kv_pages_fp8, pe_pages_fp8,
                                  kv_scale, scale, causal);
    fp.seq_lens = seq_lens;
    fp.block_table = block_table;
    fp.page_size = page_size;
    MLA_TRY_HIP(launch_flash(fp, L.flash, ctx, row_sum, at<float>(workspace, L.off_part), stream),
                "paged fp8-cache attention launch");
    GemmProblem op = out_problem(MLA_DTYPE_BF16, dims, ctx, row_sum, W_uv, out);
    MLA_TRY_HIP(launch_gemm(op, L.out, at<void>(workspace, L.off_out_ws), stream), "3d launch");
    return ok();
}

int mla_fp8_dequantize(const void* codes, int64_t n, float scale, float* out, hipStream_t stream) {
    if (n < 0) return fail(MLA_ERR_INVALID_ARGUMENT, "n must not be negative (got %lld)", (long long)n);
    if (n == 0) return ok();
    if (!codes || !out) return fail(MLA_ERR_INVALID_ARGUMENT, "codes and out must not be NULL");
    MLA_TRY_HIP(launch_fp8_dequant(codes, n, scale, out, stream), "fp8 dequantize launch");
    return ok();
}

int mla_attention_noalloc(mla_dtype_t dtype, const mla_dims_t* dims, const void* q_absorbed,
                          const void* q_rope, const void* c_kv, const void* pe_cache,
                          const void* W_uv, double scale, int causal, void* out,
                          hipStream_t stream) {
    if (dtype == MLA_DTYPE_F64) {
        MLA_CHECK(check_f64_attn_dims(dims, causal));
    } else {
        MLA_CHECK(check_dtype(dtype));
        MLA_CHECK(check_attn_dims(dtype, dims, causal));
    }
    MLA_CHECK(check_scale(scale));
    MLA_CHECK(check_ptr(q_absorbed, "q_absorbed"));
    MLA_CHECK(check_ptr(q_rope, "q_rope"));
    MLA_CHECK(check_ptr(c_kv, "c_kv"));
    MLA_CHECK(check_ptr(pe_cache, "pe_cache"));
    MLA_CHECK(check_ptr(W_uv, "W_uv"));
    MLA_CHECK(check_ptr(out, "out"));
    const size_t need = dtype == MLA_DTYPE_F64 ? attn_layout64(dims).total
                                               : attn_layout(dtype, dims).total;
    if (need > kScratchBytes)
        return fail(MLA_ERR_WORKSPACE,
                    "mla_attention_noalloc: this shape needs %zu bytes of scratch, more than "
                    "the %zu bytes the library holds per GPU; use mla_attention with a "
                    "caller workspace", need, kScratchBytes);
    void* ws = nullptr;
    MLA_CHECK(scratch_for_stream(stream, &ws));
    return mla_attention(dtype, dims, q_absorbed, q_rope, c_kv, pe_cache, W_uv, scale, causal,
                         out, ws, kScratchBytes, stream);
}

size_t mla_attention_streaming_workspace_bytes(mla_dtype_t dtype, const mla_dims_t* dims,
                                               int causal, int32_t key_chunk) {
    if (!dims || check_attn_dims(dtype, dims, causal) != MLA_OK) return 0;
    if (key_chunk < 0 || key_chunk % kScoreTile != 0) return 0;
    return stream_layout(dtype, dims, key_chunk).total;
}

int mla_attention_streaming(mla_dtype_t dtype, const mla_dims_t* dims, const void* q_absorbed,
                            const void* q_rope, const void* c_kv, const void* pe_cache,
                            const void* W_uv, double scale, int causal, int32_t key_chunk,
                            void* out, void* workspace, size_t workspace_bytes,
                            hipStream_t stream) {
    MLA_CHECK(check_dtype(dtype));
    MLA_CHECK(check_attn_dims(dtype, dims, causal));
    MLA_CHECK(check_scale(scale));
    if (key_chunk < 0 || key_chunk % kScoreTile != 0)
        return fail(MLA_ERR_INVALID_ARGUMENT, "key_chunk must be 0 or a positive multiple of %d",
                    kScoreTile);
    MLA_CHECK(check_ptr(q_absorbed, "q_absorbed"));
    MLA_CHECK(check_ptr(q_rope, "q_rope"));
    MLA_CHECK(check_ptr(c_kv, "c_kv"));
    MLA_CHECK(check_ptr(pe_cache, "pe_cache"));
    MLA_CHECK(check_ptr(W_uv, "W_uv"));
    MLA_CHECK(check_ptr(out, "out"));
    const StreamLayout L = stream_layout(dtype, dims, key_chunk);
    MLA_CHECK(check_ws(workspace, workspace_bytes, L.total));

    const int rows = dims->batch * dims->sq * dims->heads;
    const size_t esz = is_half(dtype) ? 2 : 4;
    float* p = at<float>(workspace, L.off_p);
    float* m = at<float>(workspace, L.off_m);
    float* l = at<float>(workspace, L.off_l);
    float* alpha = at<float>(workspace, L.off_alpha);
    float* sum_c = at<float>(workspace, L.off_sum_c);
    float* max_c = at<float>(workspace, L.off_max_c);
    float* ctx_c = at<float>(workspace, L.off_ctx_c);
    float* ctx = at<float>(workspace, L.off_ctx);
    float* run_max = at<float>(workspace, L.off_run_max);
    float* run_sum = at<float>(workspace, L.off_run_sum);

    for (int c0 = 0, chunk = 0; c0 < dims->sk; c0 += L.chunk, ++chunk) {
        mla_dims_t dc = *dims;
        dc.sk = std::min(L.chunk, dims->sk - c0);
        const int ld_p = mla_score_ld(dc.sk);
        const int P = cdiv(dc.sk, kScoreTile);
        const char* ck = static_cast<const char*>(c_kv) + (size_t)c0 * dims->kv_rank * esz;
        const char* pe = static_cast<const char*>(pe_cache) + (size_t)c0 * dims->rope * esz;
        // 3a on the chunk (keys c0 .. c0+sk-1 of every sequence; causal rule on absolute keys)
        MLA_CHECK(run_scores(dtype, &dc, q_absorbed, q_rope, ck, pe, scale, causal, p, ld_p, m, l,
                             stream, dims->sk, c0, dims->sk));
        // 3b: per-chunk maximum and sum relative to it
        MLA_TRY_HIP(launch_combine(m, l, alpha, sum_c, max_c, rows, P, stream), "stream 3b launch");
        // 3c on the chunk
        GemmProblem cp = ctx_problem(dtype, &dc, p, ld_p, alpha, ck, ctx_c);
        cp.sBg = (int64_t)dims->sk * dims->kv_rank;  // batch stride of the whole cache
        const GemmPlan plan = plan_gemm(cp);
        MLA_TRY_HIP(launch_gemm(cp, plan, at<void>(workspace, L.off_ctx_ws), stream),
                    "stream 3c launch");
        // online-softmax merge into the running state
        MLA_TRY_HIP(launch_stream_merge(ctx, run_max, run_sum, ctx_c, max_c, sum_c, rows,
                                        dims->kv_rank, chunk == 0, stream),
                    "stream merge launch");
    }
    // 3d on the merged state
    GemmProblem op = out_problem(dtype, dims, ctx, run_sum, W_uv, out);
    MLA_TRY_HIP(launch_gemm(op, L.out, at<void>(workspace, L.off_out_ws), stream),
                "stream 3d launch");
    return ok();
}

int mla_split_wkv_b(mla_dtype_t dtype, const mla_dims_t* dims, const void* wkv_b, void* W_uk,
                    void* W_uv, hipStream_t stream) {
    MLA_CHECK(check_dtype(dtype));
    MLA_CHECK(check_split_dims(dtype, dims));
    MLA_CHECK(check_ptr(wkv_b, "wkv_b"));
    MLA_CHECK(check_ptr(W_uk, "W_uk"));
    MLA_CHECK(check_ptr(W_uv, "W_uv"));
    const int64_t row_bytes = (int64_t)dims->kv_rank * (is_half(dtype) ? 2 : 4);
    MLA_TRY_HIP(launch_split_rows(wkv_b, W_uk, W_uv, dims->heads, dims->nope, dims->v, row_bytes,
                                  stream),
                "wkv_b split launch");
    return ok();
}

size_t mla_kv_append_workspace_bytes(mla_dtype_t dtype, const mla_dims_t* dims) {
    if (!dims || check_dtype(dtype) != MLA_OK || check_kv_dims(dtype, dims) != MLA_OK) return 0;
    return kv_ws_bytes(dtype, dims, nullptr);
}

int mla_kv_append(mla_dtype_t dtype, const mla_dims_t* dims, const void* x, const void* W_kv_a,
                  const void* kv_norm_w, const int64_t* positions, const float* inv_freq,
                  double eps, int32_t start_row, int32_t cache_rows, void* c_kv, void* pe_cache,
                  void* workspace, size_t workspace_bytes, hipStream_t stream) {
    return kv_append_impl(dtype, dims, x, W_kv_a, kv_norm_w, positions, inv_freq, eps, start_row,
                          cache_rows, nullptr, 0, c_kv, pe_cache, workspace, workspace_bytes,
                          stream);
}

int mla_kv_append_paged(mla_dtype_t dtype, const mla_dims_t* dims, const void* x,
                        const void* W_kv_a, const void* kv_norm_w, const int64_t* positions,
                        const float* inv_freq, double eps, const int32_t* block_table,
                        int32_t page_size, void* c_kv_pages, void* pe_pages, void* workspace,
                        size_t workspace_bytes, hipStream_t stream) {
    MLA_CHECK(check_ptr(block_table, "block_table"));
    return kv_append_impl(dtype, dims, x, W_kv_a, kv_norm_w, positions, inv_freq, eps, 0, 0,
                          block_table, page_size, c_kv_pages, pe_pages, workspace,
                          workspace_bytes, stream);
}

size_t mla_attention_paged_workspace_bytes(mla_dtype_t dtype, const mla_dims_t* dims,
                                           int causal, int32_t page_size) {
    if (!dims || check_dtype(dtype) != MLA_OK || check_attn_dims(dtype, dims, causal) != MLA_OK ||
        check_pages(dims, page_size) != MLA_OK)
        return 0;
    return attn_layout(dtype, dims, true).total;
}

int mla_attention_paged(mla_dtype_t dtype, const mla_dims_t* dims, const void* q_absorbed,
                        const void* q_rope, const void* c_kv_pages, const void* pe_pages,
                        const int32_t* block_table, const int32_t* seq_lens, int32_t page_size,
                        const void* W_uv, double scale, int causal, void* out, void* workspace,
                        size_t workspace_bytes, hipStream_t stream) {
    MLA_CHECK(check_dtype(dtype));
    MLA_CHECK(check_attn_dims(dtype, dims, causal));
    MLA_CHECK(check_pages(dims, page_size));
    MLA_CHECK(check_scale(scale));
    MLA_CHECK(check_ptr(q_absorbed, "q_absorbed"));
    MLA_CHECK(check_ptr(q_rope, "q_rope"));
    MLA_CHECK(check_ptr(c_kv_pages, "c_kv_pages"));
    MLA_CHECK(check_ptr(pe_pages, "pe_pages"));
    MLA_CHECK(check_ptr(block_table, "block_table"));
    MLA_CHECK(check_ptr(seq_lens, "seq_lens"));
    MLA_CHECK(check_ptr(W_uv, "W_uv"));
    MLA_CHECK(check_ptr(out, "out"));
    const AttnLayout L = attn_layout(dtype, dims, true);
    MLA_CHECK(check_ws(workspace, workspace_bytes, L.total));

    float* p = at<float>(workspace, L.off_p);
    float* m = at<float>(workspace, L.off_m);
    float* l = at<float>(workspace, L.off_l);
    float* alpha = at<float>(workspace, L.off_alpha);
    float* row_sum = at<float>(workspace, L.off_rowsum);
    float* ctx = at<float>(workspace, L.off_ctx);
    const int rows = dims->batch * dims->sq * dims->heads;

    if (L.fused) {
        // 3a+3b+3c fused over the pages (each sequence to its own length, the key chunks
        // balanced over the CUs by a work list built from seq_lens), then 3d
        FlashProblem fp = flash_problem(dtype, dims, q_absorbed, q_rope, c_kv_pages, pe_pages,
                                        scale, causal);
        fp.seq_lens = seq_lens;
        fp.block_table = block_table;
        fp.page_size = page_size;
        float* part = at<float>(workspace, L.off_part);
        if (const int osm = out_small_mode(dtype, dims, L.flash)) {
            MLA_TRY_HIP(launch_flash(fp, L.flash, ctx, row_sum, part, stream, osm == 2),
                        "fused paged attention launch");
            const FlashPartials merged = {nullptr, nullptr, nullptr, 1};
            MLA_TRY_HIP(launch_out_small(osm == 2 ? merged : flash_partials(fp, L.flash, part),
                                         ctx, row_sum,
                                         static_cast<const float*>(W_uv),
                                         static_cast<float*>(out), dims->batch, dims->sq,
                                         dims->heads, dims->kv_rank, dims->v, stream),
                        "3d launch");
            return ok();
        }
        MLA_TRY_HIP(launch_flash(fp, L.flash, ctx, row_sum, part, stream),
                    "fused paged attention launch");
        GemmProblem op = out_problem(dtype, dims, ctx, row_sum, W_uv, out);
        MLA_TRY_HIP(launch_gemm(op, L.out, at<void>(workspace, L.off_out_ws), stream),
                    "3d launch");
        return ok();
    }

    // 3a over the pages, each sequence to its own length (keys past it score as masked)
    MLA_CHECK(run_scores(dtype, dims, q_absorbed, q_rope, c_kv_pages, pe_pages, scale, causal, p,
                         L.ld_p, m, l, stream, 0, 0, 0, seq_lens, block_table, page_size));
    // 3b: a tile past a sequence's keys has m = -inf, l = 0 and gets alpha 0
    MLA_TRY_HIP(launch_combine(m, l, alpha, row_sum, nullptr, rows, L.P, stream), "3b launch");
    // 3c: K rows through the block table, K limited to each sequence's length
    GemmProblem cp = ctx_problem(dtype, dims, p, L.ld_p, alpha, c_kv_pages, ctx);
    cp.sBg = 0;
    cp.k_len = seq_lens;
    cp.b_pages = block_table; cp.page_size = page_size; cp.max_pages = dims->sk / page_size;
    MLA_TRY_HIP(launch_gemm(cp, L.ctx, at<void>(workspace, L.off_ctx_ws), stream), "3c launch");
    // 3d
    GemmProblem op = out_problem(dtype, dims, ctx, row_sum, W_uv, out);
    MLA_TRY_HIP(launch_gemm(op, L.out, at<void>(workspace, L.off_out_ws), stream), "3d launch");
    return ok();
}

int32_t mla_attention_work_list_ints(mla_dtype_t dtype, const mla_dims_t* dims) {
    if (!dims || check_dtype(dtype) != MLA_OK || check_work_list_dims(dims) != MLA_OK) return 0;
    FlashProblem fp = flash_problem(dtype, dims, nullptr, nullptr, nullptr, nullptr, 1.0, 0);
    fp.ragged = true;
    fp.want_list = true;   // the list itself, also where the attention would not build one
    return flash_worklist_ints(fp, plan_flash(fp));
}

int mla_attention_work_list(mla_dtype_t dtype, const mla_dims_t* dims, const int32_t* seq_lens,
                            int32_t* work_list, int32_t ints, hipStream_t stream) {
    MLA_CHECK(check_dtype(dtype));
    MLA_CHECK(check_work_list_dims(dims));
    MLA_CHECK(check_ptr(seq_lens, "seq_lens"));
    MLA_CHECK(check_ptr(work_list, "work_list"));
    FlashProblem fp = flash_problem(dtype, dims, nullptr, nullptr, nullptr, nullptr, 1.0, 0);
    fp.ragged = true;
    fp.want_list = true;
    fp.seq_lens = seq_lens;
    const FlashPlan plan = plan_flash(fp);
    const int need = flash_worklist_ints(fp, plan);
    if (ints < need)
        return fail(MLA_ERR_INVALID_ARGUMENT, "work_list holds %d ints, %d required", ints, need);
    MLA_TRY_HIP(launch_flash_worklist(fp, plan, work_list, stream), "work list launch");
    return ok();
}

size_t mla_o_proj_workspace_bytes(mla_dtype_t dtype, const mla_dims_t* dims) {
    if (!dims || check_dtype(dtype) != MLA_OK || check_oproj_dims(dtype, dims) != MLA_OK) return 0;
    return align_up(plan_gemm(oproj_problem(dtype, dims, nullptr, nullptr, nullptr)).workspace_bytes);
}

int mla_o_proj(mla_dtype_t dtype, const mla_dims_t* dims, const void* attn, const void* W_o,
               void* out, void* workspace, size_t workspace_bytes, hipStream_t stream) {
    MLA_CHECK(check_dtype(dtype));
    MLA_CHECK(check_oproj_dims(dtype, dims));
    MLA_CHECK(check_ptr(attn, "attn"));
    MLA_CHECK(check_ptr(W_o, "W_o"));
    MLA_CHECK(check_ptr(out, "out"));
    const GemmProblem gp = oproj_problem(dtype, dims, attn, W_o, out);
    const GemmPlan plan = plan_gemm(gp);
    MLA_CHECK(check_ws(workspace, workspace_bytes, align_up(plan.workspace_bytes)));
    MLA_TRY_HIP(launch_gemm(gp, plan, workspace, stream), "wo GEMM launch");
    return ok();
}

}  // extern "C"
#pragma GCC visibility pop
