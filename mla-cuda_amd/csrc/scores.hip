// 3a: latent scoring with the split-softmax epilogue.
//
// For a batch b the rows f = (s*H + h) of q_absorbed|q_rope form Q_b [Sq*H, R+D] and the
// keys form K_b = c_kv[b] | pe_cache[b]  [Sk, R+D]; the scores are Q_b K_b^T / scale, one
// (R+D)-deep reduction whose last D columns come from the second operand pair.
//
// Workgroup tile: 128 rows x 128 keys (one softmax partial).  Each of the 4 waves owns
// 32 rows x 128 keys = 4 v_mfma_f32_32x32x2_f32 accumulator blocks, so a row's 128 keys
// live in one wave: the row max and row sum need no LDS, only a 32-lane reduction
// (DPP + ds_swizzle) of each accumulator register.  Depth is walked in 32-deep slices
// staged through double-buffered LDS, exactly like the GEMM engine.
//
// Epilogue per row and 128-key tile j (mla_kernels.cu:971-1032 computes the same
// quantities): m_j = max over visible keys of t = s/scale, p = exp(t - m_j) stored into
// `scores` (0 for masked keys and for the row padding [Sk, ld_p)), l_j = sum p.
// Grid: batch x row tiles x key tiles, XCD-ordered so one XCD streams one batch's keys
// while its L2 keeps that batch's Q rows.

#include "common.h"
#include "kernels.h"

namespace mla {

namespace {

constexpr int kBM = 128, kBN = 128, kBK = 32, kPad = 4, kThreads = 256;

struct ScoresArgs {
    const float* qa; const float* qr; const float* ckv; const float* pe;
    float* p; float* m_part; float* l_part;
    int B, Sq, Sk, H, R, D, ld_p, P, tiles_r;
    float inv_scale;
    int causal;
};

__global__ void __launch_bounds__(kThreads, 2) scores_kernel(ScoresArgs a) {
    __shared__ __attribute__((aligned(16))) float Qs[2][kBM][kBK + kPad];
    __shared__ __attribute__((aligned(16))) float Ks[2][kBN][kBK + kPad];

    int t = xcd_logical_block(blockIdx.x, gridDim.x);
    const int kt = t % a.P; t /= a.P;
    const int tr = t % a.tiles_r;
    const int b = t / a.tiles_r;

    const int rows_b = a.Sq * a.H;             // rows of this batch
    const int r0 = tr * kBM;                   // first row (within the batch)
    const int k0 = kt * kBN;                   // first key
    const int64_t row_base = (int64_t)b * rows_b;

    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int l32 = lane & 31, kq = 4 * (lane >> 5);

    const int nsl_r = (a.R + kBK - 1) / kBK;
    const int nsl = nsl_r + (a.D + kBK - 1) / kBK;

    v4f rq[4], rk[4];
    auto load_slice = [&](int s) {
        const bool rope = s >= nsl_r;
        const int c0 = rope ? (s - nsl_r) * kBK : s * kBK;
        const int cw = rope ? a.D : a.R;
        const float* qsrc = rope ? a.qr : a.qa;
        const float* ksrc = rope ? a.pe : a.ckv;
        const int c = c0 + 4 * (tid & 7);
        #pragma unroll
        for (int i = 0; i < 4; ++i) {
            const int r = r0 + i * 32 + (tid >> 3);
            v4f v = {0.f, 0.f, 0.f, 0.f};
            if (r < rows_b && c < cw)
                v = *reinterpret_cast<const v4f*>(qsrc + (row_base + r) * cw + c);
            rq[i] = v;
            const int k = k0 + i * 32 + (tid >> 3);
            v4f w = {0.f, 0.f, 0.f, 0.f};
            if (k < a.Sk && c < cw)
                w = *reinterpret_cast<const v4f*>(ksrc + ((int64_t)b * a.Sk + k) * cw + c);
            rk[i] = w;
        }
    };
    auto store_slice = [&](int buf) {
        #pragma unroll
        for (int i = 0; i < 4; ++i) {
            *reinterpret_cast<v4f*>(&Qs[buf][i * 32 + (tid >> 3)][4 * (tid & 7)]) = rq[i];
            *reinterpret_cast<v4f*>(&Ks[buf][i * 32 + (tid >> 3)][4 * (tid & 7)]) = rk[i];
        }
    };

    v16f acc[4];
    #pragma unroll
    for (int j = 0; j < 4; ++j)
        #pragma unroll
        for (int e = 0; e < 16; ++e) acc[j][e] = 0.f;

    load_slice(0);
    store_slice(0);
    __syncthreads();
    for (int s = 0; s < nsl; ++s) {
        const int buf = s & 1;
        if (s + 1 < nsl) load_slice(s + 1);
        #pragma unroll
        for (int kk = 0; kk < kBK; kk += 8) {
            const v4f fq = *reinterpret_cast<const v4f*>(&Qs[buf][wave * 32 + l32][kk + kq]);
            v4f fk[4];
            #pragma unroll
            for (int j = 0; j < 4; ++j)
                fk[j] = *reinterpret_cast<const v4f*>(&Ks[buf][j * 32 + l32][kk + kq]);
            #pragma unroll
            for (int q = 0; q < 4; ++q)
                #pragma unroll
                for (int j = 0; j < 4; ++j) acc[j] = mfma_32x32x2(fq[q], fk[j][q], acc[j]);
        }
        if (s + 1 < nsl) store_slice(buf ^ 1);
        __syncthreads();
    }

    // ---- epilogue: per accumulator register e the lane holds row acc_row(e, lane) and
    // keys k0 + 32*j + l32 (j = 0..3).
    #pragma unroll
    for (int e = 0; e < 16; ++e) {
        const int r = r0 + wave * 32 + acc_row(e, lane);   // row within the batch
        const bool row_ok = r < rows_b;
        // causal: query index s = r / H sees keys <= Sk - Sq + s
        const int kmax = a.causal ? (a.Sk - a.Sq + (row_ok ? r / a.H : 0)) : (a.Sk - 1);
        float tv[4];
        float mx = -INFINITY;
        #pragma unroll
        for (int j = 0; j < 4; ++j) {
            const int k = k0 + 32 * j + l32;
            tv[j] = acc[j][e] * a.inv_scale;
            if (k <= kmax && k < a.Sk) mx = fmaxf(mx, tv[j]);
        }
        mx = half_wave_reduce(mx, OpMax());
        float sum = 0.f;
        float* prow = a.p + (row_base + r) * (int64_t)a.ld_p;
        #pragma unroll
        for (int j = 0; j < 4; ++j) {
            const int k = k0 + 32 * j + l32;
            const bool vis = (k <= kmax) && (k < a.Sk);
            const float pv = vis ? expf(tv[j] - mx) : 0.f;
            sum += pv;
            if (row_ok && k < a.ld_p) prow[k] = pv;
        }
        sum = half_wave_reduce(sum, OpSum());
        if (row_ok && l32 == 0) {
            a.m_part[(row_base + r) * a.P + kt] = mx;
            a.l_part[(row_base + r) * a.P + kt] = sum;
        }
    }
}

}  // namespace

hipError_t launch_scores(const ScoresProblem& p, hipStream_t stream) {
    ScoresArgs a;
    a.qa = p.qa; a.qr = p.qr; a.ckv = p.ckv; a.pe = p.pe;
    a.p = p.p; a.m_part = p.m_part; a.l_part = p.l_part;
    a.B = p.B; a.Sq = p.Sq; a.Sk = p.Sk; a.H = p.H; a.R = p.R; a.D = p.D;
    a.ld_p = p.ld_p; a.P = p.P;
    a.tiles_r = (p.Sq * p.H + kBM - 1) / kBM;
    a.inv_scale = p.inv_scale;
    a.causal = p.causal ? 1 : 0;
    const int64_t nblocks = (int64_t)p.B * a.tiles_r * a.P;
    if (nblocks <= 0 || nblocks > 0x7fffffff) return hipErrorInvalidValue;
    hipLaunchKernelGGL(scores_kernel, dim3((unsigned)nblocks), dim3(kThreads), 0, stream, a);
    return hipGetLastError();
}

}  // namespace mla
