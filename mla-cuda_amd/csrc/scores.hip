// 3a: latent scoring with the split-softmax epilogue.
//
// For a batch b the rows f = (s*H + h) of q_absorbed|q_rope form Q_b [Sq*H, R+D] and the
// keys form K_b = c_kv[b] | pe_cache[b]  [Sk, R+D]; the scores are Q_b K_b^T / scale, one
// (R+D)-deep reduction whose last D columns come from the second operand pair.
//
// Workgroup tile: 128 rows x 128 keys (one softmax partial).  Each of the 4 waves owns
// 32 rows x 128 keys = 4 MFMA accumulator blocks (fp32 or bf16 steps, mma.h), so a row's 128 keys
// live in one wave: the row max and row sum need no LDS, only a 32-lane reduction
// (DPP + ds_swizzle) of each accumulator register.  Depth is walked in 128-byte slices
// (32 fp32 / 64 bf16) staged through double-buffered LDS, exactly like the GEMM engine.
//
// Epilogue per row and 128-key tile j (mla_kernels.cu:971-1032 computes the same
// quantities): m_j = max over visible keys of t = s/scale, p = exp(t - m_j) stored into
// `scores` (0 for masked keys and for the row padding [Sk, ld_p)), l_j = sum p.
// Grid: batch x row tiles x key tiles, XCD-ordered so one XCD streams one batch's keys
// while its L2 keeps that batch's Q rows.

#include "kernels.h"
#include "mma.h"

#include <algorithm>

namespace mla {

namespace {

constexpr int kBM = 128, kBN = 128, kRowWords = 36, kThreads = 256;

struct ScoresArgs {
    const void* qa; const void* qr; const void* ckv; const void* pe;
    float* p; float* m_part; float* l_part;
    int B, Sq, Sk, H, R, D, ld_p, P, tiles_r;
    int64_t key_stride;   // key rows between batches
    int causal_base;      // sk_total - Sq - key_offset: query s sees local keys <= base + s
    float scale_log2;   // log2(e) / scale
    int causal;
};

// PD = depth of the register prefetch ring: while slice s feeds the MFMAs from LDS, slices
// s+1 .. s+PD are in flight from global memory.  fp32 is MFMA-bound with ~4K MFMA cycles
// per slice and uses PD = 1; bf16 slices hold 8x less MFMA work, so HBM latency is only
// hidden with several slices in flight (PD = 4).
template <typename TL, int PD>
__global__ void __launch_bounds__(kThreads, 2) scores_kernel(ScoresArgs a) {
    using MM = Mma<TL>;
    constexpr int E = MM::kElems, KS = MM::kSlice;
    static_assert(PD == 1 || PD % 2 == 0, "ring depth 1 or even (LDS buffer index is slot parity)");
    __shared__ __attribute__((aligned(16))) uint32_t Qs[2][kBM][kRowWords];
    __shared__ __attribute__((aligned(16))) uint32_t Ks[2][kBN][kRowWords];

    int t = xcd_logical_block(blockIdx.x, gridDim.x);
    const int kt = t % a.P; t /= a.P;
    const int tr = t % a.tiles_r;
    const int b = t / a.tiles_r;

    const int rows_b = a.Sq * a.H;             // rows of this batch
    const int r0 = tr * kBM;                   // first row (within the batch)
    const int k0 = kt * kBN;                   // first key
    const int64_t row_base = (int64_t)b * rows_b;

    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int l32 = lane & 31, half = lane >> 5;

    const int nsl_r = (a.R + KS - 1) / KS;
    const int nsl = nsl_r + (a.D + KS - 1) / KS;

    // Staging geometry, fixed for the whole tile: thread tid loads 16-byte chunk tid%8 of
    // tile rows i*32 + tid/8 (i = 0..3) of Q and of K.  Byte offsets are relative to the
    // slice's first column of the tile's first row, kOob for rows beyond the tile; the
    // latent (R-wide) and rope (D-wide) rows have their own strides.
    const TL* qa_t = static_cast<const TL*>(a.qa) + (row_base + r0) * a.R;
    const TL* qr_t = static_cast<const TL*>(a.qr) + (row_base + r0) * a.D;
    const int64_t key_row0 = (int64_t)b * a.key_stride + k0;
    const TL* ckv_t = static_cast<const TL*>(a.ckv) + key_row0 * a.R;
    const TL* pe_t = static_cast<const TL*>(a.pe) + key_row0 * a.D;
    uint32_t oq_r[4], oq_d[4], ok_r[4], ok_d[4];
    #pragma unroll
    for (int i = 0; i < 4; ++i) {
        const uint32_t row = i * 32 + (tid >> 3), cb = 16u * (tid & 7);
        const bool qv = r0 + (int)row < rows_b, kv = k0 + (int)row < a.Sk;
        oq_r[i] = qv ? row * (uint32_t)(a.R * sizeof(TL)) + cb : kOob;
        oq_d[i] = qv ? row * (uint32_t)(a.D * sizeof(TL)) + cb : kOob;
        ok_r[i] = kv ? row * (uint32_t)(a.R * sizeof(TL)) + cb : kOob;
        ok_d[i] = kv ? row * (uint32_t)(a.D * sizeof(TL)) + cb : kOob;
    }

    // Slices at or past nsl load zeros (their column test fails), so the ring needs no
    // bounds branches; the zeros land in an LDS buffer nobody reads.
    v4u rq[PD][4], rk[PD][4];
    auto load_slice = [&](int s, int slot) {
        const bool rope = s >= nsl_r;
        const int c0 = rope ? (s - nsl_r) * KS : s * KS;
        const int cw = rope ? a.D : a.R;
        const __amdgpu_buffer_rsrc_t rsq = make_rsrc((rope ? qr_t : qa_t) + c0);
        const __amdgpu_buffer_rsrc_t rsk = make_rsrc((rope ? pe_t : ckv_t) + c0);
        // column chunks at or past the row width (a partial last slice, or a slice past
        // nsl) get the kOob bit OR-ed into their offsets
        const uint32_t cmask = oob_mask(E * (tid & 7), cw - c0);
        #pragma unroll
        for (int i = 0; i < 4; ++i) {
            rq[slot][i] = load16(rsq, (rope ? oq_d[i] : oq_r[i]) | cmask);
            rk[slot][i] = load16(rsk, (rope ? ok_d[i] : ok_r[i]) | cmask);
        }
    };
    auto store_slice = [&](int buf, int slot) {
        #pragma unroll
        for (int i = 0; i < 4; ++i) {
            *reinterpret_cast<v4u*>(&Qs[buf][i * 32 + (tid >> 3)][4 * (tid & 7)]) = rq[slot][i];
            *reinterpret_cast<v4u*>(&Ks[buf][i * 32 + (tid >> 3)][4 * (tid & 7)]) = rk[slot][i];
        }
    };

    v16f acc[4];
    #pragma unroll
    for (int j = 0; j < 4; ++j)
        #pragma unroll
        for (int e = 0; e < 16; ++e) acc[j][e] = 0.f;

    #pragma unroll
    for (int u = 0; u < PD; ++u) load_slice(u, u);
    store_slice(0, 0);
    __syncthreads();
    // slice s sits in LDS buffer s&1 and came from ring slot s%PD; the loop is unrolled by
    // PD so every slot index is a compile-time constant
    for (int s0 = 0; s0 < nsl; s0 += PD) {
        #pragma unroll
        for (int u = 0; u < PD; ++u) {
            const int s = s0 + u;
            if (PD == 1 || s < nsl) {
                const int buf = (PD == 1) ? (s & 1) : (u & 1);
                load_slice(s + PD, u);
                #pragma unroll
                for (int st = 0; st < 4; ++st) {
                    const v4u fq = *reinterpret_cast<const v4u*>(&Qs[buf][wave * 32 + l32][8 * st + 4 * half]);
                    v4u fk[4];
                    #pragma unroll
                    for (int j = 0; j < 4; ++j)
                        fk[j] = *reinterpret_cast<const v4u*>(&Ks[buf][j * 32 + l32][8 * st + 4 * half]);
                    #pragma unroll
                    for (int q = 0; q < MM::kSub; ++q)
                        #pragma unroll
                        for (int j = 0; j < 4; ++j) acc[j] = MM::sub(fq, fk[j], q, acc[j]);
                }
                store_slice(buf ^ 1, (u + 1) % PD);
                sched_slice<5, 4 * MM::kSub, 8, 8>();
                __syncthreads();
            }
        }
    }

    // ---- epilogue: per accumulator register e the lane holds row acc_row(e, lane) and
    // keys k0 + 32*j + l32 (j = 0..3).  Work in the log2 domain: t2 = s * (log2(e)/scale),
    // p = 2^(t2 - max t2) is one v_exp_f32, and m = max t2 * ln(2) is stored in the natural
    // units of s/scale.  (The exponent's rounding differs from exp(s/scale - m) by ~1e-7
    // relative to |s/scale|, i.e. ~1e-6 relative in p.)
    #pragma unroll
    for (int e = 0; e < 16; ++e) {
        const int r = r0 + wave * 32 + acc_row(e, lane);   // row within the batch
        const bool row_ok = r < rows_b;
        // causal: query index s = r / H sees absolute keys <= Sk_total - Sq + s
        const int kmax = a.causal ? (a.causal_base + (row_ok ? r / a.H : 0)) : (a.Sk - 1);
        float tv[4];
        float mx = -INFINITY;
        #pragma unroll
        for (int j = 0; j < 4; ++j) {
            const int k = k0 + 32 * j + l32;
            tv[j] = acc[j][e] * a.scale_log2;
            if (k <= kmax && k < a.Sk) mx = fmaxf(mx, tv[j]);
        }
        mx = half_wave_reduce(mx, OpMax());
        float sum = 0.f;
        float* prow = a.p + (row_base + r) * (int64_t)a.ld_p;
        #pragma unroll
        for (int j = 0; j < 4; ++j) {
            const int k = k0 + 32 * j + l32;
            const bool vis = (k <= kmax) && (k < a.Sk);
            const float pv = vis ? __builtin_amdgcn_exp2f(tv[j] - mx) : 0.f;
            sum += pv;
            if (row_ok && k < a.ld_p) prow[k] = pv;
        }
        sum = half_wave_reduce(sum, OpSum());
        if (row_ok && l32 == 0) {
            a.m_part[(row_base + r) * a.P + kt] = mx * 0.69314718055994531f;  // ln 2
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
    a.key_stride = p.key_stride ? p.key_stride : p.Sk;
    a.causal_base = (p.sk_total ? p.sk_total : p.Sk) - p.Sq - p.key_offset;
    a.scale_log2 = p.inv_scale * 1.4426950408889634f;
    a.causal = p.causal ? 1 : 0;
    // every staging offset (a row of the 128-row tile) must stay below the buffer range
    const int64_t row_bytes = (int64_t)std::max(p.R, p.D) * (p.bf16 ? 2 : 4);
    if (kBM * row_bytes >= kRsrcRange) return hipErrorInvalidValue;
    const int64_t nblocks = (int64_t)p.B * a.tiles_r * a.P;
    if (nblocks <= 0 || nblocks > 0x7fffffff) return hipErrorInvalidValue;
    if (p.bf16)
        hipLaunchKernelGGL((scores_kernel<bf16_t, 4>), dim3((unsigned)nblocks), dim3(kThreads), 0, stream, a);
    else
        hipLaunchKernelGGL((scores_kernel<float, 1>), dim3((unsigned)nblocks), dim3(kThreads), 0, stream, a);
    return hipGetLastError();
}

}  // namespace mla
