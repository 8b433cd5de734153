// Batched fp32 MFMA GEMM for the layer's dense contractions:
//   2a1 / 2a2  x @ W_q_a, q_lat @ W_q_b          (NN, G = 1)
//   2c         q_nope[h] @ W_uk[h]                (NN, G = heads)
//   3c         (p * alpha) @ c_kv[b]              (NN, G = batch, A scaled by alpha)
//   3d         (ctx[h] / row_sum) @ W_uv[h]^T     (NT, G = heads, A scaled by 1/row_sum)
//
// Workgroup = 4 wave64s.  A BM x BN output tile is split 2x2 / 4x1 / 1x4 over the waves,
// each wave covering its sub-tile with 32x32 v_mfma_f32_32x32x2_f32 blocks.  K is walked in
// 32-deep slices staged through LDS with double buffering: the next slice's 128-bit global
// loads are in flight while the current slice feeds the MFMAs.  Within a slice, K is
// permuted so lane l's operands for four consecutive MFMAs are contiguous in LDS
// (k = 4*(l/32) + j), making each fragment one ds_read_b128 (K-contiguous operands) or
// four conflict-free ds_read_b32 (N-contiguous operands).
//
// LDS rows of K-contiguous tiles are padded to 36 floats (144 B): the eight lanes of a
// ds_read_b128 / ds_write_b128 phase then land on disjoint bank groups.  N-contiguous
// tiles are padded to BN + 8 so the two half-waves of a ds_read_b32 hit opposite bank
// halves.
//
// Split-K is deterministic: slices write fp32 partials to a workspace and a reduction
// kernel sums them in a fixed order (no float atomics).

#include "common.h"
#include "kernels.h"

#include <algorithm>
#include <cstdio>
#include <cstdlib>

namespace mla {

namespace {

constexpr int kBK = 32;         // K per LDS slice
constexpr int kPadK = 4;        // K-contiguous row padding (floats)
constexpr int kPadN = 8;        // N-contiguous row padding (floats)
constexpr int kThreads = 256;

struct GemmArgs {
    const float* A; int64_t lda, sAg;
    const float* B; int64_t ldb, sBg;
    void* C; int64_t ldc, sCg;
    float* ws; int64_t ws_split;   // partials [split][G][M][N] when split > 1
    int M, N, K, G;
    int split, k_chunk, tiles_m, tiles_n;
    const float* rs; int64_t rs_m, rs_g;
    const float* alpha; int alpha_ld, alpha_tile;
};

template <int BM, int BN, int WM, int WN, bool NT, int AMODE, int OUT>
__global__ void __launch_bounds__(kThreads, 2) gemm_kernel(GemmArgs a) {
    constexpr int WTM = BM / WM, WTN = BN / WN;     // rows / cols per wave
    constexpr int TM = WTM / 32, TN = WTN / 32;     // 32x32 blocks per wave
    static_assert(WM * WN == 4 && TM >= 1 && TN >= 1, "4 waves, 32x32 blocks");
    constexpr int A_LD = BM / 32;                   // float4 loads per thread for A
    constexpr int B_LD = BN / 32;                   // ... for B (both layouts)
    constexpr int BROWS = NT ? BN : kBK;
    constexpr int BCOLS = NT ? kBK + kPadK : BN + kPadN;

    __shared__ __attribute__((aligned(16))) float As[2][BM][kBK + kPadK];
    __shared__ __attribute__((aligned(16))) float Bs[2][BROWS][BCOLS];

    const int nblocks = gridDim.x;
    int t = xcd_logical_block(blockIdx.x, nblocks);
    const int tn = t % a.tiles_n; t /= a.tiles_n;
    const int tm = t % a.tiles_m; t /= a.tiles_m;
    const int sp = t % a.split;
    const int g = t / a.split;

    const int m0 = tm * BM, n0 = tn * BN;
    const int k_begin = sp * a.k_chunk;
    const int k_end = min(a.K, k_begin + a.k_chunk);

    const int tid = threadIdx.x;
    const int lane = tid & 63;
    const int wave = tid >> 6;
    const int wm = wave / WN, wn = wave % WN;

    const float* __restrict__ Ag = a.A + (int64_t)g * a.sAg;
    const float* __restrict__ Bg = a.B + (int64_t)g * a.sBg;

    // per-thread A rows are fixed across the K loop: row = i*32 + tid/8
    float row_scale[A_LD];
    #pragma unroll
    for (int i = 0; i < A_LD; ++i) {
        row_scale[i] = 1.f;
        if (AMODE == kARowRecip) {
            const int m = m0 + i * 32 + (tid >> 3);
            if (m < a.M) row_scale[i] = 1.f / a.rs[(int64_t)m * a.rs_m + (int64_t)g * a.rs_g];
        }
    }

    v4f ra[A_LD], rb[B_LD];
    float rsc[A_LD];  // per-load A scale, applied when the slice is written to LDS so the
                      // multiply does not force a wait on the load ahead of the MFMAs

    auto load_slice = [&](int k0) {
        #pragma unroll
        for (int i = 0; i < A_LD; ++i) {
            const int m = m0 + i * 32 + (tid >> 3);
            const int k = k0 + 4 * (tid & 7);
            v4f v = {0.f, 0.f, 0.f, 0.f};
            if (m < a.M && k < k_end) {
                const float* src = Ag + (int64_t)m * a.lda + k;
                if (k + 3 < k_end) {
                    v = *reinterpret_cast<const v4f*>(src);
                } else {
                    #pragma unroll
                    for (int j = 0; j < 4; ++j) v[j] = (k + j < k_end) ? src[j] : 0.f;
                }
            }
            float sc = row_scale[i];
            if (AMODE == kAAlpha)
                sc = (m < a.M && k < k_end)
                         ? a.alpha[((int64_t)g * a.M + m) * a.alpha_ld + k / a.alpha_tile]
                         : 0.f;
            rsc[i] = sc;
            ra[i] = v;
        }
        #pragma unroll
        for (int i = 0; i < B_LD; ++i) {
            v4f v = {0.f, 0.f, 0.f, 0.f};
            if (NT) {
                const int n = n0 + i * 32 + (tid >> 3);
                const int k = k0 + 4 * (tid & 7);
                if (n < a.N && k < k_end) {
                    const float* src = Bg + (int64_t)n * a.ldb + k;
                    if (k + 3 < k_end) {
                        v = *reinterpret_cast<const v4f*>(src);
                    } else {
                        #pragma unroll
                        for (int j = 0; j < 4; ++j) v[j] = (k + j < k_end) ? src[j] : 0.f;
                    }
                }
            } else {
                const int e = i * kThreads + tid;
                const int k = k0 + e / (BN / 4);
                const int n = n0 + 4 * (e % (BN / 4));
                if (k < k_end && n < a.N)
                    v = *reinterpret_cast<const v4f*>(Bg + (int64_t)k * a.ldb + n);
            }
            rb[i] = v;
        }
    };

    auto store_slice = [&](int buf) {
        #pragma unroll
        for (int i = 0; i < A_LD; ++i)
            *reinterpret_cast<v4f*>(&As[buf][i * 32 + (tid >> 3)][4 * (tid & 7)]) =
                (AMODE == kAPlain) ? ra[i] : ra[i] * rsc[i];
        #pragma unroll
        for (int i = 0; i < B_LD; ++i) {
            if (NT) {
                *reinterpret_cast<v4f*>(&Bs[buf][i * 32 + (tid >> 3)][4 * (tid & 7)]) = rb[i];
            } else {
                const int e = i * kThreads + tid;
                *reinterpret_cast<v4f*>(&Bs[buf][e / (BN / 4)][4 * (e % (BN / 4))]) = rb[i];
            }
        }
    };

    v16f acc[TM][TN];
    #pragma unroll
    for (int i = 0; i < TM; ++i)
        #pragma unroll
        for (int j = 0; j < TN; ++j)
            #pragma unroll
            for (int e = 0; e < 16; ++e) acc[i][j][e] = 0.f;

    const int nslices = (k_end > k_begin) ? (k_end - k_begin + kBK - 1) / kBK : 0;
    if (nslices > 0) {
        load_slice(k_begin);
        store_slice(0);
    }
    __syncthreads();

    const int l32 = lane & 31;
    const int kq = 4 * (lane >> 5);
    for (int s = 0; s < nslices; ++s) {
        const int buf = s & 1;
        if (s + 1 < nslices) load_slice(k_begin + (s + 1) * kBK);

        #pragma unroll
        for (int kk = 0; kk < kBK; kk += 8) {
            v4f fa[TM], fb[TN];
            #pragma unroll
            for (int i = 0; i < TM; ++i)
                fa[i] = *reinterpret_cast<const v4f*>(&As[buf][wm * WTM + i * 32 + l32][kk + kq]);
            #pragma unroll
            for (int j = 0; j < TN; ++j) {
                if (NT) {
                    fb[j] = *reinterpret_cast<const v4f*>(
                        &Bs[buf][wn * WTN + j * 32 + l32][kk + kq]);
                } else {
                    #pragma unroll
                    for (int q = 0; q < 4; ++q)
                        fb[j][q] = Bs[buf][kk + kq + q][wn * WTN + j * 32 + l32];
                }
            }
            #pragma unroll
            for (int q = 0; q < 4; ++q)
                #pragma unroll
                for (int i = 0; i < TM; ++i)
                    #pragma unroll
                    for (int j = 0; j < TN; ++j)
                        acc[i][j] = mfma_32x32x2(fa[i][q], fb[j][q], acc[i][j]);
        }

        if (s + 1 < nslices) store_slice(buf ^ 1);
        __syncthreads();
    }

    // epilogue: each accumulator register holds one row; lanes 0-31 / 32-63 write
    // 32 consecutive columns of two rows.
    #pragma unroll
    for (int i = 0; i < TM; ++i) {
        #pragma unroll
        for (int j = 0; j < TN; ++j) {
            const int col = n0 + wn * WTN + j * 32 + l32;
            #pragma unroll
            for (int e = 0; e < 16; ++e) {
                const int row = m0 + wm * WTM + i * 32 + acc_row(e, lane);
                if (row < a.M && col < a.N) {
                    if (a.split > 1) {
                        a.ws[(int64_t)sp * a.ws_split + ((int64_t)g * a.M + row) * a.N + col] =
                            acc[i][j][e];
                    } else if (OUT == kOutF32) {
                        static_cast<float*>(a.C)[(int64_t)g * a.sCg + (int64_t)row * a.ldc + col] =
                            acc[i][j][e];
                    } else {
                        static_cast<__hip_bfloat16*>(a.C)[(int64_t)g * a.sCg +
                                                          (int64_t)row * a.ldc + col] =
                            __float2bfloat16(acc[i][j][e]);
                    }
                }
            }
        }
    }
}

// Sum split-K partials [split][G][M][N] in slice order into C.
template <int OUT>
__global__ void __launch_bounds__(256) split_reduce_kernel(const float* __restrict__ ws,
                                                           int64_t ws_split, int split,
                                                           void* C, int64_t ldc, int64_t sCg,
                                                           int G, int M, int N) {
    const int64_t total = (int64_t)G * M * N;
    for (int64_t idx = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; idx < total;
         idx += (int64_t)gridDim.x * blockDim.x) {
        float s = 0.f;
        for (int q = 0; q < split; ++q) s += ws[q * ws_split + idx];
        const int n = idx % N;
        const int64_t gm = idx / N;
        const int m = gm % M;
        const int g = gm / M;
        const int64_t off = (int64_t)g * sCg + (int64_t)m * ldc + n;
        if (OUT == kOutF32) static_cast<float*>(C)[off] = s;
        else static_cast<__hip_bfloat16*>(C)[off] = __float2bfloat16(s);
    }
}

template <int BM, int BN, int WM, int WN, bool NT, int AMODE, int OUT>
hipError_t launch_cfg(const GemmArgs& args, int nblocks, hipStream_t stream) {
    hipLaunchKernelGGL((gemm_kernel<BM, BN, WM, WN, NT, AMODE, OUT>), dim3(nblocks),
                       dim3(kThreads), 0, stream, args);
    return hipGetLastError();
}

template <bool NT, int AMODE, int OUT>
hipError_t launch_tiles(const GemmArgs& args, int bm, int bn, int nblocks,
                        hipStream_t stream) {
    if (bm == 128 && bn == 128) return launch_cfg<128, 128, 2, 2, NT, AMODE, OUT>(args, nblocks, stream);
    if (bm == 128 && bn == 96) return launch_cfg<128, 96, 4, 1, NT, AMODE, OUT>(args, nblocks, stream);
    if (bm == 128 && bn == 64) return launch_cfg<128, 64, 2, 2, NT, AMODE, OUT>(args, nblocks, stream);
    if (bm == 64 && bn == 128) return launch_cfg<64, 128, 2, 2, NT, AMODE, OUT>(args, nblocks, stream);
    if (bm == 64 && bn == 64) return launch_cfg<64, 64, 2, 2, NT, AMODE, OUT>(args, nblocks, stream);
    if (bm == 32 && bn == 128) return launch_cfg<32, 128, 1, 4, NT, AMODE, OUT>(args, nblocks, stream);
    if (bm == 128 && bn == 32) return launch_cfg<128, 32, 4, 1, NT, AMODE, OUT>(args, nblocks, stream);
    return hipErrorInvalidValue;
}

template <bool NT>
hipError_t dispatch_mode(const GemmArgs& args, AMode amode, OutType out, int bm, int bn,
                         int nblocks, hipStream_t stream) {
    // partial sums are always fp32; only a direct store converts
    if (out == kOutF32 || args.split > 1) {
        switch (amode) {
            case kAPlain: return launch_tiles<NT, kAPlain, kOutF32>(args, bm, bn, nblocks, stream);
            case kARowRecip: return launch_tiles<NT, kARowRecip, kOutF32>(args, bm, bn, nblocks, stream);
            case kAAlpha: return launch_tiles<NT, kAAlpha, kOutF32>(args, bm, bn, nblocks, stream);
        }
    } else {
        switch (amode) {
            case kAPlain: return launch_tiles<NT, kAPlain, kOutBF16>(args, bm, bn, nblocks, stream);
            case kARowRecip: return launch_tiles<NT, kARowRecip, kOutBF16>(args, bm, bn, nblocks, stream);
            case kAAlpha: return launch_tiles<NT, kAAlpha, kOutBF16>(args, bm, bn, nblocks, stream);
        }
    }
    return hipErrorInvalidValue;
}

int cdiv(int a, int b) { return (a + b - 1) / b; }

}  // namespace

// Tile and split choice: a small time model evaluated for every tile shape and power-of-two
// split.  MFMA time = rounds of co-resident workgroups x the padded tile work (32x32
// blocks waste rows/cols at small M or N) at a per-tile efficiency; memory time = the
// operand bytes that must come from HBM; split-K adds its fp32 partial traffic and one
// reduction launch.  MLA_GEMM_PLAN="M,N,K,G=bm,bn,split;..." forces a plan for a matching
// problem (tuning aid; the chosen plan always goes through the same validity checks).
namespace {

struct TileShape { int bm, bn; double eff; };
constexpr TileShape kTiles[] = {
    {128, 128, 0.80}, {128, 96, 0.78}, {128, 64, 0.72}, {64, 128, 0.72},
    {64, 64, 0.60},   {32, 128, 0.55}, {128, 32, 0.55}};

int lds_bytes(int bm, int bn, bool nt) {
    const int a = 2 * bm * (kBK + kPadK);
    const int b = nt ? 2 * bn * (kBK + kPadK) : 2 * kBK * (bn + kPadN);
    return (a + b) * 4;
}

bool tile_supported(int bm, int bn) {
    for (const auto& t : kTiles)
        if (t.bm == bm && t.bn == bn) return true;
    return false;
}

bool plan_override(const GemmProblem& p, GemmPlan* out) {
    const char* env = getenv("MLA_GEMM_PLAN");
    if (!env) return false;
    const char* s = env;
    while (*s) {
        long M, N, K, G;
        int bm, bn, split, used = 0;
        if (sscanf(s, "%ld,%ld,%ld,%ld=%d,%d,%d%n", &M, &N, &K, &G, &bm, &bn, &split, &used) == 7) {
            if (M == p.M && N == p.N && K == p.K && G == p.G && tile_supported(bm, bn) &&
                split >= 1) {
                out->bm = bm; out->bn = bn; out->split = split;
                return true;
            }
            s += used;
        } else {
            break;
        }
        while (*s == ';' || *s == ' ') ++s;
    }
    return false;
}

}  // namespace

GemmPlan plan_gemm(const GemmProblem& p) {
    constexpr double kCuRate = 256.0 * 2.4e9;   // fp32 MFMA flop/s per CU
    constexpr double kHbm = 5.0e12;             // sustained HBM B/s
    constexpr double kReduceLaunch = 3e-6;      // s
    const int kslices = cdiv(p.K, kBK);
    GemmPlan best;
    double best_t = 1e300;
    if (!plan_override(p, &best)) {
        for (const auto& t : kTiles) {
            const int tm = cdiv(p.M, t.bm), tn = cdiv(p.N, t.bn);
            const int64_t tiles = (int64_t)tm * tn * p.G;
            const int occ = std::max(1, std::min(2, 163840 / lds_bytes(t.bm, t.bn, p.b_nt)));
            for (int split = 1; split <= std::max(1, kslices / 2); split *= 2) {
                const int per = cdiv(kslices, split);
                const int real_split = cdiv(kslices, per);
                if (real_split != split && split > 1) continue;
                const int64_t blocks = tiles * split;
                // the busiest CU runs ceil(blocks / CUs) workgroups back to back or side by
                // side; a lone workgroup per CU hides latency worse than two
                const int64_t per_cu = (blocks + kNumCUs - 1) / kNumCUs;
                const double hide = std::min<int64_t>(per_cu, occ) >= 2 ? 1.0 : 0.8;
                const double wg_flops = 2.0 * t.bm * t.bn * (double)per * kBK;
                const double t_mfma = per_cu * wg_flops / (kCuRate * t.eff * hide);
                // B operand streamed once per M tile (weights / cache), A once per N tile
                // (small, mostly L2), C written once
                const double bytes = 4.0 * ((double)p.K * p.N * p.G * std::min(tm, 2) +
                                            (double)p.M * p.K * p.G + (double)p.M * p.N * p.G);
                double tt = std::max(t_mfma, bytes / kHbm);
                if (split > 1)
                    tt += 4.0 * (split + 1) * (double)p.M * p.N * p.G / kHbm + kReduceLaunch;
                if (tt < best_t * 0.999) {
                    best_t = tt;
                    best.bm = t.bm; best.bn = t.bn; best.split = split;
                }
            }
        }
    }
    const int per = cdiv(kslices, std::max(1, std::min(best.split, kslices)));
    best.k_chunk = per * kBK;
    best.split = cdiv(kslices, per);  // no empty slices
    best.workspace_bytes =
        best.split > 1 ? (size_t)best.split * p.G * p.M * p.N * sizeof(float) : 0;
    return best;
}

namespace {

hipError_t launch_gemm_impl(const GemmProblem& p, const GemmPlan& plan, void* workspace,
                            bool reduce, hipStream_t stream) {
    GemmArgs a;
    a.A = p.A; a.lda = p.lda; a.sAg = p.sAg;
    a.B = p.B; a.ldb = p.ldb; a.sBg = p.sBg;
    a.C = p.C; a.ldc = p.ldc; a.sCg = p.sCg;
    a.ws = static_cast<float*>(workspace);
    a.ws_split = (int64_t)p.G * p.M * p.N;
    a.M = p.M; a.N = p.N; a.K = p.K; a.G = p.G;
    a.split = plan.split; a.k_chunk = plan.k_chunk;
    a.tiles_m = cdiv(p.M, plan.bm);
    a.tiles_n = cdiv(p.N, plan.bn);
    a.rs = p.rs; a.rs_m = p.rs_m; a.rs_g = p.rs_g;
    a.alpha = p.alpha; a.alpha_ld = p.alpha_ld; a.alpha_tile = p.alpha_tile;
    const int64_t nblocks64 = (int64_t)a.tiles_m * a.tiles_n * a.G * a.split;
    if (nblocks64 <= 0 || nblocks64 > 0x7fffffff) return hipErrorInvalidValue;
    const int nblocks = (int)nblocks64;
    hipError_t e = p.b_nt ? dispatch_mode<true>(a, p.amode, p.out_type, plan.bm, plan.bn, nblocks, stream)
                          : dispatch_mode<false>(a, p.amode, p.out_type, plan.bm, plan.bn, nblocks, stream);
    if (e != hipSuccess || plan.split == 1 || !reduce) return e;
    const int64_t total = (int64_t)p.G * p.M * p.N;
    const int rblocks = (int)std::min<int64_t>((total + 255) / 256, 8 * kNumCUs);
    if (p.out_type == kOutF32)
        hipLaunchKernelGGL(split_reduce_kernel<kOutF32>, dim3(rblocks), dim3(256), 0, stream,
                           a.ws, a.ws_split, plan.split, p.C, p.ldc, p.sCg, p.G, p.M, p.N);
    else
        hipLaunchKernelGGL(split_reduce_kernel<kOutBF16>, dim3(rblocks), dim3(256), 0, stream,
                           a.ws, a.ws_split, plan.split, p.C, p.ldc, p.sCg, p.G, p.M, p.N);
    return hipGetLastError();
}

}  // namespace

hipError_t launch_gemm(const GemmProblem& p, const GemmPlan& plan, void* workspace,
                       hipStream_t stream) {
    return launch_gemm_impl(p, plan, workspace, true, stream);
}

hipError_t launch_gemm_partials(const GemmProblem& p, const GemmPlan& plan, float* partials,
                                hipStream_t stream) {
    if (plan.split <= 1) return hipErrorInvalidValue;
    return launch_gemm_impl(p, plan, partials, false, stream);
}

}  // namespace mla
