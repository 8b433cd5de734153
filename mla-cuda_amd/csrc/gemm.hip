// Batched MFMA GEMM for the layer's dense contractions, fp32, bf16 or fp16:
//   2a1 / 2a2  x @ W_q_a, q_lat @ W_q_b          (NN, G = 1)
//   2c         q_nope[h] @ W_uk[h]                (NN, G = heads)
//   3c         (p * alpha) @ c_kv[b]              (NN, G = batch, A scaled by alpha)
//   3d         (ctx[h] / row_sum) @ W_uv[h]^T     (NT, G = heads, A scaled by 1/row_sum)
//
// Workgroup = 4 wave64s.  A BM x BN output tile is split 2x2 / 4x1 / 1x4 over the waves,
// each wave covering its sub-tile with 32x32 MFMA accumulator blocks
// (v_mfma_f32_32x32x2_f32, or the 32x32x16 bf16 / fp16 MFMA in the 16-bit paths; see
// mma.h).  K is walked in slices of 128 bytes per row (32 fp32 / 64 16-bit) staged through
// double-buffered LDS: the next slice's 128-bit global loads are in flight while the
// current slice feeds the MFMAs.  Within a slice, K is permuted so each lane's operands
// for one K step are 16 contiguous bytes: one ds_read_b128 per fragment for K-contiguous
// operands, four ds_read_b32 (fp32) / eight ds_read_u16 (16-bit) for N-contiguous ones.
// In the 16-bit paths, fp32 A operands (q_raw, p, ctx) are scaled in fp32 and rounded to
// the storage format (nearest even) as they are written to LDS.
//
// LDS rows of K-contiguous tiles are 144 B (128 B + 16 B pad): the eight lanes of a
// ds_read_b128 / ds_write_b128 phase then land on disjoint bank groups.  N-contiguous
// tiles are padded so the row read by the second half-wave is 32 banks away from the
// first half-wave's row.  The measured LDS bank-conflict counter is 0 for every kernel.
//
// Split-K is deterministic: slices write fp32 partials to a workspace and a reduction
// kernel (or the consumer, for 2a1) sums them in a fixed order -- no float atomics.

#include "mma.h"
#include "kernels.h"

#include <algorithm>
#include <cstdio>
#include <cstdlib>
#include <cstring>
#include <type_traits>

namespace mla {

namespace {

constexpr int kRowWords = 36;   // K-contiguous LDS row: 128 B of K + 16 B pad, in words
constexpr int kThreads = 256;

struct GemmArgs {
    const void* A; int64_t lda, sAg;
    const void* B; int64_t ldb, sBg;
    void* C; int64_t ldc, sCg;
    float* ws; int64_t ws_split;   // partials [split][G][M][N] when split > 1
    int M, N, K, G;
    int split, k_chunk, tiles_m, tiles_n;
    const float* rs; int64_t rs_m, rs_g;
    const float* alpha; int alpha_ld, alpha_shift;   // alpha column of k: k >> alpha_shift
    const int* k_len;                                  // per-group K limit (optional)
    const int* b_pages; int page_size, max_pages;      // paged NN B (PAGED kernels)
    // ROPE kernels (fp32 2a2 with 2b in its epilogue): the rope columns of every head go
    // rotated to rope_out [M][H][rope] instead of C, with row m's pair i at
    // rope_cs[2 (m * rope/2 + i)] (cos) and the sin after it
    float* rope_out; const float* rope_cs; int rope_H, rope_nope, rope_rope;
};

template <typename TL, int BN>
constexpr int nn_row_words() {
    // BN elements plus a pad that puts the second half-wave's row 32 banks away
    return BN * (int)sizeof(TL) / 4 + (sizeof(TL) == 4 ? 8 : 4);
}

// TL: LDS / MFMA element type (float, bf16_t or f16_t).  TA: global element type of A
// (float, or TL when TL is 16-bit).  B is always TL in global memory.
// PD = depth of the register prefetch ring (slices in flight while one feeds the MFMAs):
// 2 -- one slice of MFMA work (~4K cycles per wave in fp32, 8x less in bf16) does not
// cover the HBM latency of a long-K stream such as 3c's scores x c_kv; with two slices in
// flight 3c runs at ~83% of the fp32 MFMA peak instead of ~78%.
// PAGED: the NN B operand is a paged row pool -- K row k of group g is row
// b_pages[g*max_pages + k/page_size]*page_size + k%page_size (page_size a multiple of 64,
// so a K slice never straddles a page); used by 3c over a paged KV cache.
// PERSIST: the grid holds fewer workgroups than tiles; workgroup w walks the tiles w',
// w' + grid, ... (w' its XCD-aware logical index) and its load ring runs on across tile
// boundaries, so the next tile's first slices are in flight during the current tile's
// last ones and the epilogue's stores drain under the next tile's MFMA work.  Short-K
// products (2c: K = 128, four slices) otherwise spend about a third of a tile in the
// unoverlapped fill and epilogue.  Full tiles only, plain A, no per-group K limit or
// paging (the launcher checks).
// ROPE: fp32 C of 2a2 whose 32-column blocks in a head's rope part are rotated (2b) and
// written to rope_out instead (the pair partner of column c is column c ^ 1, the
// neighbouring lane), with the arithmetic of rope_kernel, so the bits are the same.
template <typename TL, typename TA, int BM, int BN, int WM, int WN, bool NT, int AMODE, int OUT,
          bool PAGED = false, bool PERSIST = false, bool ROPE = false>
__global__ void __launch_bounds__(kThreads, 2) gemm_kernel(GemmArgs a) {
    constexpr int PD = 2;
    using MM = Mma<TL>;
    constexpr int E = MM::kElems;          // elements per 16-byte chunk
    constexpr int KS = MM::kSlice;         // K elements per slice
    constexpr int WTM = BM / WM, WTN = BN / WN;
    constexpr int TM = WTM / 32, TN = WTN / 32;
    static_assert(WM * WN == 4 && TM >= 1 && TN >= 1, "4 waves, 32x32 blocks");
    constexpr int A_LD = BM / 32;          // 16-byte LDS chunks per thread per slice (A)
    constexpr int B_LD = BN / 32;          // ... (B, both layouts)
    // bf16 N-contiguous B (weights, c_kv) is transposed while staging so LDS holds it
    // K-contiguous like an NT operand: each of 2*BN threads loads a 4-row x 8-column block
    // and writes eight 8-byte k-runs; every fragment is then one ds_read_b128 instead of
    // eight ds_read_u16 (which made the bf16 NN kernels LDS-issue bound).
    constexpr bool TRN = !NT && sizeof(TL) == 2;
    constexpr int BROWS = (NT || TRN) ? BN : KS;
    constexpr int BWORDS = (NT || TRN) ? kRowWords : nn_row_words<TL, BN>();
    constexpr bool A_F32 = std::is_same<TA, float>::value;
    constexpr int A_F4 = A_F32 ? E / 4 : 1;  // float4 loads per A chunk
    // instruction counts of one slice, for its issue schedule
    constexpr int kStepReads = TM + TN * ((NT || TRN) ? 1 : 2);   // fp32 NN B: 2 ds_read2_b32
    constexpr int kSliceLoads = A_LD * A_F4 + (TRN ? 4 : B_LD) + (AMODE == kAAlpha ? A_LD : 0);
    constexpr int kSliceWrites = A_LD + (TRN ? 8 : B_LD);
    static_assert(A_F32 || AMODE == kAPlain, "scaled A operands are fp32");
    static_assert(!PERSIST || (AMODE == kAPlain && !PAGED), "persistent tiles: plain A only");

    __shared__ __attribute__((aligned(16))) uint32_t As[2][BM][kRowWords];
    __shared__ __attribute__((aligned(16))) uint32_t Bs[2][BROWS][BWORDS];

    int t = xcd_logical_block(blockIdx.x, gridDim.x);
    const int tn = t % a.tiles_n; t /= a.tiles_n;
    const int tm = t % a.tiles_m; t /= a.tiles_m;
    const int sp = t % a.split;
    const int g = t / a.split;

    const int m0 = tm * BM, n0 = tn * BN;
    const int k_begin = sp * a.k_chunk;
    const int k_end = min(a.k_len ? min(a.K, load_uniform(a.k_len + g)) : a.K,
                          k_begin + a.k_chunk);

    const int tid = threadIdx.x;
    const int lane = tid & 63;
    const int wave = tid >> 6;
    const int wm = wave / WN, wn = wave % WN;

    const TA* __restrict__ Ag = static_cast<const TA*>(a.A) + (int64_t)g * a.sAg;
    const TL* __restrict__ Bg = static_cast<const TL*>(a.B) + (int64_t)g * a.sBg;

    // per-thread A rows are fixed across the K loop: row = i*32 + tid/8
    float row_scale[A_LD];
    #pragma unroll
    for (int i = 0; i < A_LD; ++i) {
        row_scale[i] = 1.f;
        if (AMODE == kARowRecip) {
            const int m = m0 + i * 32 + (tid >> 3);
            // a row without visible keys (row sum 0, ctx 0) gives zeros, as the oracle's
            // softmax over no keys does
            const float rs = m < a.M ? a.rs[(int64_t)m * a.rs_m + (int64_t)g * a.rs_g] : 1.f;
            row_scale[i] = rs == 0.f ? 0.f : 1.f / rs;
        }
    }

    // Staging geometry, fixed for the whole tile.  Byte offsets are relative to the current
    // slice's origin in each operand (the scalar base walks K); rows or columns outside the
    // problem get kOob.  K-contiguous tiles (A, NT B): thread tid loads chunk tid%8 of rows
    // i*32 + tid/8.  N-contiguous B: chunk e%(BN/E) of K row e/(BN/E), e = i*256 + tid;
    // transposed bf16 B: rows 4*(tid%16) + i, columns 8*(tid/16).
    const int kc = E * (tid & 7);                  // chunk column within the slice
    uint32_t oa[A_LD], oal[A_LD];
    #pragma unroll
    for (int i = 0; i < A_LD; ++i) {
        const int r = i * 32 + (tid >> 3);
        const bool ok = m0 + r < a.M;
        oa[i] = ok ? (uint32_t)(((int64_t)r * a.lda + kc) * sizeof(TA)) : kOob;
        oal[i] = ok ? (uint32_t)((int64_t)r * a.alpha_ld * 4) : kOob;
    }
    constexpr int NB_LD = TRN ? 4 : B_LD;
    uint32_t ob[NB_LD];
    int bk[NB_LD];                                 // K row of a N-contiguous B chunk
    #pragma unroll
    for (int i = 0; i < NB_LD; ++i) {
        if constexpr (TRN) {
            const int gq = tid & 15, c = tid >> 4;
            bk[i] = 4 * gq + i;
            ob[i] = (tid < 2 * BN && n0 + 8 * c < a.N)
                        ? (uint32_t)(((int64_t)bk[i] * a.ldb + 8 * c) * sizeof(TL)) : kOob;
        } else if constexpr (NT) {
            const int r = i * 32 + (tid >> 3);
            bk[i] = 0;
            ob[i] = (n0 + r < a.N) ? (uint32_t)(((int64_t)r * a.ldb + kc) * sizeof(TL)) : kOob;
        } else {
            const int e = i * kThreads + tid;
            const int nc = E * (e % (BN / E));
            bk[i] = e / (BN / E);
            ob[i] = (n0 + nc < a.N) ? (uint32_t)(((int64_t)bk[i] * a.ldb + nc) * sizeof(TL)) : kOob;
        }
    }
    const TA* A_t = Ag + (int64_t)m0 * a.lda;
    const TL* B_t = NT ? Bg + (int64_t)n0 * a.ldb : Bg + n0;
    const float* al_t = (AMODE == kAAlpha) ? a.alpha + ((int64_t)g * a.M + m0) * a.alpha_ld : nullptr;

    // staging registers: fp32 A is kept as floats (scaled and, in the bf16 path, rounded
    // only when written to LDS, so the multiply does not wait on the load ahead of the
    // MFMAs); bf16 A and all B chunks are raw 16-byte words
    v4f raf[PD][A_LD][A_F4];
    v4u ra[PD][A_LD];
    float rsc[PD][A_LD];
    v4u rb[PD][NB_LD];

    // Slices at or past k_end load zeros (every column or K-row test fails), so the ring
    // needs no bounds branches; the zeros land in an LDS buffer nobody reads.
    // paged B: the pool row of the next slice to load, looked up one slice ahead so the
    // scalar load's latency hides behind a slice of MFMA work
    int64_t page_row = 0;
    auto lookup_row = [&](int k0) -> int64_t {
        if constexpr (!PAGED) return 0;
        const int pg = k0 < k_end
                           ? load_uniform(a.b_pages + (int64_t)g * a.max_pages + k0 / a.page_size)
                           : 0;
        return (int64_t)pg * a.page_size + k0 % a.page_size;
    };
    if constexpr (PAGED) page_row = lookup_row(k_begin);

    // one slice's global loads into ring slot `slot`: A_s / B_s are the slice's origins,
    // klim its valid K columns (A, NT B) or K rows (NN B); k0 indexes alpha
    auto issue_loads = [&](const TA* A_s, const TL* B_s, int k0, int klim, int slot) {
        const __amdgpu_buffer_rsrc_t rsa = make_rsrc(A_s);
        const __amdgpu_buffer_rsrc_t rsb = make_rsrc(B_s);
        #pragma unroll
        for (int i = 0; i < A_LD; ++i) {
            if constexpr (A_F32) {
                #pragma unroll
                for (int f = 0; f < A_F4; ++f)
                    raf[slot][i][f] = __builtin_bit_cast(
                        v4f, load16(rsa, (oa[i] + 16u * f) | oob_mask(kc + 4 * f, klim)));
            } else {
                ra[slot][i] = load16(rsa, oa[i] | oob_mask(kc, klim));
            }
            float sc = row_scale[i];
            if constexpr (AMODE == kAAlpha) {
                // one alpha per 128-key tile: every chunk of a slice shares k0 / alpha_tile
                const __amdgpu_buffer_rsrc_t rsl = make_rsrc(al_t + (k0 >> a.alpha_shift));
                sc = load_f32(rsl, oal[i] | oob_mask(kc, klim));
            }
            rsc[slot][i] = sc;
        }
        #pragma unroll
        for (int i = 0; i < NB_LD; ++i)
            rb[slot][i] = load16(rsb, ob[i] | oob_mask(NT ? kc : bk[i], klim));
    };
    auto load_slice = [&](int k0, int slot) {
        const TL* B_s = NT ? B_t + k0 : B_t + (PAGED ? page_row : (int64_t)k0) * a.ldb;
        if constexpr (PAGED) page_row = lookup_row(k0 + KS);
        issue_loads(A_t + k0, B_s, k0, k_end - k0, slot);
    };

    auto store_slice = [&](int buf, int slot) {
        #pragma unroll
        for (int i = 0; i < A_LD; ++i) {
            v4u w;
            if constexpr (A_F32 && sizeof(TL) == 4) {
                const v4f f = (AMODE == kAPlain) ? raf[slot][i][0] : raf[slot][i][0] * rsc[slot][i];
                w = __builtin_bit_cast(v4u, f);
            } else if constexpr (A_F32) {
                const float s = (AMODE == kAPlain) ? 1.f : rsc[slot][i];
                const v4f f0 = raf[slot][i][0] * s, f1 = raf[slot][i][A_F4 - 1] * s;
                w = v4u{Half<TL>::pack2(f0[0], f0[1]), Half<TL>::pack2(f0[2], f0[3]),
                        Half<TL>::pack2(f1[0], f1[1]), Half<TL>::pack2(f1[2], f1[3])};
            } else {
                w = ra[slot][i];
            }
            *reinterpret_cast<v4u*>(&As[buf][i * 32 + (tid >> 3)][4 * (tid & 7)]) = w;
        }
        if constexpr (TRN) {
            if (tid < 2 * BN) {
                const int g = tid & 15, c = tid >> 4;
                #pragma unroll
                for (int j = 0; j < 8; ++j) {
                    // column j of the 4x8 block: k-pairs (rows 0,1) and (rows 2,3)
                    const int w = j >> 1, hi = j & 1;
                    const uint32_t r0 = rb[slot][0][w], r1 = rb[slot][1][w];
                    const uint32_t r2 = rb[slot][2][w], r3 = rb[slot][3][w];
                    const uint32_t lo01 = hi ? ((r0 >> 16) | (r1 & 0xffff0000u)) : ((r0 & 0xffffu) | (r1 << 16));
                    const uint32_t lo23 = hi ? ((r2 >> 16) | (r3 & 0xffff0000u)) : ((r2 & 0xffffu) | (r3 << 16));
                    *reinterpret_cast<uint2*>(&Bs[buf][8 * c + j][2 * g]) = make_uint2(lo01, lo23);
                }
            }
            return;
        }
        #pragma unroll
        for (int i = 0; i < B_LD; ++i) {
            if (NT) {
                *reinterpret_cast<v4u*>(&Bs[buf][i * 32 + (tid >> 3)][4 * (tid & 7)]) = rb[slot][i];
            } else {
                const int e = i * kThreads + tid;
                *reinterpret_cast<v4u*>(&Bs[buf][e / (BN / E)][4 * (e % (BN / E))]) = rb[slot][i];
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

    const int l32 = lane & 31;
    const int half = lane >> 5;
    // one slice of MFMA work from LDS buffer buf
    auto mma_slice = [&](int buf) {
        #pragma unroll
        for (int st = 0; st < 4; ++st) {
            v4u fa[TM], fb[TN];
            #pragma unroll
            for (int i = 0; i < TM; ++i)
                fa[i] = *reinterpret_cast<const v4u*>(&As[buf][wm * WTM + i * 32 + l32][8 * st + 4 * half]);
            #pragma unroll
            for (int j = 0; j < TN; ++j) {
                const int n = wn * WTN + j * 32 + l32;
                if (NT || TRN) {
                    fb[j] = *reinterpret_cast<const v4u*>(&Bs[buf][n][8 * st + 4 * half]);
                } else if constexpr (sizeof(TL) == 4) {
                    #pragma unroll
                    for (int q = 0; q < 4; ++q) fb[j][q] = Bs[buf][8 * st + 4 * half + q][n];
                } else {
                    const uint16_t* b16 = reinterpret_cast<const uint16_t*>(&Bs[buf][0][0]);
                    const int r0 = 16 * st + 8 * half;
                    #pragma unroll
                    for (int q = 0; q < 4; ++q)
                        fb[j][q] = (uint32_t)b16[(r0 + 2 * q) * (2 * BWORDS) + n] |
                                   ((uint32_t)b16[(r0 + 2 * q + 1) * (2 * BWORDS) + n] << 16);
                }
            }
            #pragma unroll
            for (int q = 0; q < MM::kSub; ++q)
                #pragma unroll
                for (int i = 0; i < TM; ++i)
                    #pragma unroll
                    for (int j = 0; j < TN; ++j) acc[i][j] = MM::sub(fa[i], fb[j], q, acc[i][j]);
        }
    };

    // epilogue: each accumulator register holds one row; lanes 0-31 / 32-63 write
    // 32 consecutive columns of two rows.  Buffer stores from one descriptor per tile:
    // the lane's column (and its block's first row) is a per-lane offset fixed for the
    // block, the register's row a wave-uniform offset, and rows or columns past the
    // problem carry kOob -- no branches and no 64-bit address arithmetic per element.
    auto epilogue = [&](int g_, int m0_, int n0_, int sp_) {
        const bool to_ws = a.split > 1;
        const int64_t ld = to_ws ? a.N : a.ldc;
        constexpr bool kF32Out = (OUT == kOutF32);
        const int esz = (to_ws || kF32Out) ? 4 : 2;
        const __amdgpu_buffer_rsrc_t rso =
            to_ws ? make_rsrc(a.ws + (int64_t)sp_ * a.ws_split + ((int64_t)g_ * a.M + m0_) * a.N + n0_)
                  : (kF32Out ? make_rsrc(static_cast<float*>(a.C) + (int64_t)g_ * a.sCg +
                                         (int64_t)m0_ * a.ldc + n0_)
                             : make_rsrc(static_cast<uint16_t*>(a.C) + (int64_t)g_ * a.sCg +
                                         (int64_t)m0_ * a.ldc + n0_));
        #pragma unroll
        for (int i = 0; i < TM; ++i) {
            #pragma unroll
            for (int j = 0; j < TN; ++j) {
                const int c = wn * WTN + j * 32 + l32;              // tile column
                const int r0 = wm * WTM + i * 32 + 4 * half;          // tile row of e = 0
                if constexpr (ROPE) {
                    // a block of a head's rope part (uniform over the wave): rotate
                    const int qk = a.rope_nope + a.rope_rope;
                    const int c0 = n0_ + wn * WTN + j * 32;
                    const int hh = c0 / qk, j0 = c0 - hh * qk;
                    if (c0 < a.N && j0 >= a.rope_nope) {
                        const int half_r = a.rope_rope >> 1;
                        const int rc = j0 - a.rope_nope + l32;     // rope column of the head
                        const int pi = rc >> 1;
                        float* dst = a.rope_out + (int64_t)hh * a.rope_rope + rc;
                        const int64_t ld_r = (int64_t)a.rope_H * a.rope_rope;
                        // all 16 rows' (cos, sin) loads first, then the rotations and stores
                        // (a load after a store to rope_out would wait for it)
                        typedef float v2f_t __attribute__((ext_vector_type(2)));
                        v2f_t cs[16];
                        #pragma unroll
                        for (int e = 0; e < 16; ++e) {
                            const int row = min(m0_ + r0 + 8 * (e >> 2) + (e & 3), a.M - 1);
                            cs[e] = *reinterpret_cast<const v2f_t*>(
                                a.rope_cs + 2 * ((int64_t)row * half_r + pi));
                        }
                        #pragma unroll
                        for (int e = 0; e < 16; ++e) {
                            const float own = acc[i][j][e];
                            const float other = dpp_move<0xB1>(own);   // lane ^ 1
                            const int row = m0_ + r0 + 8 * (e >> 2) + (e & 3);
                            if (row < a.M)
                                dst[(int64_t)row * ld_r] =
                                    (l32 & 1) ? rope_odd(other, own, cs[e][0], cs[e][1])
                                              : rope_even(own, other, cs[e][0], cs[e][1]);
                        }
                        continue;
                    }
                }
                const uint32_t lane_off =
                    (uint32_t)((r0 * ld + c) * esz) | oob_mask(n0_ + c, a.N);
                #pragma unroll
                for (int e = 0; e < 16; ++e) {
                    const int re = 8 * (e >> 2) + (e & 3);
                    const int soff = __builtin_amdgcn_readfirstlane((int)(re * ld * esz));
                    const uint32_t off = lane_off | oob_mask(m0_ + r0 + re, a.M);
                    if (to_ws || kF32Out) {
                        __builtin_amdgcn_raw_buffer_store_b32(__float_as_uint(acc[i][j][e]), rso,
                                                              (int)off, soff, 0);
                    } else if constexpr (!kF32Out) {
                        __builtin_amdgcn_raw_buffer_store_b16(
                            (uint16_t)Store16<OUT>::bits(acc[i][j][e]), rso, (int)off, soff, 0);
                    }
                }
            }
        }
    };

    // Both loops below are unrolled by PD so every ring slot index is a compile-time
    // constant, and run a multiple of PD slices: a slice past the end loads zeros (every
    // offset fails its K test) and adds nothing.  An exit between the unrolled bodies would
    // give the compiler a path back to the loop head with a slot's loads still in flight,
    // and the wait counts it derives for the head would then drain the ring every slice.
    if constexpr (!PERSIST) {
        const int nslices = (k_end > k_begin) ? (k_end - k_begin + KS - 1) / KS : 0;
        const int nslices_pd = (nslices + PD - 1) / PD * PD;
        #pragma unroll
        for (int u = 0; u < PD; ++u) load_slice(k_begin + u * KS, u);
        store_slice(0, 0);
        __syncthreads();

        // slice s sits in LDS buffer s&1 and came from ring slot s%PD
        for (int s0 = 0; s0 < nslices_pd; s0 += PD) {
            #pragma unroll
            for (int u = 0; u < PD; ++u) {
                const int s = s0 + u;
                const int buf = (PD == 1) ? (s & 1) : (u & 1);
                load_slice(k_begin + (s + PD) * KS, u);
                mma_slice(buf);
                store_slice(buf ^ 1, (u + 1) % PD);
                sched_slice<kStepReads, MM::kSub * TM * TN, kSliceLoads, kSliceWrites>();
                __syncthreads();
            }
        }
        epilogue(g, m0, n0, sp);
    } else {
        // Every tile has ns = k_chunk / KS slices (the last split's tail slices load
        // zeros); the workgroup's tiles run as one stream of my_tiles * ns slices.  The load
        // cursor (l_*) runs PD slices ahead of the compute cursor (c_*); past the last tile
        // it loads zeros (klim 0: every offset gets kOob, nothing is read).
        const int stride = gridDim.x;
        const int n_tiles = a.tiles_m * a.tiles_n * a.split * a.G;
        const int first = xcd_logical_block(blockIdx.x, gridDim.x);
        const int my_tiles = (n_tiles - 1 - first) / stride + 1;   // grid <= n_tiles
        const int ns = a.k_chunk / KS;
        const int total = (my_tiles * ns + PD - 1) / PD * PD;
        struct Tile { int g, m0, n0, sp; };
        auto decode = [&](int tile) {
            int t = tile;
            const int tn_ = t % a.tiles_n; t /= a.tiles_n;
            const int tm_ = t % a.tiles_m; t /= a.tiles_m;
            return Tile{t / a.split, tm_ * BM, tn_ * BN, t % a.split};
        };
        int l_tile = first, l_s = 0;
        const TA* l_A = A_t;
        const TL* l_B = B_t;
        int l_kb = k_begin, l_ke = k_end;
        auto persist_load = [&](int slot) {
            const int k0 = l_kb + l_s * KS;
            const int klim = l_tile < n_tiles ? l_ke - k0 : 0;
            issue_loads(l_A + k0, NT ? l_B + k0 : l_B + (int64_t)k0 * a.ldb, k0, klim, slot);
            if (++l_s == ns) {
                l_s = 0;
                l_tile += stride;
                if (l_tile < n_tiles) {
                    const Tile t = decode(l_tile);
                    l_A = static_cast<const TA*>(a.A) + (int64_t)t.g * a.sAg + (int64_t)t.m0 * a.lda;
                    const TL* Bg_ = static_cast<const TL*>(a.B) + (int64_t)t.g * a.sBg;
                    l_B = NT ? Bg_ + (int64_t)t.n0 * a.ldb : Bg_ + t.n0;
                    l_kb = t.sp * a.k_chunk;
                    l_ke = min(a.K, l_kb + a.k_chunk);
                }
            }
        };
        #pragma unroll
        for (int u = 0; u < PD; ++u) persist_load(u);
        store_slice(0, 0);
        __syncthreads();

        int c_tile = first, c_s = 0;
        for (int v0 = 0; v0 < total; v0 += PD) {
            #pragma unroll
            for (int u = 0; u < PD; ++u) {
                const int buf = u & 1;
                persist_load(u);
                mma_slice(buf);
                store_slice(buf ^ 1, (u + 1) % PD);
                sched_slice<kStepReads, MM::kSub * TM * TN, kSliceLoads, kSliceWrites>();
                __syncthreads();
                // after the barrier, so the slice body above stays one scheduling region;
                // the stores drain while the next slices' MFMAs run
                if (++c_s == ns && c_tile < n_tiles) {
                    const Tile t = decode(c_tile);
                    epilogue(t.g, t.m0, t.n0, t.sp);
                    #pragma unroll
                    for (int i = 0; i < TM; ++i)
                        #pragma unroll
                        for (int j = 0; j < TN; ++j)
                            #pragma unroll
                            for (int e = 0; e < 16; ++e) acc[i][j][e] = 0.f;
                    c_s = 0;
                    c_tile += stride;
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
        if constexpr (OUT == kOutF32) static_cast<float*>(C)[off] = s;
        else static_cast<uint16_t*>(C)[off] = (uint16_t)Store16<OUT>::bits(s);
    }
}

template <typename TL, typename TA, int BM, int BN, int WM, int WN, bool NT, int AMODE, int OUT,
          bool PAGED, bool PERSIST, bool ROPE>
hipError_t launch_cfg(const GemmArgs& args, int nblocks, hipStream_t stream) {
    hipLaunchKernelGGL((gemm_kernel<TL, TA, BM, BN, WM, WN, NT, AMODE, OUT, PAGED, PERSIST, ROPE>),
                       dim3(nblocks), dim3(kThreads), 0, stream, args);
    return hipGetLastError();
}

template <typename TL, typename TA, bool NT, int AMODE, int OUT, bool PAGED = false,
          bool PERSIST = false, bool ROPE = false>
hipError_t launch_tiles(const GemmArgs& args, int bm, int bn, int nblocks, hipStream_t stream) {
#define MLA_TILE(BM_, BN_, WM_, WN_)                                                       \
    if (bm == BM_ && bn == BN_)                                                             \
        return launch_cfg<TL, TA, BM_, BN_, WM_, WN_, NT, AMODE, OUT, PAGED, PERSIST, ROPE>( \
            args, nblocks, stream);
    MLA_TILE(128, 128, 2, 2)
    MLA_TILE(128, 96, 4, 1)
    MLA_TILE(128, 64, 2, 2)
    MLA_TILE(64, 128, 2, 2)
    MLA_TILE(64, 64, 2, 2)
    MLA_TILE(32, 128, 1, 4)
    MLA_TILE(128, 32, 4, 1)
#undef MLA_TILE
    return hipErrorInvalidValue;
}

// The operand/epilogue combinations the layer uses (others are rejected):
//   fp32:  NN plain  -> f32 (2a1, 2a2, 2c) | NN alpha -> f32 (3c) | NT rowrecip -> f32 (3d)
//   16-bit (bf16 or fp16, TL): NN plain, A 16-bit -> f32 (2a1, 2a2) or -> 16-bit (wo) |
//          NN plain, A f32 -> 16-bit (2c) | NN alpha, A f32 -> f32 (3c) |
//          NT rowrecip, A f32 -> 16-bit (3d)
// A split-K launch writes fp32 partials whatever the output type.
template <typename TL>
hipError_t dispatch16(const GemmProblem& p, const GemmArgs& a, int bm, int bn, int nblocks,
                      bool persist, hipStream_t stream) {
    constexpr int O16 = Half<TL>::kF16 ? kOutF16 : kOutBF16;
    const bool split = a.split > 1;
    const bool f32_out = split || p.out_type == kOutF32;
    if (!f32_out && p.out_type != O16) return hipErrorInvalidValue;
    if (persist) {   // NN plain with f32 output or partials (2c, 2a1, 2a2)
        if (p.b_nt || p.amode != kAPlain || p.b_pages || !f32_out || p.a_f32)
            return hipErrorInvalidValue;
        return launch_tiles<TL, TL, false, kAPlain, kOutF32, false, true>(a, bm, bn, nblocks,
                                                                           stream);
    }
    if (p.b_pages) {   // paged NN B: 3c over a paged cache only
        if (p.b_nt || p.amode != kAAlpha || !f32_out || !p.a_f32) return hipErrorInvalidValue;
        return launch_tiles<TL, float, false, kAAlpha, kOutF32, true>(a, bm, bn, nblocks, stream);
    }
    if (!p.b_nt && p.amode == kAPlain && !p.a_f32) {
        if (f32_out) return launch_tiles<TL, TL, false, kAPlain, kOutF32>(a, bm, bn, nblocks, stream);
        return launch_tiles<TL, TL, false, kAPlain, O16>(a, bm, bn, nblocks, stream);
    }
    if (!p.b_nt && p.amode == kAPlain && p.a_f32) {
        if (f32_out) return launch_tiles<TL, float, false, kAPlain, kOutF32>(a, bm, bn, nblocks, stream);
        return launch_tiles<TL, float, false, kAPlain, O16>(a, bm, bn, nblocks, stream);
    }
    if (!p.b_nt && p.amode == kAAlpha && p.a_f32 && f32_out)
        return launch_tiles<TL, float, false, kAAlpha, kOutF32>(a, bm, bn, nblocks, stream);
    if (p.b_nt && p.amode == kAPlain && !p.a_f32) {   // 3d from a normalised 16-bit ctx
        if (f32_out) return launch_tiles<TL, TL, true, kAPlain, kOutF32>(a, bm, bn, nblocks, stream);
        return launch_tiles<TL, TL, true, kAPlain, O16>(a, bm, bn, nblocks, stream);
    }
    if (p.b_nt && p.amode == kARowRecip && p.a_f32) {
        if (f32_out)
            return launch_tiles<TL, float, true, kARowRecip, kOutF32>(a, bm, bn, nblocks, stream);
        return launch_tiles<TL, float, true, kARowRecip, O16>(a, bm, bn, nblocks, stream);
    }
    return hipErrorInvalidValue;
}

hipError_t dispatch(const GemmProblem& p, const GemmArgs& a, int bm, int bn, int nblocks,
                    bool persist, hipStream_t stream) {
    if (p.half)
        return p.f16 ? dispatch16<f16_t>(p, a, bm, bn, nblocks, persist, stream)
                     : dispatch16<bf16_t>(p, a, bm, bn, nblocks, persist, stream);
    const bool split = a.split > 1;
    const bool f32_out = split || p.out_type == kOutF32;
    if (persist) {   // NN plain with f32 output or partials (2c, 2a1, 2a2)
        if (p.b_nt || p.amode != kAPlain || p.b_pages || !f32_out) return hipErrorInvalidValue;
        return launch_tiles<float, float, false, kAPlain, kOutF32, false, true>(a, bm, bn,
                                                                               nblocks, stream);
    }
    if (p.b_pages) {   // paged NN B: 3c over a paged cache only
        if (p.b_nt || p.amode != kAAlpha || !f32_out) return hipErrorInvalidValue;
        return launch_tiles<float, float, false, kAAlpha, kOutF32, true>(a, bm, bn, nblocks, stream);
    }
    if (!p.b_nt && p.amode == kAPlain && f32_out && a.rope_out) {
        if (split) return hipErrorInvalidValue;
        return launch_tiles<float, float, false, kAPlain, kOutF32, false, false, true>(
            a, bm, bn, nblocks, stream);
    }
    if (!p.b_nt && p.amode == kAPlain && f32_out)
        return launch_tiles<float, float, false, kAPlain, kOutF32>(a, bm, bn, nblocks, stream);
    if (!p.b_nt && p.amode == kAAlpha && f32_out)
        return launch_tiles<float, float, false, kAAlpha, kOutF32>(a, bm, bn, nblocks, stream);
    if (p.b_nt && p.amode == kARowRecip && f32_out)
        return launch_tiles<float, float, true, kARowRecip, kOutF32>(a, bm, bn, nblocks, stream);
    return hipErrorInvalidValue;
}

int cdiv(int a, int b) { return (a + b - 1) / b; }

}  // namespace

// Tile and split choice: a small time model evaluated for every tile shape and power-of-two
// split.  MFMA time = rounds of co-resident workgroups x the padded tile work (32x32
// blocks waste rows/cols at small M or N) at a per-tile efficiency; memory time = the
// operand bytes that must come from HBM; split-K adds its fp32 partial traffic and one
// reduction launch.  MLA_GEMM_PLAN="M,N,K,G=bm,bn,split[,tiles_per_wg];..." forces a plan
// for a matching problem (tuning aid; the chosen plan always goes through the same validity
// checks).
namespace {

struct TileShape { int bm, bn; double eff; };
constexpr TileShape kTiles[] = {
    {128, 128, 0.80}, {128, 96, 0.78}, {128, 64, 0.72}, {64, 128, 0.72},
    {64, 64, 0.60},   {32, 128, 0.55}, {128, 32, 0.55}};

int lds_bytes(int bm, int bn, bool nt, bool half) {
    const int a = 2 * bm * kRowWords * 4;
    const int nn_row = half ? bn * 2 + 16 : bn * 4 + 32;
    // 16-bit N-contiguous B is staged transposed, i.e. in the NT layout
    const int b = (nt || half) ? 2 * bn * kRowWords * 4 : 2 * 32 * nn_row;
    return a + b;
}

// Measured-best plans for the GEMM shapes of the DeepSeek-V3 layer and its neighbours on
// MI355X: a sweep of every tile x power-of-two split per shape, keeping the fastest (ties
// within ~1% go to the model's choice).  Exact shape matches only; every other shape goes
// through the time model below.  M = B*Sq for the Q path / wo / KV append, M = H for 3c.
// The last column is the tiles per workgroup of a persistent grid (1: one per tile); 2c
// at B = 128 runs 128x64 tiles two per workgroup, 30.5 us against 32.8 us for one 128x128
// tile per workgroup.
struct TunedPlan { int M, N, K, G; bool nt, half; int bm, bn, split, tiles_per_wg = 1; };
constexpr TunedPlan kTuned[] = {
    // B = 128 decode, fp32: 2a1, 2a2, 2c, 3d, wo, kv
    {128, 1536, 7168, 1, false, false, 64, 64, 16},
    {128, 24576, 1536, 1, false, false, 64, 64, 1},
    {128, 512, 128, 128, false, false, 128, 64, 1, 2},
    {128, 128, 512, 128, true, false, 64, 64, 1},
    {128, 7168, 16384, 1, false, false, 128, 32, 8},
    {128, 576, 7168, 1, false, false, 64, 64, 8},
    // B = 128 decode, bf16
    {128, 1536, 7168, 1, false, true, 128, 64, 8},
    {128, 24576, 1536, 1, false, true, 128, 96, 1},
    {128, 512, 128, 128, false, true, 128, 128, 1},
    {128, 128, 512, 128, true, true, 32, 128, 1},
    {128, 7168, 16384, 1, false, true, 128, 128, 8},
    {128, 576, 7168, 1, false, true, 64, 64, 8},
    // B = 1, 8, 32 decode, fp32: 2a1, 2a2, 2c, 3d
    {1, 1536, 7168, 1, false, false, 32, 128, 16},
    {1, 24576, 1536, 1, false, false, 32, 128, 4},
    {1, 512, 128, 128, false, false, 32, 128, 1},
    {1, 128, 512, 128, true, false, 32, 128, 1},
    {8, 1536, 7168, 1, false, false, 32, 128, 16},
    {8, 24576, 1536, 1, false, false, 32, 128, 4},
    {8, 512, 128, 128, false, false, 32, 128, 1},
    {8, 128, 512, 128, true, false, 32, 128, 1},
    {32, 1536, 7168, 1, false, false, 32, 128, 16},
    {32, 24576, 1536, 1, false, false, 32, 128, 2},
    {32, 512, 128, 128, false, false, 32, 128, 1},
    {32, 128, 512, 128, true, false, 64, 64, 1},
};

bool tuned_plan(const GemmProblem& p, GemmPlan* out) {
    for (const auto& t : kTuned)
        if (t.M == p.M && t.N == p.N && t.K == p.K && t.G == p.G && t.nt == p.b_nt &&
            t.half == p.half) {
            out->bm = t.bm; out->bn = t.bn; out->split = t.split;
            out->tiles_per_wg = t.tiles_per_wg;
            return true;
        }
    return false;
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
        int bm, bn, split, used = 0, per_wg = 1, used2 = 0;
        if (sscanf(s, "%ld,%ld,%ld,%ld=%d,%d,%d%n", &M, &N, &K, &G, &bm, &bn, &split, &used) == 7) {
            if (sscanf(s + used, ",%d%n", &per_wg, &used2) == 1) used += used2;
            if (M == p.M && N == p.N && K == p.K && G == p.G && tile_supported(bm, bn) &&
                split >= 1 && per_wg >= 1) {
                out->bm = bm; out->bn = bn; out->split = split; out->tiles_per_wg = per_wg;
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

// Weight-streaming plans (wgemm.hip), exact shapes: 16-bit products whose weight operand
// dominates the traffic.  MLA_WGEMM=0 turns the engine off (every shape goes to the tiled
// engine); MLA_WGEMM_PLAN="M,N,K,G=bn,split[,stages];..." forces a weight-streaming plan for a
// matching problem (tuning aid, same validity checks).
struct WTunedPlan { int M, N, K, G; bool nt; int bn, split, stages; };
constexpr WTunedPlan kWTuned[] = {
    // B = 128 decode, bf16 / fp16: 2a1, 2a2, and the output projection beside the layer
    // (63 -> 52 us; the KV projection gained nothing and stays tiled)
    {128, 1536, 7168, 1, false, 64, 8, 4},
    {128, 24576, 1536, 1, false, 128, 1, 4},
    {128, 7168, 16384, 1, false, 128, 4, 4},
    // 3d from the normalised 16-bit ctx (NT, G = heads): 256 workgroups of 64 columns, the
    // bf16 attention with 3d 172.4-173.1 us against 174.2-175.7 us on the tiled engine
    {128, 128, 512, 128, true, 64, 1, 4},
};

bool wgemm_plan(const GemmProblem& p, GemmPlan* out) {
    const char* off = getenv("MLA_WGEMM");
    if (off && strcmp(off, "0") == 0) return false;
    int bn = 0, split = 0, stages = 4;
    if (const char* env = getenv("MLA_WGEMM_PLAN")) {
        const char* s = env;
        while (*s && !bn) {
            long M, N, K, G;
            int b, sp, used = 0, used2 = 0, ns = 4;
            if (sscanf(s, "%ld,%ld,%ld,%ld=%d,%d%n", &M, &N, &K, &G, &b, &sp, &used) != 6) break;
            if (sscanf(s + used, ",%d%n", &ns, &used2) == 1) used += used2;
            if (M == p.M && N == p.N && K == p.K && G == p.G) { bn = b; split = sp; stages = ns; }
            s += used;
            while (*s == ';' || *s == ' ') ++s;
        }
    }
    for (const auto& t : kWTuned)
        if (!bn && t.M == p.M && t.N == p.N && t.K == p.K && t.G == p.G && t.nt == p.b_nt) {
            bn = t.bn; split = t.split; stages = t.stages;
        }
    const bool ring_ok = (bn == 256 && stages == 3 && !p.b_nt) ||
                         (bn == 128 && (stages == 3 || stages == 4)) ||
                         (bn == 64 && (stages == 3 || stages == 4 || (stages == 6 && !p.b_nt)));
    if (!bn || split < 1 || !ring_ok || !wgemm_supported(p, bn, split)) return false;
    const int kslices = cdiv(p.K, 64);
    const int per = cdiv(kslices, std::min(split, kslices));
    if (!wgemm_supported(p, bn, cdiv(kslices, per))) return false;
    out->bm = 128; out->bn = bn; out->split = split; out->tiles_per_wg = 1; out->wgemm = true;
    out->stages = stages;
    return true;
}

}  // namespace

GemmPlan plan_gemm(const GemmProblem& p) {
    // fp32 MFMA: 256 flop/clk/CU at 2.4 GHz; dense bf16 MFMA is 16x that
    const double kCuRate = 256.0 * 2.4e9 * (p.half ? 16.0 : 1.0);
    constexpr double kHbm = 5.0e12;             // sustained HBM B/s
    constexpr double kReduceLaunch = 3e-6;      // s
    const int kBK = p.half ? 64 : 32;           // K per slice
    const double eb = p.half ? 2.0 : 4.0;       // bytes per B element
    const double ea = p.a_f32 || !p.half ? 4.0 : 2.0;
    const int kslices = cdiv(p.K, kBK);
    GemmPlan best;
    double best_t = 1e300;
    if (!wgemm_plan(p, &best) && !plan_override(p, &best) && !tuned_plan(p, &best)) {
        for (const auto& t : kTiles) {
            const int tm = cdiv(p.M, t.bm), tn = cdiv(p.N, t.bn);
            const int64_t tiles = (int64_t)tm * tn * p.G;
            const int occ = std::max(1, std::min(2, 163840 / lds_bytes(t.bm, t.bn, p.b_nt, p.half)));
            for (int split = 1; split <= std::max(1, kslices / 2); split *= 2) {
                const int per = cdiv(kslices, split);
                const int real_split = cdiv(kslices, per);
                if (real_split != split && split > 1) continue;
                const int64_t blocks = tiles * split;
                // the busiest CU runs ceil(blocks / CUs) workgroups back to back or side by
                // side; a lone workgroup per CU hides latency worse than two
                const int64_t per_cu = (blocks + kNumCUs - 1) / kNumCUs;
                const double hide = std::min<int64_t>(per_cu, occ) >= 2 ? 1.0 : 0.8;
                // a workgroup's first slices and its epilogue are not overlapped with MFMA
                // work: about four slices' worth of pipeline fill and drain
                const double fill = per / (per + 4.0);
                const double wg_flops = 2.0 * t.bm * t.bn * (double)per * kBK;
                const double t_mfma = per_cu * wg_flops / (kCuRate * t.eff * hide * fill);
                // HBM reaches its sustained rate only with ~2 workgroups per CU streaming
                const double conc = std::min(1.0, (double)blocks / (2.0 * kNumCUs));
                // B operand streamed once per M tile (weights / cache), A once per N tile
                // (small, mostly L2), C written once
                const double bytes = eb * (double)p.K * p.N * p.G * std::min(tm, 2) +
                                     ea * (double)p.M * p.K * p.G + 4.0 * (double)p.M * p.N * p.G;
                double tt = std::max(t_mfma, bytes / (kHbm * conc));
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
    best.k_chunk = per * kBK;  // whole slices; the kernel's slice is the same kBK
    best.split = cdiv(kslices, per);  // no empty slices
    best.workspace_bytes =
        best.split > 1 ? (size_t)best.split * p.G * p.M * p.N * sizeof(float) : 0;
    return best;
}

namespace {

// Sum split-K partials into C, converting to the output type.
hipError_t split_reduce(const GemmProblem& p, const GemmArgs& a, int split, hipStream_t stream) {
    const int64_t total = (int64_t)p.G * p.M * p.N;
    const int rblocks = (int)std::min<int64_t>((total + 255) / 256, 8 * kNumCUs);
    if (p.out_type == kOutF32)
        hipLaunchKernelGGL(split_reduce_kernel<kOutF32>, dim3(rblocks), dim3(256), 0, stream,
                           a.ws, a.ws_split, split, p.C, p.ldc, p.sCg, p.G, p.M, p.N);
    else if (p.out_type == kOutBF16)
        hipLaunchKernelGGL(split_reduce_kernel<kOutBF16>, dim3(rblocks), dim3(256), 0, stream,
                           a.ws, a.ws_split, split, p.C, p.ldc, p.sCg, p.G, p.M, p.N);
    else
        hipLaunchKernelGGL(split_reduce_kernel<kOutF16>, dim3(rblocks), dim3(256), 0, stream,
                           a.ws, a.ws_split, split, p.C, p.ldc, p.sCg, p.G, p.M, p.N);
    return hipGetLastError();
}

hipError_t launch_gemm_impl(const GemmProblem& p, const GemmPlan& plan, void* workspace,
                            bool reduce, hipStream_t stream) {
    // the epilogue addresses a tile's rows with 32-bit offsets from the tile's first row
    const int64_t out_ld = plan.split > 1 ? p.N : p.ldc;
    if ((int64_t)plan.bm * out_ld * 4 >= (int64_t)kRsrcRange) return hipErrorInvalidValue;
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
    a.alpha = p.alpha; a.alpha_ld = p.alpha_ld;
    a.k_len = p.k_len; a.b_pages = p.b_pages; a.page_size = p.page_size; a.max_pages = p.max_pages;
    a.rope_out = nullptr; a.rope_cs = nullptr; a.rope_H = a.rope_nope = a.rope_rope = 0;
    if (p.rope_epi) {
        // fp32 2a2 with 2b in its epilogue: one K split, plain NN, fp32 C, every 32-column
        // block inside one head's nope or rope part
        const QUpEpilogue& q = *p.rope_epi;
        if (p.half || plan.wgemm || plan.split != 1 || plan.tiles_per_wg > 1 || p.b_nt ||
            p.amode != kAPlain || p.out_type != kOutF32 || p.G != 1 || !q.q_rope ||
            !q.cos_sin || q.H <= 0 || q.nope <= 0 || q.nope % 32 != 0 || q.rope <= 0 ||
            q.rope % 32 != 0 || (int64_t)p.N != (int64_t)q.H * (q.nope + q.rope))
            return hipErrorInvalidValue;
        a.rope_out = static_cast<float*>(q.q_rope); a.rope_cs = q.cos_sin;
        a.rope_H = q.H; a.rope_nope = q.nope; a.rope_rope = q.rope;
    }
    if (p.b_pages && (p.page_size <= 0 || p.page_size % 64 != 0 ||
                      (int64_t)p.max_pages * p.page_size < p.K))
        return hipErrorInvalidValue;
    a.alpha_shift = 0;
    if (p.amode == kAAlpha) {
        // one alpha per slice: the tile is a power of two and a multiple of the slice
        const int ks = p.half ? 64 : 32;
        if (p.alpha_tile < ks || (p.alpha_tile & (p.alpha_tile - 1)) != 0) return hipErrorInvalidValue;
        while ((1 << a.alpha_shift) < p.alpha_tile) ++a.alpha_shift;
    }
    // every staging offset (a row of a 128-row tile) must stay below the buffer range
    const int64_t ea = (p.a_f32 || !p.half) ? 4 : 2, eb = p.half ? 2 : 4;
    if (128 * std::max({p.lda * ea, p.ldb * eb, (int64_t)p.alpha_ld * 4}) >= kRsrcRange)
        return hipErrorInvalidValue;
    const int64_t nblocks64 = (int64_t)a.tiles_m * a.tiles_n * a.G * a.split;
    if (nblocks64 <= 0 || nblocks64 > 0x7fffffff) return hipErrorInvalidValue;
    if (p.qup && !(plan.wgemm && wgemm_aligned(p))) return hipErrorInvalidValue;
    if (plan.wgemm && wgemm_aligned(p)) {
        const hipError_t e = launch_wgemm(p, plan, a.ws, stream);
        if (e != hipSuccess || plan.split == 1 || !reduce) return e;
        return split_reduce(p, a, plan.split, stream);
    }
    int nblocks = (int)nblocks64;
    // persistent grid: full tiles of a plain NN product with no per-group K limit; any
    // other problem keeps one workgroup per tile
    const bool persist = plan.tiles_per_wg > 1 && p.M % plan.bm == 0 && p.N % plan.bn == 0 &&
                         !p.b_nt && p.amode == kAPlain && !p.k_len && !p.b_pages &&
                         (p.out_type == kOutF32 || plan.split > 1) && (!p.half || !p.a_f32) &&
                         plan.k_chunk % (p.half ? 64 : 32) == 0;
    if (persist) nblocks = cdiv(nblocks, plan.tiles_per_wg);
    hipError_t e = dispatch(p, a, plan.bm, plan.bn, nblocks, persist, stream);
    if (e != hipSuccess || plan.split == 1 || !reduce) return e;
    return split_reduce(p, a, plan.split, stream);
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
