// 3a: latent scoring with the split-softmax epilogue.
//
// For a batch b the rows f = (s*H + h) of q_absorbed|q_rope form Q_b [Sq*H, R+D] and the
// keys form K_b = c_kv[b] | pe_cache[b]  [Sk, R+D]; the scores are Q_b K_b^T / scale, one
// (R+D)-deep reduction whose last D columns come from the second operand pair.
//
// Workgroup tile: 128 rows x 128 keys (one softmax partial).  Each of the 4 waves owns
// 32 rows x 128 keys = 4 MFMA accumulator blocks (fp32 or 16-bit steps, mma.h), so a row's 128 keys
// live in one wave: the row max and row sum need no LDS, only a 32-lane reduction
// (DPP + ds_swizzle) of each accumulator register.  Depth is walked in 128-byte slices
// (32 fp32 / 64 16-bit) staged through double-buffered LDS, exactly like the GEMM engine.
//
// Epilogue per row and 128-key tile j (mla_kernels.cu:971-1032 computes the same
// quantities): m_j = max over visible keys of t = s/scale, p = exp(t - m_j) stored into
// `scores` (0 for masked keys and for the row padding [Sk, ld_p)), l_j = sum p.
// Persistent grid: at most two workgroups per CU (the LDS and register budget), each walking
// a strided list of 128x128 tiles.  XCD x owns a contiguous range of the batch-major tile
// order and its workgroups interleave over it, so the tiles in flight on an XCD share one
// or two batches' Q rows in that XCD's L2.  The register prefetch ring runs straight
// across tile boundaries: the next tile's first slices are loaded while the current
// tile's last slices compute, so a tile switch exposes neither launch overhead nor the
// first slice's memory latency -- only the epilogue, which the CU's other workgroup
// covers with MFMA work.

#include "kernels.h"
#include "mma.h"

#include <algorithm>
#include <type_traits>

namespace mla {

namespace {

constexpr int kBM = 128, kBN = 128, kRowWords = 36, kThreads = 256;

struct ScoresArgs {
    const void* qa; const void* qr; const void* ckv; const void* pe;
    float* p; float* m_part; float* l_part;
    int B, Sq, Sk, H, R, D, ld_p, P, tiles_r, tiles;
    int64_t key_stride;   // key rows between batches
    int causal_base;      // sk_total - Sq - key_offset: query s sees local keys <= base + s
    float scale_log2;   // log2(e) / scale
    int causal;
    // ragged / paged keys (both optional): batch b has seq_lens[b] keys, and its key rows
    // [j*page_size, (j+1)*page_size) live in page block_table[b*max_pages + j] of ckv / pe
    const int* seq_lens;
    const int* block_table;
    int page_size, max_pages;
};

// Keys of batch b (Sk for a uniform batch).
__device__ __forceinline__ int batch_keys(const ScoresArgs& a, int b) {
    return a.seq_lens ? min(load_uniform(a.seq_lens + b), a.Sk) : a.Sk;
}

// First key row (in rows of ckv / pe) of the 64 keys [k, k + 64) of batch b: dense rows
// are b*key_stride + k; paged rows go through the block table (page_size is a multiple of
// 64, so 64 keys never straddle a page).  Keys at or past Sk read no table entry.
__device__ __forceinline__ int64_t key_row(const ScoresArgs& a, int b, int k) {
    if (!a.block_table) return (int64_t)b * a.key_stride + k;
    const int page =
        k < a.Sk ? load_uniform(a.block_table + (int64_t)b * a.max_pages + k / a.page_size) : 0;
    return (int64_t)page * a.page_size + k % a.page_size;
}

// Tile t of the batch-major order: key tile kt = t % P, row tile tr = (t / P) % tiles_r,
// batch b = t / (P * tiles_r).
struct TileId {
    int b, r0, k0, kt;
};
__device__ __forceinline__ TileId tile_id(const ScoresArgs& a, int t) {
    TileId id;
    id.kt = t % a.P;
    const int u = t / a.P;
    id.r0 = (u % a.tiles_r) * kBM;
    id.b = u / a.tiles_r;
    id.k0 = id.kt * kBN;
    return id;
}

// PD = depth of the register prefetch ring: while slice s feeds the MFMAs from LDS, slices
// s+1 .. s+PD are in flight from global memory.  fp32 is MFMA-bound with ~4K MFMA cycles
// per slice and uses PD = 1; 16-bit slices hold 8x less MFMA work and keep two slices in
// flight (PD = 2).
// PARTIAL: R or D is not a whole number of slices, so a slice's column chunks past the row
// width must read as zeros (a per-load mask that whole slices do without).
template <typename TL, int PD, bool PARTIAL>
__global__ void __launch_bounds__(kThreads, 2) scores_kernel(ScoresArgs a) {
    using MM = Mma<TL>;
    constexpr int E = MM::kElems, KS = MM::kSlice;
    __shared__ __attribute__((aligned(16))) uint32_t Qs[2][kBM][kRowWords];
    __shared__ __attribute__((aligned(16))) uint32_t Ks[2][kBN][kRowWords];

    // this workgroup's tiles: t_first, t_first + nbx, ... below x_hi
    const int x = blockIdx.x % kNumXCDs, jx = blockIdx.x / kNumXCDs;
    const int nbx = gridDim.x / kNumXCDs + (x < (int)(gridDim.x % kNumXCDs) ? 1 : 0);
    const int per_x = a.tiles / kNumXCDs, rem_x = a.tiles % kNumXCDs;
    const int x_lo = x * per_x + min(x, rem_x);
    const int x_hi = x_lo + per_x + (x < rem_x ? 1 : 0);
    if (x_lo + jx >= x_hi) return;   // whole workgroup: no barrier is left waiting

    const int rows_b = a.Sq * a.H;             // rows of a batch
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int l32 = lane & 31, half = lane >> 5;

    const int nsl_r = (a.R + KS - 1) / KS;
    const int nsl = nsl_r + (a.D + KS - 1) / KS;

    // Staging geometry: thread tid loads 16-byte chunk tid%8 of tile rows i*32 + tid/8
    // (i = 0..3) of Q and of K.  Byte offsets are relative to the slice's first column of
    // the tile's first row; latent (R-wide) and rope (D-wide) rows have their own strides.
    // Rows beyond a tile's valid count carry the kOob bit, folded in once per tile.
    uint32_t o_r[4], o_d[4];
    #pragma unroll
    for (int i = 0; i < 4; ++i) {
        const uint32_t row = i * 32 + (tid >> 3), cb = 16u * (tid & 7);
        o_r[i] = row * (uint32_t)(a.R * sizeof(TL)) + cb;
        o_d[i] = row * (uint32_t)(a.D * sizeof(TL)) + cb;
    }

    // load cursor: tile lt, slice ls; its operand tile origins and per-row offsets (every
    // row masked once lt runs past the list, so the ring's surplus loads return zeros)
    // K rows come in two 64-row halves (staging rows i = 0,1 and i = 2,3), each with its
    // own origin, so a paged cache with 64-key pages needs no per-lane address math.
    int lt = x_lo + jx, ls = 0;
    const TL *lqa, *lqr, *lka[2], *lkr[2];
    uint32_t oq_r[4], oq_d[4], ok_r[4], ok_d[4];
    auto set_load_tile = [&]() __attribute__((always_inline)) {
        const bool live = lt < x_hi;
        const TileId id = tile_id(a, live ? lt : x_lo);
        const int64_t qrow = (int64_t)id.b * rows_b + id.r0;
        lqa = static_cast<const TL*>(a.qa) + qrow * a.R;
        lqr = static_cast<const TL*>(a.qr) + qrow * a.D;
        #pragma unroll
        for (int h = 0; h < 2; ++h) {
            const int64_t krow = key_row(a, id.b, id.k0 + 64 * h);
            lka[h] = static_cast<const TL*>(a.ckv) + krow * a.R;
            lkr[h] = static_cast<const TL*>(a.pe) + krow * a.D;
        }
        const int qv = live ? min(kBM, rows_b - id.r0) : 0;
        const int kv = live ? min(kBN, batch_keys(a, id.b) - id.k0) : 0;
        #pragma unroll
        for (int i = 0; i < 4; ++i) {
            const int row = i * 32 + (tid >> 3);
            const uint32_t mq = oob_mask(row, qv), mk = oob_mask(row, kv);
            oq_r[i] = o_r[i] | mq; oq_d[i] = o_d[i] | mq;
            ok_r[i] = o_r[i & 1] | mk; ok_d[i] = o_d[i & 1] | mk;   // offsets within the half
        }
    };
    auto advance_load = [&]() __attribute__((always_inline)) {
        if (++ls == nsl) {
            ls = 0;
            lt += nbx;
            set_load_tile();
        }
    };

    v4u rq[PD][4], rk[PD][4];
    auto load_slice = [&](int slot) __attribute__((always_inline)) {
        const bool rope = ls >= nsl_r;
        const int c0 = rope ? (ls - nsl_r) * KS : ls * KS;
        const __amdgpu_buffer_rsrc_t rsq = make_rsrc((rope ? lqr : lqa) + c0);
        const __amdgpu_buffer_rsrc_t rsk0 = make_rsrc((rope ? lkr[0] : lka[0]) + c0);
        const __amdgpu_buffer_rsrc_t rsk1 = make_rsrc((rope ? lkr[1] : lka[1]) + c0);
        uint32_t cmask = 0;
        if constexpr (PARTIAL) cmask = oob_mask(E * (tid & 7), (rope ? a.D : a.R) - c0);
        #pragma unroll
        for (int i = 0; i < 4; ++i) {
            rq[slot][i] = load16(rsq, (rope ? oq_d[i] : oq_r[i]) | cmask);
            rk[slot][i] = load16(i < 2 ? rsk0 : rsk1, (rope ? ok_d[i] : ok_r[i]) | cmask);
        }
    };
    auto store_slice = [&](int buf, int slot) __attribute__((always_inline)) {
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

    // ---- epilogue of tile t: per accumulator register e the lane holds tile row
    // rr(e) = wave*32 + acc_row(e, lane) and keys k0 + 32*j + l32 (j = 0..3).  Work in the
    // log2 domain with c = log2(e)/scale: m2 = c * (row max of the raw scores) equals the
    // max of the scaled scores exactly (c > 0 and rounding are monotonic), p = 2^(s*c - m2)
    // is one fma and one v_exp_f32, and m = m2 * ln(2) is stored in the natural units of
    // s/scale.  Every instruction here costs MFMA time -- fp32 MFMAs and VALU work do not
    // overlap on a SIMD -- so full non-causal tiles take a path without visibility masks.
    // Stores are buffer stores whose offsets carry the kOob bit for rows past the tile and
    // for lanes that do not own a row's m / l, so no store branches.
    auto epilogue = [&](int t, auto causal_tag, auto full_tag) __attribute__((always_inline)) {
        constexpr bool kCausal = decltype(causal_tag)::value;
        constexpr bool kFull = decltype(full_tag)::value;     // all 128 keys visible
        const TileId id = tile_id(a, t);
        const int64_t row0 = (int64_t)id.b * rows_b + id.r0;   // first row of the tile
        const int rv = min(kBM, rows_b - id.r0);                // valid rows
        const int skb = batch_keys(a, id.b);
        const int kvis = min(kBN, skb - id.k0);                 // keys before the padding
        const int kcols = min(kBN, a.ld_p - id.k0);             // columns inside the p row
        const float c = a.scale_log2;
        const __amdgpu_buffer_rsrc_t rsp = make_rsrc(a.p + row0 * a.ld_p + id.k0);
        const __amdgpu_buffer_rsrc_t rsm = make_rsrc(a.m_part + row0 * a.P + id.kt);
        const __amdgpu_buffer_rsrc_t rsl = make_rsrc(a.l_part + row0 * a.P + id.kt);
        const uint32_t ml_lane = oob_mask(l32, 1);              // lane 0 of each half-wave
        // the lane's first tile row, made opaque here so the compiler does not hoist the
        // sixteen rows' offsets out of the tile loop (they would stay live through it)
        int rr0 = wave * 32 + 4 * half;
        asm volatile("" : "+v"(rr0));
        #pragma unroll
        for (int e = 0; e < 16; ++e) {
            const int rr = rr0 + 8 * (e >> 2) + (e & 3);       // wave*32 + acc_row(e, lane)
            const uint32_t rmask = oob_mask(rr, rv);
            int klast = kvis - 1;                               // last visible key, tile-relative
            if constexpr (kCausal) {
                // query index s = r / H sees absolute keys <= Sk_total - Sq + s
                const int r = min(id.r0 + rr, rows_b - 1);
                const int cbase = a.seq_lens ? skb - a.Sq : a.causal_base;
                klast = min(klast, cbase + r / a.H - id.k0);
            }
            float mx;
            if constexpr (kFull) {
                mx = fmaxf(fmaxf(acc[0][e], acc[1][e]), fmaxf(acc[2][e], acc[3][e]));
            } else {
                mx = -INFINITY;
                #pragma unroll
                for (int j = 0; j < 4; ++j)
                    if (32 * j + l32 <= klast) mx = fmaxf(mx, acc[j][e]);
            }
            const float m2 = half_wave_reduce(mx, OpMax()) * c;
            float sum = 0.f;
            const uint32_t prow = ((uint32_t)(rr * a.ld_p + l32) * 4u) | rmask;
            #pragma unroll
            for (int j = 0; j < 4; ++j) {
                float pv = __builtin_amdgcn_exp2f(__builtin_fmaf(acc[j][e], c, -m2));
                if constexpr (!kFull) pv = (32 * j + l32 <= klast) ? pv : 0.f;
                sum += pv;
                // ld_p and k0 are multiples of 32: a 32-key group is all in or all out
                if (kFull || 32 * j < kcols)
                    __builtin_amdgcn_raw_buffer_store_b32(__float_as_uint(pv), rsp,
                                                          (int)(prow + 128u * j), 0, 0);
            }
            sum = half_wave_reduce(sum, OpSum());
            const uint32_t mloff = ((uint32_t)(rr * a.P) * 4u) | rmask | ml_lane;
            __builtin_amdgcn_raw_buffer_store_b32(__float_as_uint(m2 * 0.69314718055994531f), rsm,
                                                  (int)mloff, 0, 0);   // * ln 2
            __builtin_amdgcn_raw_buffer_store_b32(__float_as_uint(sum), rsl, (int)mloff, 0, 0);
        }
    };

    set_load_tile();
    #pragma unroll
    for (int u = 0; u < PD; ++u) {
        load_slice(u);
        advance_load();
    }
    store_slice(0, 0);
    __syncthreads();

    // compute cursor: tile ct, slice cs.  Global slice g sits in LDS buffer g&1 and came
    // from ring slot g%PD.  One slice step per ring slot, instantiated with the slot as a
    // compile-time constant (a runtime slot index would turn the ring into indexed
    // register moves that wait for every load).  Returns true when the list is done.
    int ct = x_lo + jx, cs = 0;
    auto slice_step = [&](int g, auto slot_tag) __attribute__((always_inline)) -> bool {
        constexpr int u = decltype(slot_tag)::value;
        const int buf = g & 1;
        load_slice(u);   // global slice g + PD
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
        advance_load();
        if (++cs < nsl) return false;
        if (a.causal)
            epilogue(ct, std::true_type(), std::false_type());
        else if ((ct % a.P + 1) * kBN <= batch_keys(a, ct / (a.P * a.tiles_r)))
            epilogue(ct, std::false_type(), std::true_type());
        else
            epilogue(ct, std::false_type(), std::false_type());
        #pragma unroll
        for (int j = 0; j < 4; ++j)
            #pragma unroll
            for (int e = 0; e < 16; ++e) acc[j][e] = 0.f;
        cs = 0;
        ct += nbx;
        return ct >= x_hi;
    };
    static_assert(PD == 1 || PD == 2, "ring depth 1 or 2");
    for (int g = 0;; g += PD) {
        if (slice_step(g, std::integral_constant<int, 0>())) break;
        if constexpr (PD == 2)
            if (slice_step(g + 1, std::integral_constant<int, 1>())) break;
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
    a.seq_lens = p.seq_lens; a.block_table = p.block_table;
    a.page_size = p.page_size; a.max_pages = p.max_pages;
    if (p.block_table && (p.page_size <= 0 || p.page_size % 64 != 0 ||
                          (int64_t)p.max_pages * p.page_size < p.Sk))
        return hipErrorInvalidValue;
    // every staging offset (a row of the 128-row tile) must stay below the buffer range
    const int64_t row_bytes = (int64_t)std::max(p.R, p.D) * (p.half ? 2 : 4);
    if (kBM * row_bytes >= kRsrcRange || (int64_t)kBM * p.ld_p * 4 >= kRsrcRange)
        return hipErrorInvalidValue;
    const int64_t tiles = (int64_t)p.B * a.tiles_r * a.P;
    if (tiles <= 0 || tiles > 0x7fffffff) return hipErrorInvalidValue;
    a.tiles = (int)tiles;
    // two resident workgroups per CU (launch bounds and 74 KB of LDS each)
    const int64_t nblocks = std::min<int64_t>(tiles, 2 * kNumCUs);
    const dim3 grid((unsigned)nblocks), block(kThreads);
    const int ks = p.half ? 64 : 32;   // slice width
    const bool partial = p.R % ks != 0 || p.D % ks != 0;
    if (p.half && p.f16) {
        if (partial) hipLaunchKernelGGL((scores_kernel<f16_t, 2, true>), grid, block, 0, stream, a);
        else hipLaunchKernelGGL((scores_kernel<f16_t, 2, false>), grid, block, 0, stream, a);
    } else if (p.half) {
        if (partial) hipLaunchKernelGGL((scores_kernel<bf16_t, 2, true>), grid, block, 0, stream, a);
        else hipLaunchKernelGGL((scores_kernel<bf16_t, 2, false>), grid, block, 0, stream, a);
    } else {
        if (partial) hipLaunchKernelGGL((scores_kernel<float, 1, true>), grid, block, 0, stream, a);
        else hipLaunchKernelGGL((scores_kernel<float, 1, false>), grid, block, 0, stream, a);
    }
    return hipGetLastError();
}

}  // namespace mla
