// 3a + 3b + 3c fused for bf16 storage: one pass over the latent cache per key split.
//
// The per-step path materialises fp32 scores (3a), reduces per-tile softmax partials
// (3b) and streams c_kv a second time for ctx (3c).  With bf16 storage that path is
// HBM-bound on traffic it creates itself: at B=128, Sk=4989 it moves ~2.0 GB, of which
// only 0.74 GB is the cache.  This kernel reads every key row once, keeps the softmax
// state in registers and writes only the unnormalised ctx, its row sums and row maxima.
// The arithmetic is the reference's (mla_kernels.cu:971-1032, 1058-1079, 1247-1254):
// s = q_absorbed.c_kv + q_rope.pe, softmax over s/scale, ctx = sum_k p_k c_kv[k]; only the
// order of operations differs (an online softmax instead of per-tile partials).
//
// Workgroup: 4 waves over 64 rows (queries x heads) of one batch and one contiguous key
// range (a split).  Wave w = (rb, cw) = (w & 1, w >> 1) owns rows 32rb .. 32rb+31; the two
// waves of a row block split the work of each 32-key block between them:
//   partial S^T[32 keys x 32 rows] over depth half cw (18 bf16 MFMA K steps of the
//     576-deep row; that half of Q^T lives in 72 VGPRs for the whole kernel), exchanged
//     through LDS and summed in the same order by both waves
//   online softmax per row (duplicated in both waves): every lane holds one row (column
//     l%32 of the accumulator) and 16 of the block's keys, its partner lane l^32 the other 16
//   O^T[256 cols x 32 rows] += V_blk^T . P^T for column half cw (P^T is the S^T
//     accumulator rounded to bf16, used in place as the B operand; O^T is 128 registers)
// V_blk^T fragments come from the same key-major LDS tile as K_blk through gfx950's
// transposing ds_read_b64_tr_b16, so c_kv is staged once per workgroup, by direct
// global->LDS loads (buffer_load_dwordx4 ... lds) into a ring of NS blocks: NS-1 blocks are
// in flight while one is computed, with no VGPRs spent on staging.  The two 64-row tiles of
// a batch are placed on one XCD, so the second read of every key block hits its L2.
//
// LDS tile of a block (36 KB): 32 latent rows of 1 KB, then 32 rope rows of 128 B.  The
// 16-byte chunk c of key k sits at chunk c ^ f(k & 7), f(k) = 2(k & 3) + (k >> 2), which
// keeps both the 8-lane phases of the K fragment reads (8 keys, one chunk) and the 16-lane
// groups of the transposing reads (4 keys, two chunks) on disjoint banks.
//
// Softmax: log2 domain, t = s * log2(e)/scale.  The running maximum m is only raised when
// a block's maximum exceeds it by more than kSlack (= 8, so p <= 256): the rescale of the
// accumulators is then rare, and the result is the same softmax, since every term and the
// row sum share one m.  Rows without a visible key keep m = -inf and l = 0.

#include "kernels.h"
#include "mma.h"

#include <math.h>

#include <algorithm>
#include <type_traits>

namespace mla {

namespace {

constexpr int kFR = 512, kFD = 64;                  // latent and rope widths
constexpr int kFKeys = 32;                          // keys per block
constexpr int kFRows = 64;                          // rows per workgroup
constexpr int kFThreads = 256;
constexpr int kQSteps = (kFR + kFD) / 16;           // 36 MFMA K steps of 16
constexpr int kRSteps = kFR / 16;                   // 32 of them over the latent part
constexpr int kHSteps = kQSteps / 2;                // 18 per wave of a row block
constexpr int kColBlocks = kFR / 64;                // 8 blocks of 32 columns per wave
constexpr int kLatBytes = kFR * 2;                  // one key's latent row
constexpr int kPeBytes = kFD * 2;                   // one key's rope row
constexpr int kPeOff = kFKeys * kLatBytes;          // rope rows follow the latent rows
constexpr int kStageBytes = kPeOff + kFKeys * kPeBytes;
constexpr int kXBytes = 4 * 4 * 64 * 16;            // S^T exchange: [wave][quarter][lane] x 16 B
constexpr int kLoadsPerBlock = 9;                   // per wave: 8 latent rows, 8 rope rows
constexpr float kSlack = 8.f;                       // log2 units
constexpr int kSgValu = 0x002;                      // sched_group_barrier class: VALU

typedef __bf16 v4bf __attribute__((ext_vector_type(4)));
typedef __attribute__((address_space(3))) void lds_t;
typedef __attribute__((address_space(3))) v4bf lds_v4bf;

struct FlashArgs {
    const uint16_t* qa; const uint16_t* qr;     // [B*Sq*H, R], [B*Sq*H, D]
    const uint16_t* ckv; const uint16_t* pe;    // [B, key_stride, R], [B, key_stride, D]
    float* o;          // [n_split][B*Sq*H][R]   unnormalised ctx per split
    float* m;          // [n_split][B*Sq*H]      log2-domain row maximum per split
    float* l;          // [n_split][B*Sq*H]      row sum per split
    int B, Sq, Sk, H, n_split, keys_per_split, row_tiles;
    int64_t key_stride;
    float c;           // log2(e) / scale
    int causal;
};

// Chunk permutations (see the header).  gfx950 serves a 128-bit LDS read 16 lanes per
// cycle (256 bytes, all 64 banks) and a 64-bit read 32 lanes per cycle.  Latent rows (1 KB):
// the 16-byte chunk c of key k sits at c ^ swz(k & 15) within its 256-byte group, so the
// 16 keys of a K fragment read hit 16 distinct chunks, and the 4 keys x 64 bytes of a
// transposing read's half-wave hit 4 distinct 64-byte quarters.  Rope rows (128 B, two per
// 256 bytes): chunk c of key k sits at c ^ ((k >> 1) & 7).
__device__ __forceinline__ int swz(int k) { return ((k & 3) << 2) | ((k >> 2) & 3); }
__device__ __forceinline__ int swz_pe(int k) { return (k >> 1) & 7; }

template <int N>
__device__ __forceinline__ void wait_vm() {
    // vmcnt(N) with lgkmcnt and expcnt left at their maxima (gfx9 encoding)
    __builtin_amdgcn_s_waitcnt((N & 15) | ((N >> 4) << 14) | (0x7 << 4) | (0xF << 8));
}

// Workgroup barrier for LDS data only: this wave's LDS accesses are complete (lgkmcnt(0)),
// then s_barrier.  __syncthreads() would also wait for every outstanding global load
// (vmcnt(0)), i.e. drain the ring of direct-to-LDS prefetches.  The empty asm statements
// keep the compiler from moving memory accesses across the barrier.
__device__ __forceinline__ void lds_barrier() {
    __builtin_amdgcn_sched_barrier(0);
    asm volatile("" ::: "memory");
    __builtin_amdgcn_s_waitcnt(0xC07F);   // lgkmcnt(0), vmcnt/expcnt at their maxima
    __builtin_amdgcn_s_barrier();
    asm volatile("" ::: "memory");
    __builtin_amdgcn_sched_barrier(0);
}

typedef int32_t v4i __attribute__((ext_vector_type(4)));

// Raw buffer descriptor words (base, 32-bit data format, range kRsrcRange), as make_rsrc.
__device__ __forceinline__ v4i rsrc_words(const void* base) {
    const uint64_t p = reinterpret_cast<uint64_t>(base);
    return v4i{(int32_t)(uint32_t)p, (int32_t)((uint32_t)(p >> 32) & 0xffff), kRsrcRange,
               0x00020000};
}

// 16 bytes per lane from buffer offset soff + voff into LDS at lds + 16*lane (gfx950
// buffer_load_dwordx4 ... lds).  Written as asm so that the compiler neither tracks it
// (it would otherwise wait for every such load before any LDS read it cannot prove
// disjoint) nor reorders memory accesses across it; the kernel waits with explicit vmcnt.
// voff >= kRsrcRange (kOob) returns zeros without a memory access.
// (m0 is a reserved register: the compiler keeps no value in it across this statement;
// nothing else in these kernels uses m0.)
#pragma clang diagnostic push
#pragma clang diagnostic ignored "-Winline-asm"
__device__ __forceinline__ void dma16(v4i rsrc, uint32_t lds, uint32_t voff, uint32_t soff) {
    asm volatile("s_mov_b32 m0, %0\n\ts_nop 0\n\tbuffer_load_dwordx4 %1, %2, %3 offen lds"
                 :
                 : "s"(lds), "v"(voff), "s"(rsrc), "s"(soff)
                 : "memory", "m0");
}
#pragma clang diagnostic pop

__device__ __forceinline__ uint32_t lds_addr(const void* p) {
    return (uint32_t)reinterpret_cast<uintptr_t>((const lds_t*)p);
}

// The work of wave (rb, CW) of the workgroup; CW (depth half of S, column half of O) is a
// template parameter, and so is the ring stage of each block step, so that every LDS
// offset is an immediate.
template <int NS, int CW>
__device__ __forceinline__ void flash_wave(const FlashArgs& a, uint8_t* smem, int wg) {
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int l32 = lane & 31, h = lane >> 5, rb = wave & 1;

    const int sp = wg % a.n_split;
    const int rt = (wg / a.n_split) % a.row_tiles;
    const int b = wg / (a.n_split * a.row_tiles);
    const int rows_b = a.Sq * a.H;
    const int r0 = rt * kFRows;
    const int row = r0 + 32 * rb + l32;              // this lane's row within the batch
    const int rows_total = a.B * rows_b;

    // keys of this split; the causal rule (query s sees keys <= Sk - Sq + s) also trims
    // the range to the tile's last query
    const int k_lo = sp * a.keys_per_split;
    int k_hi = min(a.Sk, k_lo + a.keys_per_split);
    int lim = k_hi - 1;                              // last visible key of this lane's row
    if (a.causal) {
        lim = min(lim, a.Sk - a.Sq + min(row, rows_b - 1) / a.H);
        k_hi = min(k_hi, a.Sk - a.Sq + min(r0 + kFRows - 1, rows_b - 1) / a.H + 1);
    }
    const int nb = k_hi > k_lo ? (k_hi - k_lo + kFKeys - 1) / kFKeys : 0;
    // the smallest row limit of the wave: its first row's (rows ascend with the lanes)
    const int lim_wave = __builtin_amdgcn_readfirstlane(lim);

    // ---- Q^T fragments of depth half CW: lane l holds row l%32's depth 16s + 8h .. +7
    const __amdgpu_buffer_rsrc_t rq = make_rsrc(a.qa + (int64_t)b * rows_b * kFR);
    const __amdgpu_buffer_rsrc_t rr = make_rsrc(a.qr + (int64_t)b * rows_b * kFD);
    const uint32_t qmask = oob_mask(row, rows_b);
    v4u qf[kHSteps];
    #pragma unroll
    for (int i = 0; i < kHSteps; ++i) {
        const int s = kHSteps * CW + i;
        qf[i] = s < kRSteps
                    ? load16(rq, ((uint32_t)row * kLatBytes + 32u * s + 16u * h) | qmask)
                    : load16(rr, ((uint32_t)row * kPeBytes + 32u * (s - kRSteps) + 16u * h) | qmask);
    }

    // ---- direct global->LDS staging of key blocks: wave w loads keys 8w .. 8w+7
    const v4i rk = rsrc_words(a.ckv + (int64_t)b * a.key_stride * kFR);
    const v4i rp = rsrc_words(a.pe + (int64_t)b * a.key_stride * kFD);
    const uint32_t lds0 = lds_addr(smem);
    // rope rows of keys 8w .. 8w+7: lane i fills chunk i%8 of key 8w + i/8
    const uint32_t pe_lane = (uint32_t)(lane >> 3) * kPeBytes +
                             16u * ((lane & 7) ^ swz_pe(8 * wave + (lane >> 3)));
    // latent row of key 8w + q: lane i fills LDS chunk i, i.e. loads logical chunk
    // i ^ swz(key & 15) of its 256-byte group (blocks start at multiples of 32 keys)
    uint32_t lat_lane[8];
    #pragma unroll
    for (int q = 0; q < 8; ++q)
        lat_lane[q] = 16u * ((lane & ~15) | ((lane ^ swz((8 * wave + q) & 15)) & 15));

    auto issue = [&](int j, int stage) __attribute__((always_inline)) {
        const int kb = k_lo + kFKeys * j + 8 * wave;     // this wave's first key
        // the LDS base goes to M0: wave-uniform, made scalar explicitly
        const uint32_t st = __builtin_amdgcn_readfirstlane(lds0 + stage * kStageBytes + 8 * wave * kLatBytes);
        const uint32_t st_pe = __builtin_amdgcn_readfirstlane(lds0 + stage * kStageBytes + kPeOff + 8 * wave * kPeBytes);
        const uint32_t kb_s = __builtin_amdgcn_readfirstlane(kb);
        #pragma unroll
        for (int q = 0; q < 8; ++q) {
            const uint32_t voff = (int)kb_s + q < k_hi ? lat_lane[q] : kOob;
            dma16(rk, st + q * kLatBytes, voff, (kb_s + q) * kLatBytes);
        }
        const uint32_t voff = kb + (lane >> 3) < k_hi ? pe_lane : kOob;
        dma16(rp, st_pe, voff, kb_s * kPeBytes);
    };

    // ---- per-lane LDS offsets of the fragments
    // K fragment of step s: key l32, logical chunk 2s + h = 16(s/8) + (2(s%8) + h), the low
    // four bits permuted by swz(l32 & 15); rope step s' reads chunk 2s' + h of the rope row
    const int fk = swz(l32 & 15);
    uint32_t k_off[8];
    #pragma unroll
    for (int q = 0; q < 8; ++q) k_off[q] = l32 * kLatBytes + 16u * ((2 * q + h) ^ fk);
    uint32_t p_off[4];
    #pragma unroll
    for (int q = 0; q < 4; ++q)
        p_off[q] = kPeOff + l32 * kPeBytes + 16u * ((2 * q + h) ^ swz_pe(l32));
    // V^T fragment of 32-col block mb, K step t, half r2: lane (group G = l/16, j = l%16,
    // q = j/4, c = j%4) addresses key 16t + 8r2 + 4h + q, cols 32mb + 16(G%2) + 4c .. +3,
    // i.e. logical chunk 4mb + 2(G%2) + c/2 = 16(mb/4) + (4(mb%4) + 2(G%2) + c/2)
    uint32_t v_off[8];   // [r2][mb % 4]
    {
        const int G = lane >> 4, j = lane & 15, q = j >> 2, c = j & 3;
        #pragma unroll
        for (int r2 = 0; r2 < 2; ++r2) {
            const int kx = 8 * r2 + 4 * h + q, fv = swz(kx);
            #pragma unroll
            for (int m4 = 0; m4 < 4; ++m4) {
                const int chunk = 4 * m4 + 2 * (G & 1) + (c >> 1);   // low 4 bits of col/8
                v_off[4 * r2 + m4] = kx * kLatBytes + 16u * (chunk ^ fv) + 8u * (c & 1);
            }
        }
    }
    v4f* xw = reinterpret_cast<v4f*>(smem + NS * kStageBytes) + wave * 256 + lane;
    const v4f* xr = reinterpret_cast<const v4f*>(smem + NS * kStageBytes) + (wave ^ 2) * 256 + lane;

    v16f O[kColBlocks];
    #pragma unroll
    for (int i = 0; i < kColBlocks; ++i) O[i] = v16f{};
    float m_run = -INFINITY, l_run = 0.f;
    uint32_t pk[8] = {0, 0, 0, 0, 0, 0, 0, 0};   // P^T of the previous block, bf16 pairs

    // V^T fragments of the block in stage ST for K step tk (keys 16tk + {0..3, 8..11} + 4h),
    // and the MFMAs that fold them into O^T with P^T of that block
    auto read_v = [&](auto st_tag, int tk, v8bf* va) __attribute__((always_inline)) {
        constexpr int ST = decltype(st_tag)::value;
        const uint8_t* st = smem + ST * kStageBytes;
        #pragma unroll
        for (int i = 0; i < kColBlocks; ++i) {
            const int mb = kColBlocks * CW + i;
            const uint32_t imm = 256u * (mb >> 2) + 16384u * tk;
            const v4bf lo = __builtin_amdgcn_ds_read_tr16_b64_v4bf16(
                (lds_v4bf*)(st + v_off[mb & 3] + imm));
            const v4bf hi = __builtin_amdgcn_ds_read_tr16_b64_v4bf16(
                (lds_v4bf*)(st + v_off[4 + (mb & 3)] + imm));   // row offset includes 8r2
            va[i] = __builtin_shufflevector(lo, hi, 0, 1, 2, 3, 4, 5, 6, 7);
        }
    };
    auto mma_v = [&](int tk, const v8bf* va) __attribute__((always_inline)) {
        const v4u pb = {pk[4 * tk], pk[4 * tk + 1], pk[4 * tk + 2], pk[4 * tk + 3]};
        #pragma unroll
        for (int i = 0; i < kColBlocks; ++i)
            O[i] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(va[i], __builtin_bit_cast(v8bf, pb),
                                                           O[i], 0, 0, 0);
    };
    auto pv = [&](auto st_tag, int tk) __attribute__((always_inline)) {
        v8bf va[kColBlocks];
        read_v(st_tag, tk, va);
        mma_v(tk, va);
    };

    // One 32-key block j held in ring stage ST.  Block j's scores, exchange and softmax run
    // together with block j-1's P.V (stage ST-1): the first half of that P.V covers the
    // exchange writes before the barrier, the second half interleaves with the softmax.
    auto step = [&](int j, auto st_tag, auto has_prev) __attribute__((always_inline)) {
        constexpr int ST = decltype(st_tag)::value;
        constexpr bool PREV = decltype(has_prev)::value;
        constexpr int SP = (ST + NS - 1) % NS;
        const int ahead = min(nb - 1, j + NS - 3) - j;   // blocks issued after block j
        if constexpr (NS >= 4) {
            if (ahead >= 2) wait_vm<2 * kLoadsPerBlock>();
            else if (ahead == 1) wait_vm<kLoadsPerBlock>();
            else wait_vm<0>();
        } else {
            if (ahead >= 1) wait_vm<kLoadsPerBlock>();
            else wait_vm<0>();
        }
        lds_barrier();   // block j is in LDS for every wave; every wave is past block j-2's P.V
        if (j + NS - 2 < nb) issue(j + NS - 2, (ST + NS - 2) % NS);

        const uint8_t* st = smem + ST * kStageBytes;

        // partial S^T over this wave's 18 depth steps; K fragment reads run kWin steps ahead
        constexpr int kWin = 6;
        auto read_k = [&](int i) __attribute__((always_inline)) {
            const int s = kHSteps * CW + i;
            const uint32_t off = s < kRSteps ? k_off[s & 7] + 256u * (s >> 3)
                                             : p_off[(s - kRSteps) & 3];
            return *reinterpret_cast<const v4u*>(st + off);
        };
        v4u kf[kWin];
        #pragma unroll
        for (int i = 0; i < kWin; ++i) kf[i] = read_k(i);
        v8bf va0[kColBlocks];
        if constexpr (PREV) read_v(std::integral_constant<int, SP>{}, 0, va0);
        v16f sa = v16f{};
        #pragma unroll
        for (int i = 0; i < kHSteps; ++i) {
            const v4u cur = kf[i % kWin];
            if (i + kWin < kHSteps) kf[i % kWin] = read_k(i + kWin);
            sa = Mma<bf16_t>::sub(cur, qf[i], 0, sa);
        }
        #pragma unroll
        for (int q = 0; q < 4; ++q)
            xw[64 * q] = v4f{sa[4 * q], sa[4 * q + 1], sa[4 * q + 2], sa[4 * q + 3]};
        if constexpr (PREV) mma_v(0, va0);
        // issue order of this region: the first K window, the V^T reads of block j-1, the
        // score MFMAs with the remaining K reads between them, the exchange writes, then
        // block j-1's first P.V half
        __builtin_amdgcn_sched_group_barrier(kSgDsRd, kWin, 0);
        if constexpr (PREV) __builtin_amdgcn_sched_group_barrier(kSgDsRd, 2 * kColBlocks, 0);
        #pragma unroll
        for (int i = 0; i < kHSteps - kWin; ++i) {
            __builtin_amdgcn_sched_group_barrier(kSgMfma, 1, 0);
            __builtin_amdgcn_sched_group_barrier(kSgDsRd, 1, 0);
        }
        __builtin_amdgcn_sched_group_barrier(kSgMfma, kWin, 0);
        __builtin_amdgcn_sched_group_barrier(kSgDsWr, 4, 0);
        if constexpr (PREV) __builtin_amdgcn_sched_group_barrier(kSgMfma, kColBlocks, 0);
        lds_barrier();   // both halves of every row block's S^T are in LDS
        v8bf va1[kColBlocks];
        if constexpr (PREV) read_v(std::integral_constant<int, SP>{}, 1, va1);
        v16f sc;
        #pragma unroll
        for (int q = 0; q < 4; ++q) {
            const v4f o = xr[64 * q];
            #pragma unroll
            for (int e = 0; e < 4; ++e)   // the same operand order in both waves
                sc[4 * q + e] = CW == 0 ? sa[4 * q + e] + o[e] : o[e] + sa[4 * q + e];
        }
        if constexpr (PREV) mma_v(1, va1);

        // online softmax of block j; element i of lane l is key kb + 8(i/4) + 4h + i%4 of
        // row l%32
        // Work on the raw scores: c > 0, so max(s) * c is exactly max(s * c), and
        // p = 2^(s c - m) is one fma and one v_exp_f32.  Masked keys get s = -inf.  Blocks
        // whose every key is visible to every row of the wave skip the mask.
        const int kb = k_lo + kFKeys * j;
        if (kb + kFKeys - 1 > lim_wave) {
            #pragma unroll
            for (int i = 0; i < 16; ++i) {
                const int key = kb + 8 * (i >> 2) + 4 * h + (i & 3);
                sc[i] = key <= lim ? sc[i] : -INFINITY;
            }
        }
        float bm = fmaxf(fmaxf(sc[0], sc[1]), sc[2]);
        #pragma unroll
        for (int i = 3; i < 16; i += 2) bm = fmaxf(fmaxf(bm, sc[i]), sc[i + 1] );
        {
            const auto sw = __builtin_amdgcn_permlane32_swap(__float_as_uint(bm),
                                                             __float_as_uint(bm), false, false);
            bm = fmaxf(__uint_as_float(sw[0]), __uint_as_float(sw[1])) * a.c;
        }
        const bool raise = bm > m_run + kSlack;
        // 2^(m_run - bm) is 0 on a row's first raise (m_run = -inf); other rows keep 1
        const float f = raise ? __builtin_amdgcn_exp2f(m_run - bm) : 1.f;
        m_run = raise ? bm : m_run;
        // a row with no visible key so far has m_run = -inf and every s = -inf: p = 0
        const float m_neg = m_run == -INFINITY ? 0.f : -m_run;
        float ls = 0.f;
        #pragma unroll
        for (int i = 0; i < 16; i += 2) {
            const float p0 = __builtin_amdgcn_exp2f(__builtin_fmaf(sc[i], a.c, m_neg));
            const float p1 = __builtin_amdgcn_exp2f(__builtin_fmaf(sc[i + 1], a.c, m_neg));
            ls += p0 + p1;
            pk[i >> 1] = pack_bf16x2(p0, p1);
        }
        l_run = l_run * f + ls;
        // the probabilities are computed here, between block j-1's MFMAs, not sunk past the
        // rescale branch below
        asm volatile("" ::"v"(pk[0]), "v"(pk[1]), "v"(pk[2]), "v"(pk[3]), "v"(pk[4]), "v"(pk[5]),
                     "v"(pk[6]), "v"(pk[7]), "v"(l_run));
        // issue order of this region: the exchange and V^T reads, then block j-1's second
        // P.V half with the softmax VALU work spread between its MFMAs
        __builtin_amdgcn_sched_group_barrier(kSgDsRd, PREV ? 4 + 2 * kColBlocks : 4, 0);
        if constexpr (PREV) {
            #pragma unroll
            for (int i = 0; i < kColBlocks; ++i) {
                __builtin_amdgcn_sched_group_barrier(kSgMfma, 1, 0);
                __builtin_amdgcn_sched_group_barrier(kSgValu, 10, 0);
            }
        }
        // rescale after block j-1's P.V (which is in the old scale) has been accumulated
        if (__builtin_amdgcn_ballot_w64(raise)) {
            #pragma unroll
            for (int mb = 0; mb < kColBlocks; ++mb) O[mb] *= f;
        }
    };

    // ---- prologue: blocks 0 .. NS-3 in flight; block 0 without a predecessor; then the
    // blocks, NS per trip so that every step's ring stage is a constant; then the last
    // block's P.V
    #pragma unroll
    for (int j = 0; j < NS - 2; ++j)
        if (j < nb) issue(j, j);
    if (nb > 0) step(0, std::integral_constant<int, 0>{}, std::false_type{});
    for (int j0 = 1; j0 < nb; j0 += NS) {
        step(j0, std::integral_constant<int, 1 % NS>{}, std::true_type{});
        if (j0 + 1 < nb) step(j0 + 1, std::integral_constant<int, 2 % NS>{}, std::true_type{});
        if constexpr (NS > 2)
            if (j0 + 2 < nb) step(j0 + 2, std::integral_constant<int, 3 % NS>{}, std::true_type{});
        if constexpr (NS > 3)
            if (j0 + 3 < nb) step(j0 + 3, std::integral_constant<int, 4 % NS>{}, std::true_type{});
    }
    if (nb > 0) {
        // block nb-1 sits in stage (nb-1) % NS; no later loads overwrite it
        switch ((nb - 1) % NS) {
            case 0: pv(std::integral_constant<int, 0>{}, 0); pv(std::integral_constant<int, 0>{}, 1); break;
            case 1: pv(std::integral_constant<int, 1 % NS>{}, 0); pv(std::integral_constant<int, 1 % NS>{}, 1); break;
            case 2: pv(std::integral_constant<int, 2 % NS>{}, 0); pv(std::integral_constant<int, 2 % NS>{}, 1); break;
            default: pv(std::integral_constant<int, 3 % NS>{}, 0); pv(std::integral_constant<int, 3 % NS>{}, 1); break;
        }
    }

    // ---- this split's partial state: O columns 256CW .., and (CW = 0) m and l
    {
        const auto sw = __builtin_amdgcn_permlane32_swap(__float_as_uint(l_run),
                                                         __float_as_uint(l_run), false, false);
        l_run = __uint_as_float(sw[0]) + __uint_as_float(sw[1]);
    }
    if (row < rows_b) {
        const int64_t slot = (int64_t)sp * rows_total + (int64_t)b * rows_b + row;
        if (CW == 0 && h == 0) {
            a.m[slot] = m_run;
            a.l[slot] = l_run;
        }
        float* orow = a.o + slot * kFR + 256 * CW;
        #pragma unroll
        for (int i = 0; i < kColBlocks; ++i) {
            #pragma unroll
            for (int g = 0; g < 4; ++g) {
                const v4f v = {O[i][4 * g], O[i][4 * g + 1], O[i][4 * g + 2], O[i][4 * g + 3]};
                *reinterpret_cast<v4f*>(orow + 32 * i + 8 * g + 4 * h) = v;
            }
        }
    }
}

template <int NS>
__global__ void __launch_bounds__(kFThreads, 1) flash_kernel(FlashArgs a) {
    __shared__ __attribute__((aligned(1024))) uint8_t smem[NS * kStageBytes + kXBytes];
    // the two row tiles of a batch are consecutive logical workgroups on one XCD
    const int wg = xcd_logical_block(blockIdx.x, gridDim.x);
    if ((threadIdx.x >> 6) < 2) flash_wave<NS, 0>(a, smem, wg);
    else flash_wave<NS, 1>(a, smem, wg);
}

constexpr int kFStages = 4;   // LDS ring depth

// ctx = sum_s w_s O_s, row_sum = sum_s w_s l_s, w_s = 2^(m_s - max_s m_s); one thread per
// (row, 4 columns)
__global__ void __launch_bounds__(256) flash_merge_kernel(const float* __restrict__ o,
                                                          const float* __restrict__ m,
                                                          const float* __restrict__ l,
                                                          float* __restrict__ ctx,
                                                          float* __restrict__ row_sum, int rows,
                                                          int n_split) {
    const int per_row = kFR / 4;
    const int64_t idx = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (idx >= (int64_t)rows * per_row) return;
    const int r = (int)(idx / per_row), c4 = (int)(idx % per_row);
    float mx = -INFINITY;
    for (int s = 0; s < n_split; ++s) mx = fmaxf(mx, m[(int64_t)s * rows + r]);
    v4f acc = {0.f, 0.f, 0.f, 0.f};
    float ls = 0.f;
    for (int s = 0; s < n_split; ++s) {
        const float ms = m[(int64_t)s * rows + r];
        const float w = ms == -INFINITY ? 0.f : __builtin_amdgcn_exp2f(ms - mx);
        const v4f v = *reinterpret_cast<const v4f*>(o + ((int64_t)s * rows + r) * kFR + 4 * c4);
        acc += w * v;
        ls += w * l[(int64_t)s * rows + r];
    }
    *reinterpret_cast<v4f*>(ctx + (int64_t)r * kFR + 4 * c4) = acc;
    if (c4 == 0) row_sum[r] = ls;
}

}  // namespace

bool flash_supported(const FlashProblem& p) {
    return p.R == kFR && p.D == kFD && p.B > 0 && p.Sq > 0 && p.H > 0 && p.Sk > 0;
}

FlashPlan plan_flash(const FlashProblem& p) {
    FlashPlan f;
    f.row_tiles = (p.Sq * p.H + kFRows - 1) / kFRows;
    const int base = p.B * f.row_tiles;
    const int blocks = (p.Sk + kFKeys - 1) / kFKeys;
    // about one workgroup per CU (the LDS ring admits one per CU), at least 4 key blocks
    // per split
    int split = std::max(1, (kNumCUs + base / 2) / base);
    split = std::min(split, std::max(1, blocks / 4));
    const int per = (blocks + split - 1) / split;
    f.keys_per_split = per * kFKeys;
    f.n_split = (blocks + per - 1) / per;
    const size_t rows = (size_t)p.B * p.Sq * p.H;
    // split partials (O, m, l); with one split O and l go straight to ctx / row_sum and
    // only the row maxima need a scratch row
    f.partial_bytes = f.n_split > 1 ? rows * f.n_split * (kFR + 2) * sizeof(float)
                                    : rows * sizeof(float);
    return f;
}

hipError_t launch_flash(const FlashProblem& p, const FlashPlan& f, float* ctx, float* row_sum,
                        float* partials, hipStream_t stream) {
    const int rows = p.B * p.Sq * p.H;
    FlashArgs a;
    a.qa = static_cast<const uint16_t*>(p.qa);
    a.qr = static_cast<const uint16_t*>(p.qr);
    a.ckv = static_cast<const uint16_t*>(p.ckv);
    a.pe = static_cast<const uint16_t*>(p.pe);
    float* m_split;
    if (f.n_split > 1) {
        a.o = partials;
        a.m = partials + (size_t)f.n_split * rows * kFR;
        a.l = a.m + (size_t)f.n_split * rows;
        m_split = a.m;
    } else {
        a.o = ctx;
        a.l = row_sum;
        a.m = partials;   // the row maxima are not needed: a small scratch row
        m_split = nullptr;
    }
    a.B = p.B; a.Sq = p.Sq; a.Sk = p.Sk; a.H = p.H;
    a.n_split = f.n_split; a.keys_per_split = f.keys_per_split; a.row_tiles = f.row_tiles;
    a.key_stride = p.key_stride > 0 ? p.key_stride : p.Sk;
    a.c = 1.4426950408889634f / p.scale;
    a.causal = p.causal ? 1 : 0;
    const int grid = p.B * f.row_tiles * f.n_split;
    hipLaunchKernelGGL(flash_kernel<kFStages>, dim3(grid), dim3(kFThreads), 0, stream, a);
    hipError_t e = hipGetLastError();
    if (e != hipSuccess || f.n_split == 1) return e;
    const int64_t n = (int64_t)rows * (kFR / 4);
    hipLaunchKernelGGL(flash_merge_kernel, dim3((unsigned)((n + 255) / 256)), dim3(256), 0,
                       stream, a.o, m_split, a.l, ctx, row_sum, rows, f.n_split);
    return hipGetLastError();
}

}  // namespace mla
