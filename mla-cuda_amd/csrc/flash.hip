// 3a + 3b + 3c fused: one pass over the latent cache per key split, for 16-bit storage
// (flash16_kernel) and fp32 storage (flash32_kernel, further below).
//
// The per-step path materialises fp32 scores (3a), reduces per-tile softmax partials
// (3b) and streams c_kv a second time for ctx (3c).  With bf16 storage that path is
// HBM-bound on traffic it creates itself: at B=128, Sk=4989 it moves ~2.0 GB, of which
// only 0.74 GB is the cache; in fp32 it is MFMA-bound and the extra passes cost the
// score epilogue, the combine and a second launch tail.  These kernels read every key row
// once, keep the softmax state in registers and write only the unnormalised ctx, its row
// sums and (for a split) row maxima.
// The arithmetic is the reference's (mla_kernels.cu:971-1032, 1058-1079, 1247-1254):
// s = q_absorbed.c_kv + q_rope.pe, softmax over s/scale, ctx = sum_k p_k c_kv[k]; only the
// order of operations differs (a streaming softmax instead of per-tile partials).
//
// Workgroup: 4 waves over 64 rows (queries x heads) of one batch and one contiguous key
// range (a split).  Key blocks reach LDS through direct global->LDS loads
// (buffer_load_dwordx4 ... lds) into a ring of four blocks -- two in flight while two are
// in use -- with no VGPRs spent on staging; one barrier per block guards the ring.  The
// two 64-row tiles of a batch are placed on one XCD, so the second read of every key
// block hits its L2.  V^T fragments come from the same key-major LDS tile as K, through
// gfx950's transposing ds_read_b64_tr_b16, so c_kv is staged once per workgroup.
//
// Softmax (log2 domain, t = s * log2(e)/scale): each row keeps a fixed reference, the
// maximum of its first visible block.  Every term is 2^(t - reference) and the output
// accumulators are never rescaled; a row whose maximum passes the reference by a wide
// margin (2^64 in bf16, 2^40 in fp32: far from any overflow) raises it, and the pass
// over the split is repeated from its first key with the raised references.  The result is
// the same softmax, since every term and the row sum share one reference.  Rows without a
// visible key keep the reference -inf and the row sum 0.

#include "kernels.h"
#include "mma.h"
#include "stage.h"
#include "worklist.h"

#include <math.h>

#include <algorithm>
#include <cstdlib>
#include <cstring>
#include <type_traits>
#include <utility>

namespace mla {

namespace {

typedef uint32_t v2u __attribute__((ext_vector_type(2)));

constexpr int kFR = 512, kFD = 64;                  // latent and rope widths
constexpr int kFKeys = 32;                          // keys per block
constexpr int kFRows = 64;                          // rows per workgroup
constexpr int kFThreads = 256;
constexpr int kQSteps = (kFR + kFD) / 32;           // 18 MFMA K steps of 32
constexpr int kRSteps = kFR / 32;                   // 16 of them over the latent part
constexpr int kLatBytes = kFR * 2;                  // one key's latent row
constexpr int kPeBytes = kFD * 2;                   // one key's rope row

struct FlashArgs {
    const uint16_t* qa; const uint16_t* qr;     // [B*Sq*H, R], [B*Sq*H, D]
    const uint16_t* ckv; const uint16_t* pe;    // [B, key_stride, R], [B, key_stride, D]
    float* o;          // [n_split][B*Sq*H][R]   unnormalised ctx per split
    float* m;          // [n_split][B*Sq*H]      log2-domain row maximum per split
    float* l;          // [n_split][B*Sq*H]      row sum per split
    int B, Sq, Sk, H, n_split, keys_per_split, row_tiles;
    int64_t key_stride;
    float c;           // log2(e) / scale (times kv_scale for an fp8 cache)
    float o_scale;     // factor of the ctx rows written (kv_scale for an fp8 cache, else 1)
    int causal;
    // ragged / paged keys (both optional): batch b has min(seq_lens[b], Sk) keys, and its
    // key rows [j*page_size, (j+1)*page_size) are rows of page block_table[b*max_pages + j]
    // of ckv / pe (page_size a multiple of 64, so no key block straddles a page)
    const int* seq_lens;
    const int* block_table;
    int page_size, max_pages;
    // balanced work list of a ragged batch (optional; flash_worklist_kernel): workgroup
    // (item, row tile) runs chunk c of batch b for item = {b, c}; a batch of one chunk
    // writes o_direct / l_direct (ctx, row_sum), the others partial slot first[b] + c
    const int* wl;
    float* o_direct;
    float* l_direct;
    // dense unsplit 16-bit pass only (flash_ctx16_ok): instead of o / l, write each row
    // already normalised and rounded to the storage format, (o_scale O) (1 / l) -- what
    // 3d's A staging forms from ctx and row_sum -- at ctx16[row][R]
    void* ctx16;
};

// What one workgroup of the attention pass computes: batch b, row tile rt, keys
// [k_lo, k_lo + k_len) (clipped to the batch), and where its state goes: partial slot
// `slot` (rows slot * rows_b ..), or ctx / row_sum directly.
struct FlashWork {
    int b, rt, k_lo, k_len;
    int64_t slot;
    bool direct, skip;
};
// Uniform splits: the logical workgroup order is XCD-major (the two row tiles of a batch
// are neighbours on one XCD, so the second read of a key block hits its L2).  Work list:
// workgroup i runs on XCD i % 8 in the dispatcher's order, and item t's row tiles are
// workgroups 8 (row_tiles (t / 8) + rt) + t % 8 -- one XCD per item, the items (longest
// first) spread over the XCDs in list order, and the unused tail of the grid spread too.
__device__ __forceinline__ FlashWork flash_work(const FlashArgs& a) {
    FlashWork w;
    w.direct = false;
    w.skip = false;
    if (!a.wl) {
        const int wg = xcd_logical_block(blockIdx.x, gridDim.x);
        const int sp = wg % a.n_split;
        w.rt = (wg / a.n_split) % a.row_tiles;
        w.b = wg / (a.n_split * a.row_tiles);
        w.k_lo = sp * a.keys_per_split;
        w.k_len = a.keys_per_split;
        w.slot = (int64_t)sp * a.B + w.b;
        return w;
    }
    const int x = blockIdx.x % kNumXCDs, q = blockIdx.x / kNumXCDs;
    const int it = (q / a.row_tiles) * kNumXCDs + x;
    w.rt = q % a.row_tiles;
    w.b = 0; w.k_lo = 0; w.k_len = 0; w.slot = 0;
    if (it >= load_uniform(a.wl)) {
        w.skip = true;
        return w;
    }
    const int* items = a.wl + kWlHead + 2 * a.B;
    w.b = load_uniform(items + 2 * it);
    const int c = load_uniform(items + 2 * it + 1);
    w.k_len = load_uniform(a.wl + 1);
    w.k_lo = c * w.k_len;
    w.direct = load_uniform(a.wl + kWlHead + a.B + w.b) == 1;
    w.slot = (int64_t)load_uniform(a.wl + kWlHead + w.b) + c;
    return w;
}

// Keys of batch b, and the cache row of key k (a wave-uniform key inside the sequence; a
// key past it maps to row 0, which only out-of-range loads then address).
__device__ __forceinline__ int flash_batch_keys(const FlashArgs& a, int b) {
    return a.seq_lens ? min(load_uniform(a.seq_lens + b), a.Sk) : a.Sk;
}
__device__ __forceinline__ int64_t flash_key_row(const FlashArgs& a, int b, int k, int k_end) {
    if (!a.block_table) return (int64_t)b * a.key_stride + k;
    if (k >= k_end) return 0;
    const int page = load_uniform(a.block_table + (int64_t)b * a.max_pages + k / a.page_size);
    return (int64_t)page * a.page_size + k % a.page_size;
}

// Chunk permutation of the fp32 pass's LDS rows: 16-byte chunk c of key k sits at
// c ^ swz(k & 15) within its 256-byte group, swz = rotate left by one bit of four.
__device__ __forceinline__ int swz(int k) { return ((k << 1) | (k >> 3)) & 15; }

// Max / sum over the 4 lanes l%16 + 16g (g = 0..3) that hold one row: v_permlane16_swap
// pairs the rows of 16 lanes (0,1) and (2,3), v_permlane32_swap the two halves; given the
// same value twice each returns the pair's two values in every lane, combined in one order.
template <class Op>
__device__ __forceinline__ float row4_reduce(float v, Op op) {
    const auto a = __builtin_amdgcn_permlane16_swap(__float_as_uint(v), __float_as_uint(v),
                                                    false, false);
    v = op(__uint_as_float(a[0]), __uint_as_float(a[1]));
    const auto b = __builtin_amdgcn_permlane32_swap(__float_as_uint(v), __float_as_uint(v),
                                                    false, false);
    return op(__uint_as_float(b[0]), __uint_as_float(b[1]));
}

// ------------------------------------------------------------------ 16-bit: key-split waves
// The 16-bit pass on 32-row waves that split the keys.  A workgroup's 64 rows are two
// 32-row tiles; wave w = 2 rt + kh owns row tile rt and keys 16kh .. 16kh+15 of every
// 32-key block, at the full 576 depths, so the waves never exchange scores and none
// repeats another's softmax (32 rows per wave is the most the register file holds: the
// output accumulators take all 256 AGPRs, Q^T 144 VGPRs):
//   S^T[16 keys x 32 rows]: two 16x16x32 MFMAs per K fragment (one per 16-row half of the
//     tile), 18 K steps; the wave's Q^T (both halves, 576 deep) lives in 144 VGPRs.  K step
//     s < 16 is latent depth chunk 16g + s for lane group g = l/16 (the groups read four
//     256-byte quarters of a key row), step 16 + r rope chunk 4r + g.  Accumulator element
//     i of lane l is key 4g + i of row (16 half) + l%16.
//   softmax per lane: 8 scores, against a fixed per-row reference (first visible block's
//     maximum; a row that passes it by the headroom (2^64 for bf16, 2^15 for fp16, which
//     P^T is rounded to) raises it and the pass is repeated, as in
//     flash32_kernel), so the 256 O accumulators are never rescaled
//   O^T[512 cols x 32 rows] += V^T[512 x 16 keys] . P^T[16 keys x 32 rows]: sixteen
//     32x32x16 MFMAs.  P^T is the score accumulator rounded to 16 bits after one
//     v_permlane16_swap per register pair, which moves lane l's 4 keys of one row half next
//     to lane l^16's 4 keys of the same row: lane l then holds keys 8(l/32) .. +7 of row l%32,
//     the MFMA's B layout.  V^T comes from two transposing 64-bit reads per MFMA.
// The two key halves of a row tile merge once, through LDS, after the last block (the
// standard rescale by 2^(m_half - max)).  Per wave and 32-key block: 36 + 16 MFMAs (1088
// MFMA cycles), 18 KB of K reads and 16 KB of V reads.
// Measured on one wave per SIMD: a 16x16x32 MFMA issues every 16-17 cycles and a 32x32x16
// every 32, dependent or not; a simple VALU instruction takes ~5 cycles and v_exp_f32 ~14,
// and VALU work issued between MFMAs runs under them.  So the step keeps the MFMA stream
// fed around the barrier (the previous block's P.V goes first), keeps the softmax's rare
// cases behind uniform branches and interleaves its common VALU work with P.V MFMAs, and
// spreads the block's nine cache loads over the step.
// LDS: the latent rows of the NS stages (32 x 1 KB each), then their rope rows; chunk c of
// latent key k sits at (c & ~15) | ((c & 15) ^ sw16(k & 15)), chunk c of rope key k at
// c ^ ((k >> 1) & 7).  gfx950 serves a 128-bit LDS read in 16-lane cycles made of the lane
// octets (56-63, 0-7), (8-15, 16-23), (24-31, 32-39), (40-47, 48-55), and a 64-bit read
// (also the transposing one) in 32-lane halves; a cycle is conflict-free when its lanes
// touch distinct 16-byte (8-byte) slots of 256 bytes.  Under that rule (measured with a
// probe and the SQ_LDS_BANK_CONFLICT counter) every K, V and staging access is conflict-free,
// and each is one per-lane base XOR a constant plus an immediate offset.
constexpr int k2Keys = 32;
constexpr int k2LatStage = k2Keys * kLatBytes;            // 32 KB
constexpr int k2PeStage = k2Keys * kPeBytes;              // 4 KB
constexpr int k2Loads = 9;                                // cache loads per wave and block
constexpr int k8Loads = 5;                                // (fp8 cache: 4 latent, 1 rope)
constexpr float k2Headroom = 64.f;                        // log2 units above a row's reference
constexpr int k2MaxPasses = 8;

__device__ __forceinline__ int sw16(int k) { return ((k & 3) << 2) | ((k >> 2) & 3); }

// 32x32x16 MFMA in the storage format TL (bf16_t or f16_t)
template <typename TL>
__device__ __forceinline__ v16f mfma32h(v4u a, v4u b, v16f c) {
    if constexpr (Half<TL>::kF16)
        return __builtin_amdgcn_mfma_f32_32x32x16_f16(__builtin_bit_cast(v8h, a),
                                                      __builtin_bit_cast(v8h, b), c, 0, 0, 0);
    else
        return __builtin_amdgcn_mfma_f32_32x32x16_bf16(__builtin_bit_cast(v8bf, a),
                                                       __builtin_bit_cast(v8bf, b), c, 0, 0, 0);
}

// The score MFMAs of flash16_kernel (16x16x32 bf16: lane l supplies A[l%16][8(l/16) .. +7]
// and B[8(l/16) .. +7][l%16]; accumulator element i of lane l is D[4(l/16) + i][l%16]),
// written as inline asm so that their accumulators stay in
// VGPRs (the 256 AGPRs hold the output accumulators; left to itself, the register allocator
// puts these in AGPRs and moves output blocks back and forth every block).  The hazards the
// compiler would otherwise resolve for them: two independent chains alternate, so an MFMA
// never reads the accumulator the previous one wrote; the K fragments come from LDS reads
// the compiler waits for; and after the last MFMA of a block 16 wait states pass before any
// VALU reads an accumulator (the 16x16x32 bf16 MFMA needs at most 11).
// (TL picks the bf16 or the fp16 form; both have the same layout and timing.)
template <typename TL>
__device__ __forceinline__ void mfma16_v_first(v4u a, v4u b, v4f& c) {
    if constexpr (Half<TL>::kF16)
        asm("v_mfma_f32_16x16x32_f16 %0, %1, %2, 0" : "=&v"(c) : "v"(a), "v"(b));
    else
        asm("v_mfma_f32_16x16x32_bf16 %0, %1, %2, 0" : "=&v"(c) : "v"(a), "v"(b));
}
template <typename TL>
__device__ __forceinline__ void mfma16_v(v4u a, v4u b, v4f& c) {
    if constexpr (Half<TL>::kF16)
        asm("v_mfma_f32_16x16x32_f16 %0, %1, %2, %0" : "+v"(c) : "v"(a), "v"(b));
    else
        asm("v_mfma_f32_16x16x32_bf16 %0, %1, %2, %0" : "+v"(c) : "v"(a), "v"(b));
}
template <typename TL>
__device__ __forceinline__ void mfma16_v_last(v4u a, v4u b, v4f& c) {
    if constexpr (Half<TL>::kF16)
        asm("v_mfma_f32_16x16x32_f16 %0, %1, %2, %0\n\ts_nop 7\n\ts_nop 7" : "+v"(c) : "v"(a), "v"(b));
    else
        asm("v_mfma_f32_16x16x32_bf16 %0, %1, %2, %0\n\ts_nop 7\n\ts_nop 7" : "+v"(c) : "v"(a), "v"(b));
}

// fp8 cache staging, shared by both 16-bit kernels.  The loader of keys 8w .. 8w+7 of a
// block puts their raw rows, R and D bytes each, unpermuted into its 5 KB region of fp8
// stage j & 1 (4 KB latent, 512 B rope, 512 B that the rope load's idle lanes fill with
// zeros), and converts them into the bf16 ring in the layout the direct loads write.  Part
// q < 4 is one 16-byte read per lane: lane l holds bytes 16 (l % 32) .. +15 of key 2q + l/32,
// i.e. bf16 chunks c0 = 2 (l % 32) and c0 + 1 of that key; part 4 is the rope rows (lanes
// < 32: key l/4, chunks 2 (l % 4), +1).  OCP e4m3 -> bf16 is exact
// (v_cvt_scalef32_pk_bf16_fp8 with scale 1); the cache scale is applied to the scores and
// the output instead.  Since c0 is even, chunk c0 + 1 sits at chunk c0's position XOR 16.
constexpr int kF8Wave = 5120, kF8Stage = 4 * kF8Wave;
struct F8Stage {
    uint32_t lat[4], pe;   // bf16 ring offsets (stage 0) of this lane's chunks
    __device__ F8Stage(int w, int lane, uint32_t pe_base) {
        #pragma unroll
        for (int q = 0; q < 4; ++q) {
            const int kw = 8 * w + 2 * q + (lane >> 5);
            lat[q] = kw * kLatBytes + 256u * ((lane & 31) >> 3) + 16u * ((2 * (lane & 7)) ^ sw16(kw & 15));
        }
        const int kwp = 8 * w + ((lane >> 2) & 7);
        pe = pe_base + kwp * kPeBytes + 16u * ((2 * (lane & 3)) ^ ((kwp >> 1) & 7));
    }
    // part q of the raw rows in the loader's region at byte offset `region`
    __device__ v4u read(const uint8_t* smem, uint32_t region, int q, int lane) const {
        return *reinterpret_cast<const v4u*>(smem + region + (q < 4 ? 1024 * q : 8 * kFR) + 16u * lane);
    }
    // part q, converted, into bf16 ring stage st
    __device__ void write(uint8_t* smem, int st, int q, v4u raw, int lane) const {
        // bytes 0-1 (word_sel false) and 2-3 (true) of a dword to two bf16
        auto lo2 = [](uint32_t w) __attribute__((always_inline)) {
            return __builtin_bit_cast(uint32_t, __builtin_amdgcn_cvt_scalef32_pk_bf16_fp8(w, 1.f, false));
        };
        auto hi2 = [](uint32_t w) __attribute__((always_inline)) {
            return __builtin_bit_cast(uint32_t, __builtin_amdgcn_cvt_scalef32_pk_bf16_fp8(w, 1.f, true));
        };
        const v4u c0 = {lo2(raw[0]), hi2(raw[0]), lo2(raw[1]), hi2(raw[1])};
        const v4u c1 = {lo2(raw[2]), hi2(raw[2]), lo2(raw[3]), hi2(raw[3])};
        if (q < 4) {
            const uint32_t o = lat[q] + (uint32_t)st * k2LatStage;
            *reinterpret_cast<v4u*>(smem + o) = c0;
            *reinterpret_cast<v4u*>(smem + (o ^ 16u)) = c1;
        } else if (lane < 32) {
            const uint32_t o = pe + (uint32_t)st * k2PeStage;
            *reinterpret_cast<v4u*>(smem + o) = c0;
            *reinterpret_cast<v4u*>(smem + (o ^ 16u)) = c1;
        }
    }
};

template <int NS, typename TL, bool FP8>
__global__ void __launch_bounds__(kFThreads, 1) flash16_kernel(FlashArgs a) {
    // P^T is rounded to TL: with bf16's 8 exponent bits a term may reach 2^64 over its
    // row's reference; fp16 stops at 65504, so there a term stays below 2^15
    constexpr float kHeadroom = Half<TL>::kF16 ? 15.f : k2Headroom;
    static_assert(NS == (FP8 ? 3 : 4), "stage offsets: stage 2 (3) is stage 0 (1) XOR 64 KB");
    static_assert(!FP8 || !Half<TL>::kF16, "an fp8 cache is read with bf16 queries");
    constexpr int kPeBase = NS * k2LatStage;                    // 128 KB (fp8: 96 KB)
    // fp8 cache: two stages of raw cache bytes, 5 KB per wave (F8Stage)
    constexpr int kF8Base = kPeBase + NS * k2PeStage;
    constexpr int kLoads = FP8 ? k8Loads : k2Loads;             // cache loads per wave and block
    __shared__ __attribute__((aligned(1024))) uint8_t smem[kF8Base + (FP8 ? 2 * kF8Stage : 0)];
    const int tid = threadIdx.x, lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);   // a scalar from here on
    const int rt = wave >> 1, kh = wave & 1;
    const int l16 = lane & 15, g = lane >> 4, l32 = lane & 31, hw = lane >> 5;
    const FlashWork work = flash_work(a);
    if (work.skip) return;   // past the end of a work list: the whole workgroup leaves

    const int b = work.b;
    const int rows_b = a.Sq * a.H;
    const int r0 = work.rt * kFRows;
    const int rbase = r0 + 32 * rt;                  // first row of this wave's tile
    const int rowS0 = rbase + l16, rowS1 = rbase + 16 + l16;   // score-layout rows
    const int rowO = rbase + l32;                    // output-layout row

    const int skb = flash_batch_keys(a, b);
    const int k_lo = work.k_lo;
    int k_hi = min(skb, k_lo + work.k_len);
    int lim0 = k_hi - 1, lim1 = k_hi - 1;            // last visible key of each score row
    if (a.causal) {
        lim0 = min(lim0, skb - a.Sq + min(rowS0, rows_b - 1) / a.H);
        lim1 = min(lim1, skb - a.Sq + min(rowS1, rows_b - 1) / a.H);
        k_hi = min(k_hi, skb - a.Sq + min(r0 + kFRows - 1, rows_b - 1) / a.H + 1);
    }
    const int nb = k_hi > k_lo ? (k_hi - k_lo + k2Keys - 1) / k2Keys : 0;
    // the wave's smallest row limit: its first row's (lane 0, first half)
    const int lim_wave = __builtin_amdgcn_readfirstlane(lim0);

    // ---- Q^T of both row halves: latent step s is depth chunk 16g + s, rope step 16 + r
    // rope chunk 4r + g
    const __amdgpu_buffer_rsrc_t rq = make_rsrc(a.qa + (int64_t)b * rows_b * kFR);
    const __amdgpu_buffer_rsrc_t rr = make_rsrc(a.qr + (int64_t)b * rows_b * kFD);
    v4u qf[2][kQSteps];
    #pragma unroll
    for (int t = 0; t < 2; ++t) {
        const int row = t ? rowS1 : rowS0;
        const uint32_t qmask = oob_mask(row, rows_b);
        #pragma unroll
        for (int s = 0; s < kQSteps; ++s)
            qf[t][s] = s < kRSteps
                           ? load16(rq, ((uint32_t)row * kLatBytes + 256u * g + 16u * s) | qmask)
                           : load16(rr, ((uint32_t)row * kPeBytes + 64u * (s - kRSteps) + 16u * g) | qmask);
    }
    // Q is in registers before the first key block is requested: the cache loads are not
    // seen by the compiler's wait-count tracking, which would otherwise keep waiting on Q
    // (and so on every cache load issued since) inside the key loop
    wait_vm<0>();

    // ---- direct global->LDS staging: wave w loads keys 8w .. 8w+7 of a block; lane i
    // fills physical chunk i of a latent row, i.e. loads logical chunk i ^ sw16(key & 15)
    const uint32_t lds0 = lds_addr(smem);
    const uint32_t pe_lane = (uint32_t)(lane >> 3) * kPeBytes +
                             16u * ((lane & 7) ^ ((8 * wave + (lane >> 3)) >> 1 & 7));
    const uint32_t lane16 = 16u * lane;
    const uint64_t ck_base = reinterpret_cast<uint64_t>(a.ckv);
    const uint64_t pe_base = reinterpret_cast<uint64_t>(a.pe);
    const int k_hi_s = __builtin_amdgcn_readfirstlane(k_hi);
    // The descriptors cover exactly the wave's keys in range (its 8 keys are consecutive cache
    // rows of one page), so keys past the end read as zeros with no per-lane work; a block
    // past the last one loads nothing but zeros, so every step issues its 9 loads and every
    // wait counts the same 9 per block.  The 9 loads of a block go out one at a time between
    // the MFMAs of a step: issued back to back by all four waves they queue in the CU's
    // address unit and stall the MFMA stream behind them.
    struct Loads { v4i rk, rp; uint32_t st, st_pe; };
    // (fp8 cache: the raw rows, R and D bytes each, go to the wave's region of fp8 stage
    // j & 1 unpermuted; the wave converts them into the bf16 ring itself, see below)
    auto loads_of = [&](int j) __attribute__((always_inline)) {
        const int stage = j % NS;
        const int kb = __builtin_amdgcn_readfirstlane(k_lo + k2Keys * j + 8 * wave);
        const uint32_t left = (uint32_t)max(0, min(8, k_hi_s - kb));
        Loads d;
        const uint64_t row0 = (uint64_t)flash_key_row(a, b, kb, k_hi_s);
        if constexpr (FP8) {
            d.st = __builtin_amdgcn_readfirstlane(lds0 + kF8Base + (j & 1) * kF8Stage + wave * kF8Wave);
            d.st_pe = d.st + 8 * kFR;
            d.rk = rsrc_span(ck_base + row0 * kFR, 0, left * kFR);
            d.rp = rsrc_span(pe_base + row0 * kFD, 0, left * kFD);
        } else {
            d.st = __builtin_amdgcn_readfirstlane(lds0 + stage * k2LatStage + 8 * wave * kLatBytes);
            d.st_pe = __builtin_amdgcn_readfirstlane(lds0 + kPeBase + stage * k2PeStage + 8 * wave * kPeBytes);
            d.rk = rsrc_span(ck_base + row0 * kLatBytes, 0, left * kLatBytes);
            d.rp = rsrc_span(pe_base + row0 * kPeBytes, 0, left * kPeBytes);
        }
        return d;
    };
    const uint32_t pe8_lane = lane < 32 ? lane16 : kOob;   // 8 rope rows of 64 B: 32 lanes
    auto issue_one = [&](const Loads& d, int q) __attribute__((always_inline)) {
        if constexpr (FP8) {
            if (q < 4) dma16(d.rk, d.st + q * 1024, lane16, q * 1024);
            else dma16(d.rp, d.st_pe, pe8_lane, 0);
        } else {
            if (q < 8) dma16(d.rk, d.st + q * kLatBytes, lane16 ^ (16u * sw16((8 * wave + q) & 15)), q * kLatBytes);
            else dma16(d.rp, d.st_pe, pe_lane, 0);
        }
    };

    // ---- fp8 cache: each wave converts the rows it loaded (keys 8w .. 8w+7 of a block) into
    // the bf16 ring (F8Stage)
    const F8Stage f8(wave, lane, kPeBase);
    auto f8_read = [&](int j, int q) __attribute__((always_inline)) {
        return f8.read(smem, kF8Base + (j & 1) * kF8Stage + wave * kF8Wave, q, lane);
    };
    auto f8_write = [&](int j, int q, v4u raw) __attribute__((always_inline)) {
        f8.write(smem, j % NS, q, raw, lane);
    };

    // ---- per-lane LDS bases (byte offsets from smem); each read is base XOR a constant
    // plus an immediate, re-derived per step so no offset is held across the loop
    const int kk = 16 * kh + l16;                    // this lane's key in a block (K reads)
    uint32_t kb0 = kk * kLatBytes + 256u * g + 16u * sw16(l16);
    uint32_t pb0 = kPeBase + kk * kPeBytes + 16u * (g ^ ((kk >> 1) & 7));
    uint32_t vb0;
    {
        const int ch = g & 1, q = l16 >> 2, r = l16 & 3;
        vb0 = (16 * kh + 8 * hw + q) * kLatBytes + 16u * ((q << 2) | ((2 * ch + (r >> 1)) ^ (2 * hw))) +
              8u * (r & 1);
    }
    // stage st's copy of a latent base is base ^ 64 KB (st >> 1) + 32 KB (st & 1), of a rope
    // base base + 4 KB st; the bases stay below 32 KB (rope: inside their 4 KB), so no carry
    // reaches the bits the reads XOR in
    auto lat_base = [&](uint32_t base, int st) __attribute__((always_inline)) {
        return (base ^ (65536u * (uint32_t)(st >> 1))) + (uint32_t)(st & 1) * k2LatStage;
    };
    auto k_read = [&](uint32_t kbs, uint32_t pbs, int s) __attribute__((always_inline)) {
        const uint32_t off = s < kRSteps ? (kbs ^ (16u * s)) : (pbs ^ (64u * (s - kRSteps)));
        return *reinterpret_cast<const v4u*>(smem + off);
    };
    typedef short v4s __attribute__((ext_vector_type(4)));
    typedef __attribute__((address_space(3))) v4s lds_v4s;
    // V^T of column block cb (columns 32cb ..), keys 8(l/32) .. +7 of the wave's half
    auto v_read = [&](uint32_t vbs, int cb) __attribute__((always_inline)) {
        const uint32_t o = 256u * (cb >> 2);
        const uint32_t c = 64u * (cb & 3);
        const v4s lo = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_v4s*)(smem + ((vbs ^ c) + o)));
        const v4s hi = __builtin_amdgcn_ds_read_tr16_b64_v4i16(
            (lds_v4s*)(smem + ((vbs ^ (c | 16u)) + o + 4 * kLatBytes)));
        return __builtin_bit_cast(v4u, __builtin_shufflevector(lo, hi, 0, 1, 2, 3, 4, 5, 6, 7));
    };

    v16f O[16];
    float m_ref[2] = {-INFINITY, -INFINITY}, m_neg[2] = {0.f, 0.f};
    float thr[2] = {-INFINITY, -INFINITY}, l_run[2] = {0.f, 0.f};
    int pass = 1;
    bool overflow = false;   // this pass raised a row's reference (wave-uniform)
    v4u pb = {};             // P^T of the previous block in the B layout of the P.V MFMA
    v4u vq[2];               // the next two V^T fragments of the previous block

    // The softmax of block j's scores sc[0..1] against the rows' fixed references.  The
    // rare cases come first, each behind one wave-uniform branch: a block with masked keys
    // (the end of the range, a causal limit, or the block past the end, whose scores are
    // then all masked), and a row maximum past its reference's threshold (or a row without
    // a reference yet), which reduces the row maxima over the row's four lanes and moves
    // the reference (flagging the pass for a repeat if it had one).  The common path --
    // numerators, row sums, 16-bit P^T -- is branch-free and goes out in four parts that
    // the step interleaves with P.V MFMAs.
    struct Soft { v4f sc[2]; float e[2][4]; uint32_t x[2], y[2]; v4u pb; };
    auto soft_rare = [&](Soft& t, int j) __attribute__((always_inline)) {
        const int kq0 = k_lo + k2Keys * j + 16 * kh;
        if (kq0 + 15 > lim_wave) {
            const int kq = kq0 + 4 * g;
            #pragma unroll
            for (int i = 0; i < 4; ++i) {
                t.sc[0][i] = kq + i <= lim0 ? t.sc[0][i] : -INFINITY;
                t.sc[1][i] = kq + i <= lim1 ? t.sc[1][i] : -INFINITY;
            }
        }
        float mx[2];
        #pragma unroll
        for (int h = 0; h < 2; ++h)
            mx[h] = fmaxf(fmaxf(t.sc[h][0], t.sc[h][1]), fmaxf(t.sc[h][2], t.sc[h][3]));
        // rows are uniform over their four lanes after the reduction; NaN scores come here too
        if (__builtin_amdgcn_ballot_w64(!(mx[0] * a.c <= thr[0]) || !(mx[1] * a.c <= thr[1]))) {
            #pragma unroll
            for (int h = 0; h < 2; ++h) {
                const float bm = row4_reduce(mx[h], OpMax{}) * a.c;
                const bool over = pass < k2MaxPasses && m_ref[h] != -INFINITY && bm > thr[h];
                overflow |= __builtin_amdgcn_ballot_w64(over) != 0;
                if (m_ref[h] == -INFINITY || over) {
                    m_ref[h] = bm;
                    m_neg[h] = bm == -INFINITY ? 0.f : -bm;
                    thr[h] = bm + kHeadroom;
                }
            }
        }
    };
    auto soft_part = [&](Soft& t, auto part_tag) __attribute__((always_inline)) {
        constexpr int P = decltype(part_tag)::value;
        if constexpr (P == 0 || P == 1) {   // numerators of one row half
            #pragma unroll
            for (int i = 0; i < 4; ++i)
                t.e[P][i] = __builtin_amdgcn_exp2f(__builtin_fmaf(t.sc[P][i], a.c, m_neg[P]));
        } else if constexpr (P == 2) {   // row sums; 16-bit P^T
            l_run[0] += (t.e[0][0] + t.e[0][1]) + (t.e[0][2] + t.e[0][3]);
            l_run[1] += (t.e[1][0] + t.e[1][1]) + (t.e[1][2] + t.e[1][3]);
            #pragma unroll
            for (int d = 0; d < 2; ++d) {
                t.x[d] = Half<TL>::pack2(t.e[0][2 * d], t.e[0][2 * d + 1]);
                t.y[d] = Half<TL>::pack2(t.e[1][2 * d], t.e[1][2 * d + 1]);
            }
        } else {   // lane l (row half l/16 & 1) takes the other half's keys from lane l ^ 16
            const auto s0 = __builtin_amdgcn_permlane16_swap(t.x[0], t.y[0], false, false);
            const auto s1 = __builtin_amdgcn_permlane16_swap(t.x[1], t.y[1], false, false);
            t.pb = v4u{s0[0], s1[0], s0[1], s1[1]};
        }
    };

    // One 32-key block j in stage j % NS.  On entry pb and vq hold block j-1's P^T and its
    // first two V^T fragments (read before the barrier from a stage no load overwrites
    // before step j+1), so the MFMA stream resumes right after the barrier:
    //   P.V column blocks 0, 1 of block j-1 while block j's first K fragments arrive;
    //   18 K steps of block j's scores (two MFMAs each), with column blocks 2..7 of block
    //   j-1 and the nine loads of block j+2 spread among them;
    //   column blocks 8, 9 under block j's rare softmax cases, then its common softmax in
    //   four parts beside column blocks 10..15;
    //   block j's first two V^T fragments for the next step.
    // Step 0 has no previous block, and step nb only finishes block nb-1 (its scores, of
    // whatever stage nb % NS holds, are all masked).
    auto step = [&](int j, auto has_prev) __attribute__((always_inline)) {
        constexpr bool PREV = decltype(has_prev)::value;
        const Loads next = loads_of(j + 2);   // scalar work, ahead of the barrier
        if constexpr (FP8)
            wait_vm<0>();         // block j+1's raw rows (loaded in step j-1) have landed
        else
            wait_vm<kLoads>();    // block j has landed; block j+1's loads may be in flight
        lds_barrier();   // block j is in LDS for every wave; every wave is past block j-2's P.V

        constexpr int kWin = 3;
        asm volatile("" : "+v"(kb0), "+v"(pb0), "+v"(vb0));   // offsets derived per step
        const int st = j % NS;
        const uint32_t kbs = lat_base(kb0, st), pbs = pb0 + (uint32_t)st * k2PeStage;
        const uint32_t vbs = lat_base(vb0, (j + NS - 1) % NS);
        v4u kf[kWin];
        #pragma unroll
        for (int i = 0; i < kWin; ++i) kf[i] = k_read(kbs, pbs, i);
        auto pv = [&](int cb) __attribute__((always_inline)) {
            const v4u vc = vq[cb & 1];
            if (cb + 2 < 16) vq[cb & 1] = v_read(vbs, cb + 2);
            O[cb] = mfma32h<TL>(vc, pb, O[cb]);
        };
        if constexpr (PREV) {
            pv(0);
            pv(1);
        }
        Soft t;
        v4u f8raw;
        #pragma unroll
        for (int s = 0; s < kQSteps; ++s) {
            const v4u cur = kf[s % kWin];
            if (s + kWin < kQSteps) kf[s % kWin] = k_read(kbs, pbs, s + kWin);
            if (s == 0) {
                mfma16_v_first<TL>(cur, qf[0][s], t.sc[0]);
                mfma16_v_first<TL>(cur, qf[1][s], t.sc[1]);
            } else if (s + 1 < kQSteps) {
                mfma16_v<TL>(cur, qf[0][s], t.sc[0]);
                mfma16_v<TL>(cur, qf[1][s], t.sc[1]);
            } else {
                mfma16_v<TL>(cur, qf[0][s], t.sc[0]);
                mfma16_v_last<TL>(cur, qf[1][s], t.sc[1]);
            }
            if constexpr (FP8) {
                // block j+2's raw rows into the fp8 stage block j left; block j+1's into
                // the bf16 stage block j-2 left, each part read a K step before it is written
                if (s < kLoads) issue_one(next, s);
                if (s >= 5 && s < 15 && (s & 1)) f8raw = f8_read(j + 1, (s - 5) / 2);
                if (s >= 6 && s < 16 && !(s & 1)) f8_write(j + 1, (s - 6) / 2, f8raw);
            } else {
                if (s % 2 == 0) issue_one(next, s / 2);
            }
            if constexpr (PREV) {
                if (s % 3 == 0) pv(2 + s / 3);
            }
        }
        __builtin_amdgcn_sched_barrier(0);
        if constexpr (PREV) {
            pv(8);
            pv(9);
        }
        __builtin_amdgcn_sched_barrier(0);
        soft_rare(t, j);
        __builtin_amdgcn_sched_barrier(0);
        auto part = [&](auto p_tag, int cb0, int ncb) __attribute__((always_inline)) {
            if constexpr (PREV) {
                for (int cb = cb0; cb < cb0 + ncb; ++cb) pv(cb);
            }
            soft_part(t, p_tag);
            __builtin_amdgcn_sched_barrier(0);
        };
        part(std::integral_constant<int, 0>{}, 10, 2);
        part(std::integral_constant<int, 1>{}, 12, 2);
        part(std::integral_constant<int, 2>{}, 14, 1);
        part(std::integral_constant<int, 3>{}, 15, 1);
        pb = t.pb;
        const uint32_t vbn = lat_base(vb0, st);
        vq[0] = v_read(vbn, 0);
        vq[1] = v_read(vbn, 1);
    };

    // A pass over the split's keys; repeated from the first key, by every wave, only when a
    // row's maximum outgrew its reference (each repeat raises that row's reference by more
    // than the headroom; after k2MaxPasses passes the last one stands).  A pass that raised
    // a reference runs to its end (its sums are then discarded); the waves learn of it
    // through four flags in the then idle ring.
    int* flags = reinterpret_cast<int*>(smem);
    for (;; ++pass) {
        #pragma unroll
        for (int i = 0; i < 16; ++i) O[i] = v16f{};
        l_run[0] = l_run[1] = 0.f;
        overflow = false;
        if (nb == 0) break;
        #pragma unroll
        for (int j = 0; j < 2; ++j) {
            const Loads d = loads_of(j);
            #pragma unroll
            for (int q = 0; q < kLoads; ++q) issue_one(d, q);
        }
        if constexpr (FP8) {   // block 0 into the bf16 ring before the first step
            wait_vm<kLoads>();
            #pragma unroll
            for (int q = 0; q < kLoads; ++q) f8_write(0, q, f8_read(0, q));
        }
        step(0, std::false_type{});
        #pragma unroll 1
        for (int j = 1; j <= nb; ++j) step(j, std::true_type{});
        wait_vm<0>();    // the zero loads of the blocks past the end have landed
        lds_barrier();   // every wave is done with the ring
        if (lane == 0) flags[wave] = overflow ? 1 : 0;
        lds_barrier();
        const bool again = (flags[0] | flags[1] | flags[2] | flags[3]) != 0;
        lds_barrier();   // the flags are read before the ring is written again
        if (!again) break;
    }

    // ---- merge the two key halves of each row tile: wave (rt, 1) leaves its O, row maxima
    // and row sums in LDS, wave (rt, 0) rescales both to the larger maximum and writes
    // (O region: 64 KB per row tile, lane-major so each lane reads back its own layout)
    l_run[0] = row4_reduce(l_run[0], OpSum{});
    l_run[1] = row4_reduce(l_run[1], OpSum{});
    float* ml = reinterpret_cast<float*>(smem + 2 * 65536);   // [rt][kh][m, l][32 rows]
    v4f* oreg = reinterpret_cast<v4f*>(smem + rt * 65536) + lane;
    if (g == 0) {
        float* mlw = ml + (rt * 2 + kh) * 64;
        mlw[l16] = m_ref[0];
        mlw[16 + l16] = m_ref[1];
        mlw[32 + l16] = l_run[0];
        mlw[48 + l16] = l_run[1];
    }
    if (kh == 1) {
        #pragma unroll
        for (int cb = 0; cb < 16; ++cb)
            #pragma unroll
            for (int q = 0; q < 4; ++q)
                oreg[64 * (4 * cb + q)] = v4f{O[cb][4 * q], O[cb][4 * q + 1], O[cb][4 * q + 2], O[cb][4 * q + 3]};
    }
    lds_barrier();
    if (kh == 1) return;
    const float* mla = ml + (rt * 2) * 64;
    const float* mlb = mla + 64;
    const float ma = mla[l32], mb = mlb[l32];
    const float M = fmaxf(ma, mb);
    const float fa = ma == -INFINITY ? 0.f : __builtin_amdgcn_exp2f(ma - M);
    const float fb = mb == -INFINITY ? 0.f : __builtin_amdgcn_exp2f(mb - M);
    const float lsum = mla[32 + l32] * fa + mlb[32 + l32] * fb;
    // an fp8 cache's values are its codes times kv_scale: ctx takes the factor once here
    const float oa_f = FP8 ? fa * a.o_scale : fa, ob_f = FP8 ? fb * a.o_scale : fb;
    if (rowO < rows_b) {
        const int64_t slot = (work.direct ? (int64_t)b : work.slot) * rows_b + rowO;
        if (hw == 0) {
            if (!work.direct) a.m[slot] = M;
            (work.direct ? a.l_direct : a.l)[slot] = lsum;
        }
        float* orow = (work.direct ? a.o_direct : a.o) + slot * kFR + 4 * hw;
        #pragma unroll
        for (int cb = 0; cb < 16; ++cb)
            #pragma unroll
            for (int q = 0; q < 4; ++q) {
                const v4f ob = oreg[64 * (4 * cb + q)];
                const v4f oa = {O[cb][4 * q], O[cb][4 * q + 1], O[cb][4 * q + 2], O[cb][4 * q + 3]};
                *reinterpret_cast<v4f*>(orow + 32 * cb + 8 * q) = oa * oa_f + ob * ob_f;
            }
    }
}

// ------------------------------------------------------------------ 16-bit: specialised waves
// The same 64-row tile, 32-key blocks, staging and LDS ring as flash16_kernel, on eight
// waves whose work is split by kind instead of by key half (two waves per SIMD, so one
// issues while the other waits on LDS):
//   score waves 0-3 (row tile rt = w/2, key half kh = w%2): K reads, the 36 score MFMAs
//     and the softmax of flash16_kernel; they write P^T (16-bit, 32 rows x 16 keys) into
//     one of two LDS P stages instead of keeping it;
//   P.V waves 4-7 (row tile rt, column half ch): O^T for 256 columns x 32 rows (128
//     VGPRs), one block behind: in step j they read block j-1's P^T for both key halves
//     and its V^T fragments (transposing reads, as before) and run 16 32x32x16 MFMAs;
//     they also issue the staging loads (flash16_kernel's, block j+2 in step j) between
//     their MFMAs and wait for them before each step's barrier.  With the loads in the
//     score waves instead, the pass took about 10% longer: the score waves carry the
//     longer MFMA chain and the softmax, and the loads' issue cost lands on it.
// Both key halves of a row must share one reference for their P^T to sum in one O, so at
// the first block of a pass the two score waves of a row tile exchange their proposals
// through LDS (the row maximum over the block, or the reference a previous pass raised)
// and both take the larger; a row's first visible key lies in that block's first half, so
// every row with keys gets a finite reference there.  A row that later passes it raises
// its own half's reference and flags the pass for a repeat, as before.  P.V of block j-1
// reads stage (j-1) % 4 of the ring while block j+2 loads into stage (j+2) % 4, and P^T
// stage (j-1) & 1 while the score waves write stage j & 1: one barrier per step orders all
// of it.  The two kinds run separate loops with the same barriers, so neither holds the
// other's registers: Q^T (144) and O^T (128) both fit the 256 VGPRs of a wave at two waves
// per SIMD, with no AGPRs.  The P.V loop starts at block 1 (block 0's step only has its
// barriers), so the accumulators never meet a branch inside the loop; with that step inside
// the loop the register allocator copies and spills them.  No key-half merge at the end:
// the score waves leave row sums and references in LDS and the P.V waves write the rows.
// An fp8 cache (FP8): the P.V waves load the raw rows into two fp8 stages (F8Stage) and,
// during step j, convert block j+1 into the bf16 ring (three stages, into the one block j-2
// left) while block j+2's raw rows load; the score waves see the same bf16 ring as ever.
constexpr int kXThreads = 512;
constexpr int kXPPitch = 80;                              // bytes per P^T row: 32 keys + pad
constexpr int kXPStage = 2 * 32 * kXPPitch;               // both row tiles

// PV64: each P.V wave covers all 64 rows of the tile and a quarter of the columns (128),
// instead of one row tile and half the columns: the same 128 accumulator registers and 16
// MFMAs per block, half the V^T fragment reads (each V^T fragment feeds both row tiles) for
// twice the P^T reads.
template <typename TL, bool FP8, bool PV64 = false>
__global__ void __launch_bounds__(kXThreads, 1) flash16x_kernel(FlashArgs a) {
    static_assert(!FP8 || !Half<TL>::kF16, "an fp8 cache is read with bf16 queries");
    constexpr int NS = FP8 ? 3 : 4;                             // bf16 ring stages
    constexpr float kHeadroom = Half<TL>::kF16 ? 15.f : k2Headroom;
    constexpr int kLoads = FP8 ? k8Loads : k2Loads;             // cache loads per wave and block
    constexpr int kPeBase = NS * k2LatStage;                    // 128 KB (fp8: 96 KB)
    constexpr int kPBase = kPeBase + NS * k2PeStage;            // two P^T stages
    constexpr int kF8Base = kPBase + 2 * kXPStage;              // fp8: two raw stages
    constexpr int kXBase = kF8Base + (FP8 ? 2 * kF8Stage : 0);  // references, sums, flags
    __shared__ __attribute__((aligned(1024))) uint8_t smem[kXBase + 2 * 128 * 4 + 64];
    float* xref = reinterpret_cast<float*>(smem + kXBase);      // [rt][kh][32 rows]
    float* xl = xref + 128;                                     // [rt][kh][32 rows]
    int* flags = reinterpret_cast<int*>(xl + 128);              // [score wave]
    const int tid = threadIdx.x, lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int l16 = lane & 15, g = lane >> 4, l32 = lane & 31, hw = lane >> 5;
    const FlashWork work = flash_work(a);
    if (work.skip) return;   // past the end of a work list: the whole workgroup leaves

    const int b = work.b;
    const int rows_b = a.Sq * a.H;
    const int r0 = work.rt * kFRows;
    const int skb = flash_batch_keys(a, b);
    const int k_lo = work.k_lo;
    const int k_end = min(skb, k_lo + work.k_len);
    int k_hi = k_end;
    if (a.causal) k_hi = min(k_hi, skb - a.Sq + min(r0 + kFRows - 1, rows_b - 1) / a.H + 1);
    const int nb = k_hi > k_lo ? (k_hi - k_lo + k2Keys - 1) / k2Keys : 0;
    auto lat_base = [&](uint32_t base, int st) __attribute__((always_inline)) {
        return (base ^ (65536u * (uint32_t)(st >> 1))) + (uint32_t)(st & 1) * k2LatStage;
    };

    if (wave < 4) {
        // ================================ score waves
        const int rt = wave >> 1, kh = wave & 1;
        const int rbase = r0 + 32 * rt;
        const int rowS0 = rbase + l16, rowS1 = rbase + 16 + l16;
        int lim0 = k_end - 1, lim1 = k_end - 1;
        if (a.causal) {
            lim0 = min(lim0, skb - a.Sq + min(rowS0, rows_b - 1) / a.H);
            lim1 = min(lim1, skb - a.Sq + min(rowS1, rows_b - 1) / a.H);
        }
        const int lim_wave = __builtin_amdgcn_readfirstlane(lim0);
        const __amdgpu_buffer_rsrc_t rq = make_rsrc(a.qa + (int64_t)b * rows_b * kFR);
        const __amdgpu_buffer_rsrc_t rr = make_rsrc(a.qr + (int64_t)b * rows_b * kFD);
        v4u qf[2][kQSteps];
        #pragma unroll
        for (int t = 0; t < 2; ++t) {
            const int row = t ? rowS1 : rowS0;
            const uint32_t qmask = oob_mask(row, rows_b);
            #pragma unroll
            for (int s = 0; s < kQSteps; ++s)
                qf[t][s] = s < kRSteps
                               ? load16(rq, ((uint32_t)row * kLatBytes + 256u * g + 16u * s) | qmask)
                               : load16(rr, ((uint32_t)row * kPeBytes + 64u * (s - kRSteps) + 16u * g) | qmask);
        }
        wait_vm<0>();   // Q in registers

        const int kk = 16 * kh + l16;
        uint32_t kb0 = kk * kLatBytes + 256u * g + 16u * sw16(l16);
        uint32_t pb0 = kPeBase + kk * kPeBytes + 16u * (g ^ ((kk >> 1) & 7));
        auto k_read = [&](uint32_t kbs, uint32_t pbs, int s) __attribute__((always_inline)) {
            const uint32_t off = s < kRSteps ? (kbs ^ (16u * s)) : (pbs ^ (64u * (s - kRSteps)));
            return *reinterpret_cast<const v4u*>(smem + off);
        };
        // P^T writes: rows 16h + l16 of the tile, keys 16kh + 4g .. +3 (8 bytes)
        const uint32_t pw0 = kPBase + rt * 32 * kXPPitch + l16 * kXPPitch + 2u * (16 * kh + 4 * g);

        float m_ref[2] = {-INFINITY, -INFINITY}, m_neg[2] = {0.f, 0.f};
        float thr[2] = {-INFINITY, -INFINITY}, l_run[2] = {0.f, 0.f};
        for (int pass = 1;; ++pass) {
            l_run[0] = l_run[1] = 0.f;
            bool overflow = false;
            if (nb == 0) break;
            #pragma unroll 1
            for (int j = 0; j <= nb; ++j) {
                lds_barrier();        // A_j: block j is in LDS, P.V of block j-2 is done
                v4f sc[2];
                if (j < nb) {
                    constexpr int kWin = 3;
                    asm volatile("" : "+v"(kb0), "+v"(pb0));
                    const int st = j % NS;
                    const uint32_t kbs = lat_base(kb0, st), pbs = pb0 + (uint32_t)st * k2PeStage;
                    v4u kf[kWin];
                    #pragma unroll
                    for (int i = 0; i < kWin; ++i) kf[i] = k_read(kbs, pbs, i);
                    #pragma unroll
                    for (int s = 0; s < kQSteps; ++s) {
                        const v4u cur = kf[s % kWin];
                        if (s + kWin < kQSteps) kf[s % kWin] = k_read(kbs, pbs, s + kWin);
                        if (s == 0) {
                            mfma16_v_first<TL>(cur, qf[0][s], sc[0]);
                            mfma16_v_first<TL>(cur, qf[1][s], sc[1]);
                        } else if (s + 1 < kQSteps) {
                            mfma16_v<TL>(cur, qf[0][s], sc[0]);
                            mfma16_v<TL>(cur, qf[1][s], sc[1]);
                        } else {
                            mfma16_v<TL>(cur, qf[0][s], sc[0]);
                            mfma16_v_last<TL>(cur, qf[1][s], sc[1]);
                        }
                    }
                    __builtin_amdgcn_sched_barrier(0);
                    const int kq0 = k_lo + k2Keys * j + 16 * kh;
                    if (kq0 + 15 > lim_wave) {
                        const int kq = kq0 + 4 * g;
                        #pragma unroll
                        for (int i = 0; i < 4; ++i) {
                            sc[0][i] = kq + i <= lim0 ? sc[0][i] : -INFINITY;
                            sc[1][i] = kq + i <= lim1 ? sc[1][i] : -INFINITY;
                        }
                    }
                    if (j == 0) {
                        // the pass's reference proposal of each row: the raised one of a
                        // previous pass, else this block's maximum over the half's keys
                        #pragma unroll
                        for (int h = 0; h < 2; ++h) {
                            const float mx = fmaxf(fmaxf(sc[h][0], sc[h][1]), fmaxf(sc[h][2], sc[h][3]));
                            const float bm = row4_reduce(mx, OpMax{}) * a.c;
                            const float prop = m_ref[h] == -INFINITY ? bm : m_ref[h];
                            if (g == 0) xref[(rt * 2 + kh) * 32 + 16 * h + l16] = prop;
                        }
                    }
                }
                if (j == 0) {
                    lds_barrier();    // X: both halves' proposals are in LDS
                    #pragma unroll
                    for (int h = 0; h < 2; ++h) {
                        const int r = 16 * h + l16;
                        const float ref = fmaxf(xref[(rt * 2) * 32 + r], xref[(rt * 2 + 1) * 32 + r]);
                        m_ref[h] = ref;
                        m_neg[h] = ref == -INFINITY ? 0.f : -ref;
                        thr[h] = ref + kHeadroom;
                    }
                }
                if (j < nb) {
                    float mx[2];
                    #pragma unroll
                    for (int h = 0; h < 2; ++h)
                        mx[h] = fmaxf(fmaxf(sc[h][0], sc[h][1]), fmaxf(sc[h][2], sc[h][3]));
                    // a row past its threshold raises its reference and flags a repeat (NaN
                    // scores come here too); rows without a reference have no visible key
                    if (__builtin_amdgcn_ballot_w64(!(mx[0] * a.c <= thr[0]) || !(mx[1] * a.c <= thr[1]))) {
                        #pragma unroll
                        for (int h = 0; h < 2; ++h) {
                            const float bm = row4_reduce(mx[h], OpMax{}) * a.c;
                            const bool over = pass < k2MaxPasses && m_ref[h] != -INFINITY && bm > thr[h];
                            overflow |= __builtin_amdgcn_ballot_w64(over) != 0;
                            if (over) {
                                m_ref[h] = bm;
                                m_neg[h] = -bm;
                                thr[h] = bm + kHeadroom;
                            }
                        }
                    }
                    const uint32_t pws = pw0 + (uint32_t)(j & 1) * kXPStage;
                    #pragma unroll
                    for (int h = 0; h < 2; ++h) {
                        float e[4];
                        #pragma unroll
                        for (int i = 0; i < 4; ++i)
                            e[i] = __builtin_amdgcn_exp2f(__builtin_fmaf(sc[h][i], a.c, m_neg[h]));
                        l_run[h] += (e[0] + e[1]) + (e[2] + e[3]);
                        typedef uint32_t v2u __attribute__((ext_vector_type(2)));
                        *reinterpret_cast<v2u*>(smem + pws + 16u * h * kXPPitch) =
                            v2u{Half<TL>::pack2(e[0], e[1]), Half<TL>::pack2(e[2], e[3])};
                    }
                }
            }
            lds_barrier();   // B1: every wave is done with the ring
            if (lane == 0) flags[wave] = overflow ? 1 : 0;
            lds_barrier();   // B2
            const bool again = (flags[0] | flags[1] | flags[2] | flags[3]) != 0;
            lds_barrier();   // B3: the flags are read before they are written again
            if (!again) break;
        }
        // row sums of the half and the shared references for the P.V waves
        #pragma unroll
        for (int h = 0; h < 2; ++h) {
            const float l = row4_reduce(l_run[h], OpSum{});
            if (g == 0) {
                xl[(rt * 2 + kh) * 32 + 16 * h + l16] = l;
                if (kh == 0) xref[(rt * 2) * 32 + 16 * h + l16] = m_ref[h];
            }
        }
        lds_barrier();   // F: sums and references are in LDS
        return;
    }

    // ==================================== P.V waves
    const int rt = (wave - 4) >> 1, ch = (wave - 4) & 1;
    const int cq = wave - 4;             // PV64: column quarter
    const int rowO = r0 + 32 * rt + l32;
    // V^T fragments of key half ks (keys 16ks + 8(l/32) .. +7) of column block cb
    uint32_t vb0[2];
    #pragma unroll
    for (int ks = 0; ks < 2; ++ks) {
        const int cq = g & 1, q = l16 >> 2, r = l16 & 3;
        vb0[ks] = (16 * ks + 8 * hw + q) * kLatBytes +
                  16u * ((q << 2) | ((2 * cq + (r >> 1)) ^ (2 * hw))) + 8u * (r & 1);
    }
    typedef short v4s __attribute__((ext_vector_type(4)));
    typedef __attribute__((address_space(3))) v4s lds_v4s;
    auto v_read = [&](uint32_t vbs, int cb) __attribute__((always_inline)) {
        const uint32_t o = 256u * (cb >> 2);
        const uint32_t c = 64u * (cb & 3);
        const v4s lo = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_v4s*)(smem + ((vbs ^ c) + o)));
        const v4s hi = __builtin_amdgcn_ds_read_tr16_b64_v4i16(
            (lds_v4s*)(smem + ((vbs ^ (c | 16u)) + o + 4 * kLatBytes)));
        return __builtin_bit_cast(v4u, __builtin_shufflevector(lo, hi, 0, 1, 2, 3, 4, 5, 6, 7));
    };
    // P^T of key half ks in the B layout: row l32, keys 16ks + 8(l/32) .. +7 (PV64: of row
    // tile 0; row tile 1's is 32 rows further)
    const uint32_t pr0 = kPBase + (PV64 ? 0 : rt * 32 * kXPPitch) + l32 * kXPPitch + 16u * hw;
    // staging: P.V wave 4 + w loads keys 8w .. 8w+7 of a block (flash16_kernel's layout),
    // block j+2 during step j, and waits for block j before barrier A_j (fp8: for block j+1
    // before converting it, in the same step)
    const int wv = wave - 4;
    const uint32_t lds0 = lds_addr(smem);
    const uint32_t pe_lane = (uint32_t)(lane >> 3) * kPeBytes +
                             16u * ((lane & 7) ^ ((8 * wv + (lane >> 3)) >> 1 & 7));
    const uint32_t lane16 = 16u * lane;
    const uint64_t ck_base = reinterpret_cast<uint64_t>(a.ckv);
    const uint64_t pe_base = reinterpret_cast<uint64_t>(a.pe);
    const int k_hi_s = __builtin_amdgcn_readfirstlane(k_hi);
    struct Loads { v4i rk, rp; uint32_t st, st_pe; };
    auto loads_of = [&](int j) __attribute__((always_inline)) {
        const int stage = j % NS;
        const int kb = __builtin_amdgcn_readfirstlane(k_lo + k2Keys * j + 8 * wv);
        const uint32_t left = (uint32_t)max(0, min(8, k_hi_s - kb));
        Loads d;
        const uint64_t row0 = (uint64_t)flash_key_row(a, b, kb, k_hi_s);
        if constexpr (FP8) {
            d.st = __builtin_amdgcn_readfirstlane(lds0 + kF8Base + (j & 1) * kF8Stage + wv * kF8Wave);
            d.st_pe = d.st + 8 * kFR;
            d.rk = rsrc_span(ck_base + row0 * kFR, 0, left * kFR);
            d.rp = rsrc_span(pe_base + row0 * kFD, 0, left * kFD);
        } else {
            d.st = __builtin_amdgcn_readfirstlane(lds0 + stage * k2LatStage + 8 * wv * kLatBytes);
            d.st_pe = __builtin_amdgcn_readfirstlane(lds0 + kPeBase + stage * k2PeStage + 8 * wv * kPeBytes);
            d.rk = rsrc_span(ck_base + row0 * kLatBytes, 0, left * kLatBytes);
            d.rp = rsrc_span(pe_base + row0 * kPeBytes, 0, left * kPeBytes);
        }
        return d;
    };
    const uint32_t pe8_lane = lane < 32 ? lane16 : kOob;   // 8 rope rows of 64 B: 32 lanes
    auto issue_one = [&](const Loads& d, int q) __attribute__((always_inline)) {
        if constexpr (FP8) {
            if (q < 4) dma16(d.rk, d.st + q * 1024, lane16, q * 1024);
            else dma16(d.rp, d.st_pe, pe8_lane, 0);
        } else {
            if (q < 8) dma16(d.rk, d.st + q * kLatBytes, lane16 ^ (16u * sw16((8 * wv + q) & 15)), q * kLatBytes);
            else dma16(d.rp, d.st_pe, pe_lane, 0);
        }
    };
    const F8Stage f8(wv, lane, kPeBase);
    auto f8_read = [&](int j, int q) __attribute__((always_inline)) {
        return f8.read(smem, kF8Base + (j & 1) * kF8Stage + wv * kF8Wave, q, lane);
    };
    auto f8_write = [&](int j, int q, v4u raw) __attribute__((always_inline)) {
        f8.write(smem, j % NS, q, raw, lane);
    };
    v16f O[8];
    for (int pass = 1;; ++pass) {
        #pragma unroll
        for (int i = 0; i < 8; ++i) O[i] = v16f{};
        if (nb == 0) break;
        #pragma unroll
        for (int j = 0; j < 2; ++j) {
            const Loads d = loads_of(j);
            #pragma unroll
            for (int q = 0; q < kLoads; ++q) issue_one(d, q);
        }
        wait_vm<kLoads>();                 // block 0 has landed; block 1 may be in flight
        if constexpr (FP8) {               // block 0 into the bf16 ring
            #pragma unroll
            for (int q = 0; q < kLoads; ++q) f8_write(0, q, f8_read(0, q));
        }
        lds_barrier();                     // A_0
        {
            const Loads d = loads_of(2);   // stage 2 is free from the pass's start
            #pragma unroll
            for (int q = 0; q < kLoads; ++q) issue_one(d, q);
        }
        if constexpr (FP8) {               // block 1, landed, into the bf16 ring
            wait_vm<kLoads>();
            #pragma unroll
            for (int q = 0; q < kLoads; ++q) f8_write(1, q, f8_read(1, q));
        }
        lds_barrier();                     // X
        #pragma unroll 1
        for (int j = 1; j <= nb; ++j) {
            const Loads next = loads_of(j + 2);
            if constexpr (!FP8)
                wait_vm<k2Loads>();        // block j has landed; block j+1 may be in flight
            lds_barrier();                 // A_j (fp8: block j was converted in step j-1)
            // Wave priority (the default layout): the step's first 4 of 16 MFMAs go ahead of
            // the score wave's on the SIMD, the rest behind.  cfg4 bf16, the same bits: equal
            // priorities 172.2-176.9 us, this 169.5-171.9 us; the first 2, 6, 8 or 12 MFMAs
            // 171.7, 172.5, 177.5 and 179.5 us (medians), the whole step 5-8% slower.
            if constexpr (PV64 && !FP8) __builtin_amdgcn_s_setprio(1);
            {
                asm volatile("" : "+v"(vb0[0]), "+v"(vb0[1]));
                const int st = (j - 1) % NS;
                const uint32_t prs = pr0 + (uint32_t)((j - 1) & 1) * kXPStage;
                // P^T fragments [row tile][key half] (without PV64 only row tile 0's slot
                // is used: this wave's own tile)
                v4u pf[2][2];
                #pragma unroll
                for (int t = 0; t < (PV64 ? 2 : 1); ++t)
                    #pragma unroll
                    for (int ks = 0; ks < 2; ++ks)
                        pf[t][ks] = *reinterpret_cast<const v4u*>(smem + prs + t * 32 * kXPPitch + 32u * ks);
                const uint32_t vs0 = lat_base(vb0[0], st), vs1 = lat_base(vb0[1], st);
                constexpr int kVWin = 4;
                v4u vf[kVWin];
                // without PV64, fragment f (one per MFMA t): key half f/8, column block
                // 8ch + f%8; with PV64 (one per two MFMAs, t = 2f and 2f + 1 for the two row
                // tiles): key half f/4, column block 4cq + f%4.  Consecutive MFMAs use
                // different accumulators; each one's next use comes 8 MFMAs later.
                constexpr int kVFrags = PV64 ? 8 : 16;
                auto vfrag = [&](int f) __attribute__((always_inline)) {
                    if constexpr (PV64) return v_read((f >> 2) ? vs1 : vs0, 4 * cq + (f & 3));
                    else return v_read((f >> 3) ? vs1 : vs0, 8 * ch + (f & 7));
                };
                #pragma unroll
                for (int f = 0; f < kVWin; ++f) vf[f] = vfrag(f);
                v4u f8raw;
                v4u cur;
                #pragma unroll
                for (int t = 0; t < 16; ++t) {
                    const int f = PV64 ? t >> 1 : t;
                    if (!PV64 || (t & 1) == 0) {
                        cur = vf[f % kVWin];
                        if (f + kVWin < kVFrags) vf[f % kVWin] = vfrag(f + kVWin);
                    }
                    if constexpr (PV64)
                        O[t & 7] = mfma32h<TL>(cur, pf[t & 1][f >> 2], O[t & 7]);
                    else
                        O[t & 7] = mfma32h<TL>(cur, pf[0][t >> 3], O[t & 7]);
                    if constexpr (FP8) {
                        // block j+2's raw rows into the fp8 stage block j left; then block
                        // j+1's, landed, into bf16 stage (j+1) % 3, which block j-2 left at
                        // barrier A_j, each part read an MFMA before it is written
                        if (t < kLoads) issue_one(next, t);
                        if (t == kLoads) wait_vm<kLoads>();
                        if (t >= 5 && t < 15 && (t & 1)) f8raw = f8_read(j + 1, (t - 5) / 2);
                        if (t >= 6 && t < 16 && !(t & 1)) f8_write(j + 1, (t - 6) / 2, f8raw);
                    } else {
                        // block j+2 into stage (j+2) % 4, which block j-2 left at barrier A_j
                        if (t % 2 == 0) issue_one(next, t / 2);
                        if (t == 15) issue_one(next, 8);
                    }
                    if constexpr (PV64 && !FP8)
                        if (t == 3) __builtin_amdgcn_s_setprio(0);
                }
            }
        }
        wait_vm<0>();    // the zero loads of the blocks past the end have landed
        lds_barrier();   // B1
        lds_barrier();   // B2
        const bool again = (flags[0] | flags[1] | flags[2] | flags[3]) != 0;
        lds_barrier();   // B3
        if (!again) break;
    }
    lds_barrier();       // F
    // an fp8 cache's values are its codes times kv_scale: ctx takes the factor here
    const float of = FP8 ? a.o_scale : 1.f;
    if constexpr (PV64) {
        // both row tiles, columns 128cq .. +127: O[2 cb + t] is column block cb of row tile t
        #pragma unroll
        for (int t = 0; t < 2; ++t) {
            const int row = r0 + 32 * t + l32;
            if (row >= rows_b) continue;
            const float* xlr = xl + t * 64;
            const float lsum = xlr[l32] + xlr[32 + l32];
            const float M = xref[t * 64 + l32];
            const int64_t slot = (work.direct ? (int64_t)b : work.slot) * rows_b + row;
            if (a.ctx16) {
                const float r = lsum == 0.f ? 0.f : 1.f / lsum;
                uint16_t* crow = static_cast<uint16_t*>(a.ctx16) + slot * kFR + 128 * cq + 4 * hw;
                #pragma unroll
                for (int cb = 0; cb < 4; ++cb)
                    #pragma unroll
                    for (int q = 0; q < 4; ++q) {
                        const v4f v = v4f{O[2 * cb + t][4 * q], O[2 * cb + t][4 * q + 1],
                                          O[2 * cb + t][4 * q + 2], O[2 * cb + t][4 * q + 3]} * of;
                        const v4f w = v * r;
                        *reinterpret_cast<v2u*>(crow + 32 * cb + 8 * q) =
                            v2u{Half<TL>::pack2(w[0], w[1]), Half<TL>::pack2(w[2], w[3])};
                    }
                continue;
            }
            if (cq == 0 && hw == 0) {
                if (!work.direct) a.m[slot] = M;
                (work.direct ? a.l_direct : a.l)[slot] = lsum;
            }
            float* orow = (work.direct ? a.o_direct : a.o) + slot * kFR + 128 * cq + 4 * hw;
            #pragma unroll
            for (int cb = 0; cb < 4; ++cb)
                #pragma unroll
                for (int q = 0; q < 4; ++q)
                    *reinterpret_cast<v4f*>(orow + 32 * cb + 8 * q) =
                        v4f{O[2 * cb + t][4 * q], O[2 * cb + t][4 * q + 1],
                            O[2 * cb + t][4 * q + 2], O[2 * cb + t][4 * q + 3]} * of;
        }
    } else if (rowO < rows_b) {
        const float* xlr = xl + rt * 64;
        const float lsum = xlr[l32] + xlr[32 + l32];
        const float M = xref[rt * 64 + l32];
        const int64_t slot = (work.direct ? (int64_t)b : work.slot) * rows_b + rowO;
        if (ch == 0 && hw == 0) {
            if (!work.direct) a.m[slot] = M;
            (work.direct ? a.l_direct : a.l)[slot] = lsum;
        }
        float* orow = (work.direct ? a.o_direct : a.o) + slot * kFR + 256 * ch + 4 * hw;
        #pragma unroll
        for (int cb = 0; cb < 8; ++cb)
            #pragma unroll
            for (int q = 0; q < 4; ++q)
                *reinterpret_cast<v4f*>(orow + 32 * cb + 8 * q) =
                    v4f{O[cb][4 * q], O[cb][4 * q + 1], O[cb][4 * q + 2], O[cb][4 * q + 3]} * of;
    }
}

// ------------------------------------------------------------------ fp8 cache: a ring of codes
// The fp8-cache pass on flash16x_kernel's eight specialised waves (PV64 layout: each P.V
// wave covers the tile's 64 rows and 128 columns), with only the e4m3 codes in LDS: every
// fragment is read as codes and converted to bf16 in registers, straight into the MFMA
// operand (v_cvt_scalef32_pk_bf16_fp8, exact, scale 1; kv_scale goes to the score
// coefficient and the output as before).  A block is 18 KB (32 keys x 512 latent bytes,
// then 32 x 64 rope bytes) instead of the bf16 ring's 36 KB, so the ring holds eight
// blocks: the P.V waves issue block j+6 during step j, 108 KB in flight per workgroup.
//   Score waves: K step s of lane group g = l/16 is depth 32s + 8g .. +7 of key 16kh + l%16
//     (Q^T is loaded in the same order): an 8-byte read (ds_read_b64) and four conversions.
//   P.V waves: the V^T fragment of key half ks and column block cb (32 columns) comes from
//     ds_read_b64_tr_b8: within each 16-lane group, lanes 2r and 2r+1 address bytes
//     0-7 and 8-15 of one 16-byte row (key r of the group's eight) and lane j receives byte
//     column j of those eight rows -- eight keys of one column, the operand lane's K values.
//   Layout: 16-byte chunk c of latent row k sits at c ^ swz(k & 15) (bits 0-3 of the chunk
//     index: within its 256-byte window), chunk c of rope row k at c ^ ((k >> 2) & 3).
//     Each 32-lane half of a K read then touches 16 keys x 2 halves of chunks and each
//     half of a V^T read 8 keys x 4 eight-byte slots, all distinct 8-byte slots of 256
//     bytes: no bank conflicts.  The direct-to-LDS loads write chunk positions in order and
//     take the permutation in their global offsets.
//   Loads: P.V wave w loads latent keys 8w .. 8w+7 (four 1 KB loads, two rows each); waves
//     0 and 1 also load the rope rows of keys 16w .. 16w+15 (one 1 KB load).
constexpr int k8LatBytes = kFR;                        // 512 B of codes per latent row
constexpr int k8PeBytes = kFD;                         // 64 B per rope row
constexpr int k8LatStage = 32 * k8LatBytes;            // 16 KB
constexpr int k8Stage = k8LatStage + 32 * k8PeBytes;   // 18 KB per block
constexpr int k8NS = 8;                                // ring stages
constexpr int k8Ahead = k8NS - 2;                      // blocks in flight past the next one

typedef int32_t v2i __attribute__((ext_vector_type(2)));

// eight e4m3 codes (bytes 0..7) -> eight bf16 in operand order
__device__ __forceinline__ v4u fp8x8_bf16(v2u r) {
    auto lo2 = [](uint32_t w) __attribute__((always_inline)) {
        return __builtin_bit_cast(uint32_t, __builtin_amdgcn_cvt_scalef32_pk_bf16_fp8(w, 1.f, false));
    };
    auto hi2 = [](uint32_t w) __attribute__((always_inline)) {
        return __builtin_bit_cast(uint32_t, __builtin_amdgcn_cvt_scalef32_pk_bf16_fp8(w, 1.f, true));
    };
    return v4u{lo2(r[0]), hi2(r[0]), lo2(r[1]), hi2(r[1])};
}

__global__ void __launch_bounds__(kXThreads, 1) flash16x8_kernel(FlashArgs a) {
    typedef bf16_t TL;
    constexpr float kHeadroom = k2Headroom;
    constexpr int kPBase = k8NS * k8Stage;                      // 144 KB: two P^T stages
    constexpr int kXBase = kPBase + 2 * kXPStage;               // references, sums, flags
    __shared__ __attribute__((aligned(1024))) uint8_t smem[kXBase + 2 * 128 * 4 + 64];
    float* xref = reinterpret_cast<float*>(smem + kXBase);      // [rt][kh][32 rows]
    float* xl = xref + 128;                                     // [rt][kh][32 rows]
    int* flags = reinterpret_cast<int*>(xl + 128);              // [score wave]
    const int tid = threadIdx.x, lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int l16 = lane & 15, g = lane >> 4, l32 = lane & 31, hw = lane >> 5;
    const FlashWork work = flash_work(a);
    if (work.skip) return;   // past the end of a work list: the whole workgroup leaves

    const int b = work.b;
    const int rows_b = a.Sq * a.H;
    const int r0 = work.rt * kFRows;
    const int skb = flash_batch_keys(a, b);
    const int k_lo = work.k_lo;
    const int k_end = min(skb, k_lo + work.k_len);
    int k_hi = k_end;
    if (a.causal) k_hi = min(k_hi, skb - a.Sq + min(r0 + kFRows - 1, rows_b - 1) / a.H + 1);
    const int nb = k_hi > k_lo ? (k_hi - k_lo + k2Keys - 1) / k2Keys : 0;

    if (wave < 4) {
        // ================================ score waves
        const int rt = wave >> 1, kh = wave & 1;
        const int rbase = r0 + 32 * rt;
        const int rowS0 = rbase + l16, rowS1 = rbase + 16 + l16;
        int lim0 = k_end - 1, lim1 = k_end - 1;
        if (a.causal) {
            lim0 = min(lim0, skb - a.Sq + min(rowS0, rows_b - 1) / a.H);
            lim1 = min(lim1, skb - a.Sq + min(rowS1, rows_b - 1) / a.H);
        }
        const int lim_wave = __builtin_amdgcn_readfirstlane(lim0);
        const __amdgpu_buffer_rsrc_t rq = make_rsrc(a.qa + (int64_t)b * rows_b * kFR);
        const __amdgpu_buffer_rsrc_t rr = make_rsrc(a.qr + (int64_t)b * rows_b * kFD);
        // Q^T fragments: step s of lane group g is depth 32s + 8g .. +7 (bf16: 16 bytes)
        v4u qf[2][kQSteps];
        #pragma unroll
        for (int t = 0; t < 2; ++t) {
            const int row = t ? rowS1 : rowS0;
            const uint32_t qmask = oob_mask(row, rows_b);
            #pragma unroll
            for (int s = 0; s < kQSteps; ++s)
                qf[t][s] = s < kRSteps
                               ? load16(rq, ((uint32_t)row * kLatBytes + 64u * s + 16u * g) | qmask)
                               : load16(rr, ((uint32_t)row * kPeBytes + 64u * (s - kRSteps) + 16u * g) | qmask);
        }
        wait_vm<0>();   // Q in registers

        // K step s: bytes 32s + 8g of key kk's latent row, i.e. chunk 2s + g/2 at position
        // (2s + g/2) ^ x, x = swz(kk & 15): 32 (s ^ x/2) + 16 (g/2 ^ x%2) + 8 (g%2); the rope
        // steps likewise with y = (kk >> 2) & 3 over 64-byte rows
        const int kk = 16 * kh + l16;
        const int x = swz(kk & 15), y = (kk >> 2) & 3;
        uint32_t kb0 = kk * k8LatBytes + 8u * (g & 1) + 16u * ((g >> 1) ^ (x & 1)) + 32u * (x >> 1);
        uint32_t pb0 = k8LatStage + kk * k8PeBytes + 8u * (g & 1) + 16u * ((g >> 1) ^ (y & 1)) +
                             32u * (y >> 1);
        auto k_read = [&](uint32_t sbase, int s) __attribute__((always_inline)) {
            const uint32_t off = s < kRSteps ? (kb0 ^ (32u * s)) : (pb0 ^ (32u * (s - kRSteps)));
            return *reinterpret_cast<const v2u*>(smem + sbase + off);
        };
        // P^T writes: rows 16h + l16 of the tile, keys 16kh + 4g .. +3 (8 bytes)
        const uint32_t pw0 = kPBase + rt * 32 * kXPPitch + l16 * kXPPitch + 2u * (16 * kh + 4 * g);

        float m_ref[2] = {-INFINITY, -INFINITY}, m_neg[2] = {0.f, 0.f};
        float thr[2] = {-INFINITY, -INFINITY}, l_run[2] = {0.f, 0.f};
        for (int pass = 1;; ++pass) {
            l_run[0] = l_run[1] = 0.f;
            bool overflow = false;
            if (nb == 0) break;
            #pragma unroll 1
            for (int j = 0; j <= nb; ++j) {
                lds_barrier();        // A_j: block j is in LDS, P.V of block j-2 is done
                v4f sc[2];
                if (j < nb) {
                    constexpr int kWin = 4;
                    asm volatile("" : "+v"(kb0), "+v"(pb0));
                    const uint32_t sbase = (uint32_t)(j % k8NS) * k8Stage;
                    v2u kf[kWin];
                    #pragma unroll
                    for (int i = 0; i < kWin; ++i) kf[i] = k_read(sbase, i);
                    // the compiler's own MFMA (not the asm form of the bf16 kernel): the K
                    // operand is written by the conversions just before, a VALU-write ->
                    // MFMA-read dependency whose wait states only the compiler inserts
                    sc[0] = sc[1] = v4f{};
                    #pragma unroll
                    for (int s = 0; s < kQSteps; ++s) {
                        const v4u cur = fp8x8_bf16(kf[s % kWin]);
                        if (s + kWin < kQSteps) kf[s % kWin] = k_read(sbase, s + kWin);
                        #pragma unroll
                        for (int h = 0; h < 2; ++h)
                            sc[h] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(
                                __builtin_bit_cast(v8bf, cur), __builtin_bit_cast(v8bf, qf[h][s]), sc[h],
                                0, 0, 0);
                    }
                    __builtin_amdgcn_sched_barrier(0);
                    const int kq0 = k_lo + k2Keys * j + 16 * kh;
                    if (kq0 + 15 > lim_wave) {
                        const int kq = kq0 + 4 * g;
                        #pragma unroll
                        for (int i = 0; i < 4; ++i) {
                            sc[0][i] = kq + i <= lim0 ? sc[0][i] : -INFINITY;
                            sc[1][i] = kq + i <= lim1 ? sc[1][i] : -INFINITY;
                        }
                    }
                    if (j == 0) {
                        // the pass's reference proposal of each row: the raised one of a
                        // previous pass, else this block's maximum over the half's keys
                        #pragma unroll
                        for (int h = 0; h < 2; ++h) {
                            const float mx = fmaxf(fmaxf(sc[h][0], sc[h][1]), fmaxf(sc[h][2], sc[h][3]));
                            const float bm = row4_reduce(mx, OpMax{}) * a.c;
                            const float prop = m_ref[h] == -INFINITY ? bm : m_ref[h];
                            if (g == 0) xref[(rt * 2 + kh) * 32 + 16 * h + l16] = prop;
                        }
                    }
                }
                if (j == 0) {
                    lds_barrier();    // X: both halves' proposals are in LDS
                    #pragma unroll
                    for (int h = 0; h < 2; ++h) {
                        const int r = 16 * h + l16;
                        const float ref = fmaxf(xref[(rt * 2) * 32 + r], xref[(rt * 2 + 1) * 32 + r]);
                        m_ref[h] = ref;
                        m_neg[h] = ref == -INFINITY ? 0.f : -ref;
                        thr[h] = ref + kHeadroom;
                    }
                }
                if (j < nb) {
                    float mx[2];
                    #pragma unroll
                    for (int h = 0; h < 2; ++h)
                        mx[h] = fmaxf(fmaxf(sc[h][0], sc[h][1]), fmaxf(sc[h][2], sc[h][3]));
                    // a row past its threshold raises its reference and flags a repeat (NaN
                    // scores come here too); rows without a reference have no visible key
                    if (__builtin_amdgcn_ballot_w64(!(mx[0] * a.c <= thr[0]) || !(mx[1] * a.c <= thr[1]))) {
                        #pragma unroll
                        for (int h = 0; h < 2; ++h) {
                            const float bm = row4_reduce(mx[h], OpMax{}) * a.c;
                            const bool over = pass < k2MaxPasses && m_ref[h] != -INFINITY && bm > thr[h];
                            overflow |= __builtin_amdgcn_ballot_w64(over) != 0;
                            if (over) {
                                m_ref[h] = bm;
                                m_neg[h] = -bm;
                                thr[h] = bm + kHeadroom;
                            }
                        }
                    }
                    const uint32_t pws = pw0 + (uint32_t)(j & 1) * kXPStage;
                    #pragma unroll
                    for (int h = 0; h < 2; ++h) {
                        float e[4];
                        #pragma unroll
                        for (int i = 0; i < 4; ++i)
                            e[i] = __builtin_amdgcn_exp2f(__builtin_fmaf(sc[h][i], a.c, m_neg[h]));
                        l_run[h] += (e[0] + e[1]) + (e[2] + e[3]);
                        *reinterpret_cast<v2u*>(smem + pws + 16u * h * kXPPitch) =
                            v2u{Half<TL>::pack2(e[0], e[1]), Half<TL>::pack2(e[2], e[3])};
                    }
                }
            }
            lds_barrier();   // B1: every wave is done with the ring
            if (lane == 0) flags[wave] = overflow ? 1 : 0;
            lds_barrier();   // B2
            const bool again = (flags[0] | flags[1] | flags[2] | flags[3]) != 0;
            lds_barrier();   // B3: the flags are read before they are written again
            if (!again) break;
        }
        // row sums of the half and the shared references for the P.V waves
        #pragma unroll
        for (int h = 0; h < 2; ++h) {
            const float l = row4_reduce(l_run[h], OpSum{});
            if (g == 0) {
                xl[(rt * 2 + kh) * 32 + 16 * h + l16] = l;
                if (kh == 0) xref[(rt * 2) * 32 + 16 * h + l16] = m_ref[h];
            }
        }
        lds_barrier();   // F: sums and references are in LDS
        return;
    }

    // ==================================== P.V waves: columns 128cq .. +127, both row tiles
    const int cq = wave - 4;
    // V^T fragment of key half ks: lane 16G + 2r + h addresses key 16ks + 8(G/2) + r, byte
    // column 16 (G%2) + 8h of the column block, i.e. chunk (2cb + G%2) ^ x at 8h, with
    // x = swz(key & 15): 32 (cb ^ x/2) + 16 (G%2 ^ x%2) + 8h
    uint32_t vb0[2];
    #pragma unroll
    for (int ks = 0; ks < 2; ++ks) {
        const int G = lane >> 4, r = (lane & 15) >> 1, h = lane & 1;
        const int key = 16 * ks + 8 * (G >> 1) + r;
        const int x = swz(key & 15);
        vb0[ks] = key * k8LatBytes + 8u * h + 16u * ((G & 1) ^ (x & 1)) + 32u * (x >> 1);
    }
    typedef __attribute__((address_space(3))) v2i lds_v2i_t;
    auto v_read = [&](uint32_t sbase, int ks, int cb) __attribute__((always_inline)) {
        const v2i r = __builtin_amdgcn_ds_read_tr8_b64_v2i32(
            (lds_v2i_t*)(smem + sbase + (vb0[ks] ^ (32u * cb))));
        return __builtin_bit_cast(v2u, r);
    };
    // P^T of row tile t, key half ks in the B layout: row l32, keys 16ks + 8(l/32) .. +7
    const uint32_t pr0 = kPBase + l32 * kXPPitch + 16u * hw;
    // staging (see above): latent keys 8cq .. 8cq+7; waves 0 and 1 also the rope rows of keys
    // 16cq .. 16cq+15
    const int wv = cq;
    const bool pe_loader = wv < 2;
    const uint32_t lds0 = lds_addr(smem);
    uint32_t lat_voff[4];
    #pragma unroll
    for (int q = 0; q < 4; ++q) {
        const int key = 8 * wv + 2 * q + hw;
        lat_voff[q] = (uint32_t)(2 * q + hw) * k8LatBytes + 16u * ((lane & 31) ^ swz(key & 15));
    }
    const int pkey = 16 * wv + (lane >> 2);
    const uint32_t pe_voff = (uint32_t)(lane >> 2) * k8PeBytes + 16u * ((lane & 3) ^ ((pkey >> 2) & 3));
    const uint64_t ck_base = reinterpret_cast<uint64_t>(a.ckv);
    const uint64_t pe_base = reinterpret_cast<uint64_t>(a.pe);
    const int k_hi_s = __builtin_amdgcn_readfirstlane(k_hi);
    struct Loads { v4i rk, rp; uint32_t st, st_pe; };
    auto loads_of = [&](int j) __attribute__((always_inline)) {
        const uint32_t sb = lds0 + (uint32_t)(j % k8NS) * k8Stage;
        const int kb = __builtin_amdgcn_readfirstlane(k_lo + k2Keys * j + 8 * wv);
        const uint32_t left = (uint32_t)max(0, min(8, k_hi_s - kb));
        Loads d;
        d.st = __builtin_amdgcn_readfirstlane(sb + 8 * wv * k8LatBytes);
        d.rk = rsrc_span(ck_base + (uint64_t)flash_key_row(a, b, kb, k_hi_s) * kFR, 0, left * kFR);
        // (waves 2 and 3 keep a descriptor they never use)
        const int kp = __builtin_amdgcn_readfirstlane(k_lo + k2Keys * j + 16 * (wv & 1));
        const uint32_t left_p = (uint32_t)max(0, min(16, k_hi_s - kp));
        d.st_pe = __builtin_amdgcn_readfirstlane(sb + k8LatStage + 16 * (wv & 1) * k8PeBytes);
        d.rp = rsrc_span(pe_base + (uint64_t)flash_key_row(a, b, kp, k_hi_s) * kFD, 0, left_p * kFD);
        return d;
    };
    auto issue_one = [&](const Loads& d, int q) __attribute__((always_inline)) {
        if (q < 4) dma16(d.rk, d.st + q * 1024, lat_voff[q], 0);
        else dma16(d.rp, d.st_pe, pe_voff, 0);
    };
    // loads per block: 5 for the rope loaders, 4 for the others; wait until at most n
    // blocks' loads are outstanding
    auto issue_block = [&](const Loads& d) __attribute__((always_inline)) {
        #pragma unroll
        for (int q = 0; q < 4; ++q) issue_one(d, q);
        if (pe_loader) issue_one(d, 4);
    };
    auto wait_blocks = [&](auto n_blocks) __attribute__((always_inline)) {
        constexpr int n = decltype(n_blocks)::value;
        if (pe_loader) wait_vm<5 * n>();
        else wait_vm<4 * n>();
    };
    v16f O[8];
    for (int pass = 1;; ++pass) {
        #pragma unroll
        for (int i = 0; i < 8; ++i) O[i] = v16f{};
        if (nb == 0) break;
        #pragma unroll
        for (int j = 0; j < k8Ahead; ++j) issue_block(loads_of(j));
        wait_blocks(std::integral_constant<int, k8Ahead - 1>{});   // block 0 has landed
        lds_barrier();                     // A_0
        issue_block(loads_of(k8Ahead));    // its stage is free from the pass's start
        lds_barrier();                     // X
        #pragma unroll 1
        for (int j = 1; j <= nb; ++j) {
            const Loads next = loads_of(j + k8Ahead);
            // blocks 0 .. j+5 are issued: block j has landed when at most five are in flight
            wait_blocks(std::integral_constant<int, k8Ahead - 1>{});
            lds_barrier();                 // A_j
            {
                asm volatile("" : "+v"(vb0[0]), "+v"(vb0[1]));
                const uint32_t sbase = (uint32_t)((j - 1) % k8NS) * k8Stage;
                const uint32_t prs = pr0 + (uint32_t)((j - 1) & 1) * kXPStage;
                v4u pf[2][2];
                #pragma unroll
                for (int t = 0; t < 2; ++t)
                    #pragma unroll
                    for (int ks = 0; ks < 2; ++ks)
                        pf[t][ks] = *reinterpret_cast<const v4u*>(smem + prs + t * 32 * kXPPitch + 32u * ks);
                // fragment f (one per two MFMAs, t = 2f and 2f + 1 for the two row tiles):
                // key half f/4, column block 4cq + f%4
                constexpr int kVWin = 3;
                v2u vf[kVWin];
                #pragma unroll
                for (int f = 0; f < kVWin; ++f) vf[f] = v_read(sbase, f >> 2, 4 * cq + (f & 3));
                v4u cur;
                #pragma unroll
                for (int t = 0; t < 16; ++t) {
                    const int f = t >> 1;
                    if ((t & 1) == 0) {
                        cur = fp8x8_bf16(vf[f % kVWin]);
                        if (f + kVWin < 8) vf[f % kVWin] = v_read(sbase, (f + kVWin) >> 2, 4 * cq + ((f + kVWin) & 3));
                    }
                    O[t & 7] = mfma32h<TL>(cur, pf[t & 1][f >> 2], O[t & 7]);
                    // block j+6 into stage (j+6) % 8, which block j-2 left at barrier A_j
                    if (t % 3 == 0 && t / 3 < 4) issue_one(next, t / 3);
                    if (t == 13 && pe_loader) issue_one(next, 4);
                }
            }
        }
        wait_vm<0>();    // the zero loads of the blocks past the end have landed
        lds_barrier();   // B1
        lds_barrier();   // B2
        const bool again = (flags[0] | flags[1] | flags[2] | flags[3]) != 0;
        lds_barrier();   // B3
        if (!again) break;
    }
    lds_barrier();       // F
    // both row tiles, columns 128cq .. +127: O[2 cb + t] is column block cb of row tile t; an
    // fp8 cache's values are its codes times kv_scale, so ctx takes the factor here
    #pragma unroll
    for (int t = 0; t < 2; ++t) {
        const int row = r0 + 32 * t + l32;
        if (row >= rows_b) continue;
        const float* xlr = xl + t * 64;
        const float lsum = xlr[l32] + xlr[32 + l32];
        const float M = xref[t * 64 + l32];
        const int64_t slot = (work.direct ? (int64_t)b : work.slot) * rows_b + row;
        if (a.ctx16) {
            const float r = lsum == 0.f ? 0.f : 1.f / lsum;
            uint16_t* crow = static_cast<uint16_t*>(a.ctx16) + slot * kFR + 128 * cq + 4 * hw;
            #pragma unroll
            for (int cb = 0; cb < 4; ++cb)
                #pragma unroll
                for (int q = 0; q < 4; ++q) {
                    const v4f v = v4f{O[2 * cb + t][4 * q], O[2 * cb + t][4 * q + 1],
                                      O[2 * cb + t][4 * q + 2], O[2 * cb + t][4 * q + 3]} * a.o_scale;
                    const v4f w = v * r;
                    *reinterpret_cast<v2u*>(crow + 32 * cb + 8 * q) =
                        v2u{Half<bf16_t>::pack2(w[0], w[1]), Half<bf16_t>::pack2(w[2], w[3])};
                }
            continue;
        }
        if (cq == 0 && hw == 0) {
            if (!work.direct) a.m[slot] = M;
            (work.direct ? a.l_direct : a.l)[slot] = lsum;
        }
        float* orow = (work.direct ? a.o_direct : a.o) + slot * kFR + 128 * cq + 4 * hw;
        #pragma unroll
        for (int cb = 0; cb < 4; ++cb)
            #pragma unroll
            for (int q = 0; q < 4; ++q)
                *reinterpret_cast<v4f*>(orow + 32 * cb + 8 * q) =
                    v4f{O[2 * cb + t][4 * q], O[2 * cb + t][4 * q + 1], O[2 * cb + t][4 * q + 2],
                        O[2 * cb + t][4 * q + 3]} * a.o_scale;
    }
}

// ------------------------------------------------------------------ fp32 variant
// Same pass with fp32 storage on the 16x16x4 fp32 MFMA (lane l supplies A[l%16][l/16] and
// B[l/16][l%16]; accumulator element i of lane l is D[4(l/16) + i][l%16]).  A 16-key block
// is 272 MFMAs of 32 cycles per wave, and a SIMD runs fp32 MFMAs and VALU instructions one
// after the other (they do not overlap, and every switch between the two costs a drain of
// the MFMA pipeline), so the kernel keeps VALU work per block to a few dozen instructions:
//   S^T[16 keys x 16 rows]: lane group g reads the depth quarter [128g, 128g + 128) of the
//     latent row in 16-byte chunks (4 depths per read feed 4 MFMAs) and the rope depths
//     [16g, 16g + 16); the wave's Q^T lives in 144 VGPRs
//   P^T: element i of lane l is key 4(l/16) + i of row l%16 -- the B operand of K step i
//   O^T[512 x 16]: 32 accumulator blocks; block (mh, r) holds columns 32mh + 2j + r, so a
//     64-bit read of V gives two blocks' A operands
//   exponentials against a fixed per-row reference (k32Headroom): no O rescaling, no row
//     reductions per block
//   cache loads: the buffer descriptor is rebased on each block's first key in scalar
//     registers and its range ends at the split's last key, so out-of-range keys read as
//     zeros with no per-lane address work
// LDS per stage: the rope rows of the NS stages first (16 x 256 B each, chunk c of key k at
// c ^ swz(k & 15)), then the latent rows (16 keys x 2 KB at a pitch of 2064 bytes).  The K
// reads (16 keys at one offset) and the 64-bit V reads (4 keys x 16 consecutive column
// pairs) are free of bank conflicts (measured), and every LDS read is a per-lane base plus
// an immediate offset: stages 0-1 and 2-3 of the latent region each have their own base.
constexpr int k32Keys = 16;
constexpr int k32Pitch = kFR * 4 + 16;
constexpr int k32PeBytes = kFD * 4;
constexpr int k32PeStage = k32Keys * k32PeBytes;     // 4 KB
constexpr int k32LatStage = k32Keys * k32Pitch;      // 33024 B
constexpr int k32StageBytes = k32PeStage + k32LatStage;
constexpr int k32LatReads = kFR / 16;               // 32: 16-byte K reads per lane, latent
constexpr int k32PeReads = kFD / 16;                // 4: rope
constexpr int k32Loads = 9;                         // cache loads per wave and block

__device__ __forceinline__ v4f mfma16f(float a, float b, v4f c) {
    return __builtin_amdgcn_mfma_f32_16x16x4f32(a, b, c, 0, 0, 0);
}

// Reference point of a row's exponentials in the fp32 pass: p = 2^(s*c - m_ref) with m_ref
// the first visible block's maximum, kept while the row's maximum stays below
// m_ref + k32Headroom.  P then stays below 2^64, the row sum below 2^64 times the key count,
// and O needs no rescaling (a rescale of the 128 accumulator registers costs more in the
// compiler's register assignment for every block than the multiplies themselves).  A row
// that outgrows its reference restarts the workgroup's pass with the larger reference.
constexpr float k32Headroom = 64.f;
constexpr int k32MaxPasses = 8;

template <int NS>
__global__ void __launch_bounds__(kFThreads, 1) flash32_kernel(FlashArgs a) {
    static_assert(NS == 4, "two latent bases cover stages 0-1 and 2-3");
    __shared__ __attribute__((aligned(1024))) uint8_t smem[NS * k32StageBytes];
    __shared__ int restart[2];   // [block parity]: some row outgrew its reference
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int l16 = lane & 15, g = lane >> 4;
    if (tid < 2) restart[tid] = 0;   // read only after the first block's barrier
    const float* qa = reinterpret_cast<const float*>(a.qa);
    const float* qr = reinterpret_cast<const float*>(a.qr);

    const FlashWork work = flash_work(a);
    if (work.skip) return;   // the whole workgroup leaves (restart[] is not read before a barrier)

    const int rt = work.rt;
    const int b = work.b;
    const int rows_b = a.Sq * a.H;
    const int r0 = rt * kFRows;
    const int row = r0 + 16 * wave + l16;

    const int skb = flash_batch_keys(a, b);
    const int k_lo = work.k_lo;
    int k_hi = min(skb, k_lo + work.k_len);
    int lim = k_hi - 1;
    if (a.causal) {
        lim = min(lim, skb - a.Sq + min(row, rows_b - 1) / a.H);
        k_hi = min(k_hi, skb - a.Sq + min(r0 + kFRows - 1, rows_b - 1) / a.H + 1);
    }
    const int nb = k_hi > k_lo ? (k_hi - k_lo + k32Keys - 1) / k32Keys : 0;
    const int lim_wave = __builtin_amdgcn_readfirstlane(lim);
    const int k_hi_s = __builtin_amdgcn_readfirstlane(k_hi);

    // ---- Q^T: read r of lane group g is depths 128g + 4r .. +3 (latent), 16g + 4r' (rope)
    const __amdgpu_buffer_rsrc_t rq = make_rsrc(qa + (int64_t)b * rows_b * kFR);
    const __amdgpu_buffer_rsrc_t rr = make_rsrc(qr + (int64_t)b * rows_b * kFD);
    const uint32_t qmask = oob_mask(row, rows_b);
    v4u qf[k32LatReads + k32PeReads];
    #pragma unroll
    for (int r = 0; r < k32LatReads; ++r)
        qf[r] = load16(rq, ((uint32_t)row * (kFR * 4) + 512u * g + 16u * r) | qmask);
    #pragma unroll
    for (int r = 0; r < k32PeReads; ++r)
        qf[k32LatReads + r] = load16(rr, ((uint32_t)row * k32PeBytes + 64u * g + 16u * r) | qmask);
    wait_vm<0>();   // Q is in registers before the first cache load (see flash16_kernel)

    // ---- direct global->LDS staging: wave w loads keys 4w .. 4w+3 of a block
    const uint64_t ck_base = reinterpret_cast<uint64_t>(a.ckv);
    const uint64_t pe_base = reinterpret_cast<uint64_t>(a.pe);
    const uint32_t lds0 = lds_addr(smem);
    // latent: instruction q fills half q%2 of key q/2's row; rope (one instruction for the
    // 4 keys): lane i fills chunk i%16 of key 4w + i/16, i.e. loads its logical chunk
    // (i%16) ^ swz(key & 15)
    uint32_t lat_lane[4];
    #pragma unroll
    for (int k = 0; k < 4; ++k) lat_lane[k] = 16u * lane + (uint32_t)k * (kFR * 4);
    const uint32_t pe_lane = (uint32_t)(lane >> 4) * k32PeBytes +
                             16u * ((lane & 15) ^ swz((4 * wave + (lane >> 4)) & 15));
    auto issue = [&](int j, int stage) __attribute__((always_inline)) {
        const int kb = __builtin_amdgcn_readfirstlane(k_lo + k32Keys * j + 4 * wave);
        const uint32_t left = (uint32_t)max(0, k_hi_s - kb);   // keys of this wave in range
        // the wave's 4 keys are consecutive cache rows (one page)
        const uint64_t row0 = (uint64_t)flash_key_row(a, b, kb, k_hi_s);
        const v4i rk = rsrc_span(ck_base + row0 * (kFR * 4), 0, min(left, 4u) * (kFR * 4));
        const v4i rp = rsrc_span(pe_base + row0 * k32PeBytes, 0, min(left, 4u) * k32PeBytes);
        const uint32_t st = __builtin_amdgcn_readfirstlane(
            lds0 + NS * k32PeStage + stage * k32LatStage + 4 * wave * k32Pitch);
        const uint32_t st_pe = __builtin_amdgcn_readfirstlane(
            lds0 + stage * k32PeStage + 4 * wave * k32PeBytes);
        #pragma unroll
        for (int k = 0; k < 4; ++k) {
            dma16_imm<0>(rk, st + k * k32Pitch, lat_lane[k]);
            dma16_imm<1024>(rk, st + k * k32Pitch, lat_lane[k]);   // second KB of the row
        }
        dma16_imm<0>(rp, st_pe, pe_lane);
    };

    // ---- per-lane LDS bases (byte offsets from smem)
    // (the asm statements hide that the second base is the first plus a constant, which
    // the compiler would otherwise add back per read: the sum exceeds the 16-bit offset)
    const uint32_t lat0 = NS * k32PeStage;
    uint32_t k_base[2] = {lat0 + l16 * k32Pitch + 512u * g,
                          lat0 + 2 * k32LatStage + l16 * k32Pitch + 512u * g};
    uint32_t v_base[2] = {lat0 + 4 * g * k32Pitch + 8u * l16,
                          lat0 + 2 * k32LatStage + 4 * g * k32Pitch + 8u * l16};
    asm volatile("" : "+v"(k_base[1]), "+v"(v_base[1]));
    uint32_t p_off[k32PeReads];
    #pragma unroll
    for (int r = 0; r < k32PeReads; ++r)
        p_off[r] = l16 * k32PeBytes + 16u * ((4 * g + r) ^ swz(l16));

    v4f O[2 * 16];   // [mh][r]
    float m_ref = -INFINITY, m_neg = 0.f, thr = -INFINITY, l_run = 0.f;
    int pass = 1;

    typedef uint32_t v2u __attribute__((ext_vector_type(2)));
    auto k_read = [&](auto st_tag, int r) __attribute__((always_inline)) {
        constexpr int ST = decltype(st_tag)::value;
        const uint32_t off = r < k32LatReads
                                 ? k_base[ST >> 1] + (ST & 1) * k32LatStage + 16u * r
                                 : p_off[r - k32LatReads] + ST * k32PeStage;
        return *reinterpret_cast<const v4u*>(smem + off);
    };
    // V read t: K step i = t / 16 (keys 4g + i), column pair 32mh + 2*l16 with mh = t % 16
    auto v_read = [&](auto st_tag, int t) __attribute__((always_inline)) {
        constexpr int ST = decltype(st_tag)::value;
        return *reinterpret_cast<const v2u*>(smem + v_base[ST >> 1] + (ST & 1) * k32LatStage +
                                             (t >> 4) * k32Pitch + 128u * (t & 15));
    };

    // One block; returns true (before any work) when a row asked for a restart in block j-1.
    auto step = [&](int j, auto st_tag) __attribute__((always_inline)) {
        constexpr int ST = decltype(st_tag)::value;
        constexpr int KW = 4;    // K reads in flight ahead of the MFMAs that use them
        constexpr int VW = 8;    // V reads in flight
        constexpr int KR = k32LatReads + k32PeReads;
        const int ahead = min(nb - 1, j + NS - 2) - j;   // blocks issued after block j
        if (ahead >= 2) wait_vm<2 * k32Loads>();
        else if (ahead == 1) wait_vm<k32Loads>();
        else wait_vm<0>();
        lds_barrier();   // block j is in LDS for every wave; every wave is past block j-1
        if (j > 0 && __builtin_amdgcn_readfirstlane(restart[(j - 1) & 1])) return true;
        if (j + NS - 1 < nb) issue(j + NS - 1, (ST + NS - 1) % NS);

        // S^T: 36 16-byte K reads per lane, 4 MFMAs each, alternating two accumulators
        v4u kq[KW];
        #pragma unroll
        for (int r = 0; r < KW; ++r) kq[r] = k_read(st_tag, r);
        v4f s2[2] = {v4f{}, v4f{}};
        #pragma unroll
        for (int r = 0; r < KR; ++r) {
            const v4u cur = kq[r % KW];
            if (r + KW < KR) kq[r % KW] = k_read(st_tag, r + KW);
            #pragma unroll
            for (int q = 0; q < 4; ++q)
                s2[q & 1] = mfma16f(__uint_as_float(cur[q]), __uint_as_float(qf[r][q]), s2[q & 1]);
        }
        // the first V reads of the P.V pass go out under the last score MFMAs
        v2u vq[VW];
        #pragma unroll
        for (int t = 0; t < VW; ++t) vq[t] = v_read(st_tag, t);
        __builtin_amdgcn_sched_group_barrier(kSgDsRd, KW, 0);
        #pragma unroll
        for (int r = 0; r < KR - KW; ++r) {
            __builtin_amdgcn_sched_group_barrier(kSgMfma, 4, 0);
            __builtin_amdgcn_sched_group_barrier(kSgDsRd, 1, 0);
        }
        #pragma unroll
        for (int r = 0; r < KW; ++r) {
            __builtin_amdgcn_sched_group_barrier(kSgMfma, 4, 0);
            __builtin_amdgcn_sched_group_barrier(kSgDsRd, VW / KW, 0);
        }
        __builtin_amdgcn_sched_barrier(0);
        v4f sc = s2[0] + s2[1];

        // softmax numerators: element i of lane l is key kb + 4g + i of row l%16
        const int kb = k_lo + k32Keys * j;
        if (kb + k32Keys - 1 > lim_wave) {
            #pragma unroll
            for (int i = 0; i < 4; ++i) sc[i] = kb + 4 * g + i <= lim ? sc[i] : -INFINITY;
        }
        const float smax = fmaxf(fmaxf(sc[0], sc[1]), fmaxf(sc[2], sc[3]));
        // a row's first visible keys set its reference (O is still zero for it); a row
        // whose maximum passes reference + headroom asks for a restart (rows are uniform
        // over their 4 lanes after the reduction, and NaN scores take this path too)
        if (__builtin_amdgcn_ballot_w64(!(smax * a.c <= thr))) {
            const float bm = row4_reduce(smax, OpMax{}) * a.c;
            const bool over = pass < k32MaxPasses && m_ref != -INFINITY && bm > thr;
            if (__builtin_amdgcn_ballot_w64(over) && lane == 0) restart[j & 1] = 1;
            if (m_ref == -INFINITY || over) {
                m_ref = bm;
                m_neg = bm == -INFINITY ? 0.f : -bm;
                thr = bm + k32Headroom;
            }
        }
        float p[4];
        #pragma unroll
        for (int i = 0; i < 4; ++i) p[i] = __builtin_amdgcn_exp2f(__builtin_fmaf(sc[i], a.c, m_neg));
        l_run += (p[0] + p[1]) + (p[2] + p[3]);
        __builtin_amdgcn_sched_barrier(0);   // all VALU work of the block before its P.V

        // O^T += V^T . P^T: K step i (keys 4g + i) is 16 64-bit V reads x 2 MFMAs
        #pragma unroll
        for (int t = 0; t < 64; ++t) {
            const v2u cur = vq[t % VW];
            if (t + VW < 64) vq[t % VW] = v_read(st_tag, t + VW);
            const int mh = t & 15, i = t >> 4;
            O[2 * mh] = mfma16f(__uint_as_float(cur[0]), p[i], O[2 * mh]);
            O[2 * mh + 1] = mfma16f(__uint_as_float(cur[1]), p[i], O[2 * mh + 1]);
        }
        #pragma unroll
        for (int t = 0; t < 64 - VW; ++t) {
            __builtin_amdgcn_sched_group_barrier(kSgMfma, 2, 0);
            __builtin_amdgcn_sched_group_barrier(kSgDsRd, 1, 0);
        }
        __builtin_amdgcn_sched_group_barrier(kSgMfma, 2 * VW, 0);
        __builtin_amdgcn_sched_barrier(0);
        return false;
    };

    // A pass over the split's keys; repeated (from the first key, every wave) only when a
    // row's maximum outgrew its reference point.  Each repeat raises that row's reference by
    // more than k32Headroom; after k32MaxPasses passes the last one stands (exponents past
    // 2^128 then overflow to inf, as a plain softmax without the max subtraction would).
    for (;; ++pass) {
        #pragma unroll
        for (int i = 0; i < 32; ++i) O[i] = v4f{};
        l_run = 0.f;
        #pragma unroll
        for (int j = 0; j < NS - 1; ++j)
            if (j < nb) issue(j, j);
        bool again = false;
        for (int j0 = 0; j0 < nb && !again; j0 += NS) {
            again = step(j0, std::integral_constant<int, 0>{});
            if (!again && j0 + 1 < nb) again = step(j0 + 1, std::integral_constant<int, 1>{});
            if (!again && j0 + 2 < nb) again = step(j0 + 2, std::integral_constant<int, 2>{});
            if (!again && j0 + 3 < nb) again = step(j0 + 3, std::integral_constant<int, 3>{});
        }
        if (nb == 0) break;
        if (!again) {   // the last block's request
            lds_barrier();
            again = __builtin_amdgcn_readfirstlane(restart[(nb - 1) & 1]) != 0;
            if (!again) break;
        }
        wait_vm<0>();    // no cache load still writes the ring
        lds_barrier();   // every wave has read the request
        if (tid < 2) restart[tid] = 0;
        lds_barrier();
    }

    // ---- partial state: lane l holds row l%16, columns 32mh + 8g + 2i + r of O[mh][r][i]
    l_run = row4_reduce(l_run, OpSum{});
    if (row < rows_b) {
        const int64_t slot = (work.direct ? (int64_t)b : work.slot) * rows_b + row;
        if (g == 0) {
            if (!work.direct) a.m[slot] = m_ref;
            (work.direct ? a.l_direct : a.l)[slot] = l_run;
        }
        float* orow = (work.direct ? a.o_direct : a.o) + slot * kFR;
        #pragma unroll
        for (int mh = 0; mh < 16; ++mh) {
            const v4f lo = {O[2 * mh][0], O[2 * mh + 1][0], O[2 * mh][1], O[2 * mh + 1][1]};
            const v4f hi = {O[2 * mh][2], O[2 * mh + 1][2], O[2 * mh][3], O[2 * mh + 1][3]};
            *reinterpret_cast<v4f*>(orow + 32 * mh + 8 * g) = lo;
            *reinterpret_cast<v4f*>(orow + 32 * mh + 8 * g + 4) = hi;
        }
    }
}

// ------------------------------------------------------------------ fp32: specialised waves
// flash32_kernel's 64-row tile, 16-key blocks, LDS ring and softmax on eight waves split by
// kind, two per SIMD, so that one wave's MFMAs run while the other waits on LDS, on the
// barrier or on its softmax:
//   score wave w (rows 16w .. 16w+15): Q^T in 144 VGPRs, the K reads, the 144 score MFMAs
//     and the softmax (reference, threshold and repeat flag as in flash32_kernel); it
//     writes P^T in its accumulator layout (element i of lane l is key 4(l/16) + i of row
//     l%16) to its pair's 1 KB slot of P stage j & 1;
//   P.V wave 4 + w (the same rows): O^T in 128 VGPRs, one block behind: in step j it reads
//     block j-1's P^T slot, whose lane layout is its B operand, and runs the 128 P.V MFMAs
//     over block j-1's V^T; it also issues the staging loads (block j+2 in step j, spread
//     over its MFMAs) and waits for block j before the step's barrier.
// A wave pair owns its 16 rows whole, so no reference crosses waves.  One barrier per step
// orders the ring (K of block j, V of block j-1, block j+2 loading into the stage block
// j-2 left) and the P stages.  A pass runs to its end; a repeat is decided from the score
// waves' flags after it.  The P.V loop starts at block 1 (block 0's step only has its
// barrier), so the accumulators meet no branch inside the loop.
constexpr int k32XPStage = 4 * 1024;      // P^T slots of the four wave pairs

template <int NS>
__global__ void __launch_bounds__(kXThreads, 1) flash32x_kernel(FlashArgs a) {
    static_assert(NS == 4, "the ring keeps block j-1 (V), block j (K) and two in flight");
    constexpr int kPBase = NS * k32StageBytes;
    constexpr int kXBase = kPBase + 2 * k32XPStage;
    __shared__ __attribute__((aligned(1024))) uint8_t smem[kXBase + 2 * 64 * 4 + 16];
    float* xm = reinterpret_cast<float*>(smem + kXBase);   // [64 rows] references
    float* xl = xm + 64;                                   // [64 rows] row sums
    int* flags = reinterpret_cast<int*>(xl + 64);          // [score wave]
    const int tid = threadIdx.x, lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int pw = wave & 3;                               // the wave pair
    const int l16 = lane & 15, g = lane >> 4;
    const FlashWork work = flash_work(a);
    if (work.skip) return;   // past the end of a work list: the whole workgroup leaves

    const int b = work.b;
    const int rows_b = a.Sq * a.H;
    const int r0 = work.rt * kFRows;
    const int row = r0 + 16 * pw + l16;
    const int skb = flash_batch_keys(a, b);
    const int k_lo = work.k_lo;
    int k_hi = min(skb, k_lo + work.k_len);
    int lim = k_hi - 1;
    if (a.causal) {
        lim = min(lim, skb - a.Sq + min(row, rows_b - 1) / a.H);
        k_hi = min(k_hi, skb - a.Sq + min(r0 + kFRows - 1, rows_b - 1) / a.H + 1);
    }
    const int nb = k_hi > k_lo ? (k_hi - k_lo + k32Keys - 1) / k32Keys : 0;
    const uint32_t lat0 = NS * k32PeStage;
    const uint32_t pslot = kPBase + pw * 1024 + 16u * lane;   // + stage * k32XPStage

    if (wave < 4) {
        // ================================ score waves
        const int lim_wave = __builtin_amdgcn_readfirstlane(lim);
        const float* qa = reinterpret_cast<const float*>(a.qa);
        const float* qr = reinterpret_cast<const float*>(a.qr);
        const __amdgpu_buffer_rsrc_t rq = make_rsrc(qa + (int64_t)b * rows_b * kFR);
        const __amdgpu_buffer_rsrc_t rr = make_rsrc(qr + (int64_t)b * rows_b * kFD);
        const uint32_t qmask = oob_mask(row, rows_b);
        v4u qf[k32LatReads + k32PeReads];
        #pragma unroll
        for (int r = 0; r < k32LatReads; ++r)
            qf[r] = load16(rq, ((uint32_t)row * (kFR * 4) + 512u * g + 16u * r) | qmask);
        #pragma unroll
        for (int r = 0; r < k32PeReads; ++r)
            qf[k32LatReads + r] = load16(rr, ((uint32_t)row * k32PeBytes + 64u * g + 16u * r) | qmask);
        wait_vm<0>();   // Q in registers

        uint32_t k_base = lat0 + l16 * k32Pitch + 512u * g;   // + stage * k32LatStage
        uint32_t p_off[k32PeReads];
        #pragma unroll
        for (int r = 0; r < k32PeReads; ++r)
            p_off[r] = l16 * k32PeBytes + 16u * ((4 * g + r) ^ swz(l16));
        float m_ref = -INFINITY, m_neg = 0.f, thr = -INFINITY, l_run = 0.f;
        for (int pass = 1;; ++pass) {
            l_run = 0.f;
            bool overflow = false;
            if (nb == 0) break;
            #pragma unroll 1
            for (int j = 0; j <= nb; ++j) {
                lds_barrier();        // A_j: block j is in LDS, P.V of block j-2 is done
                if (j < nb) {
                    constexpr int KW = 4;
                    constexpr int KR = k32LatReads + k32PeReads;
                    asm volatile("" : "+v"(k_base));
                    const int st = j % NS;
                    const uint32_t kbs = k_base + (uint32_t)st * k32LatStage;
                    const uint32_t pbs = (uint32_t)st * k32PeStage;
                    auto k_read = [&](int r) __attribute__((always_inline)) {
                        const uint32_t off = r < k32LatReads ? kbs + 16u * r : p_off[r - k32LatReads] + pbs;
                        return *reinterpret_cast<const v4u*>(smem + off);
                    };
                    v4u kq[KW];
                    #pragma unroll
                    for (int r = 0; r < KW; ++r) kq[r] = k_read(r);
                    v4f s2[2] = {v4f{}, v4f{}};
                    #pragma unroll
                    for (int r = 0; r < KR; ++r) {
                        const v4u cur = kq[r % KW];
                        if (r + KW < KR) kq[r % KW] = k_read(r + KW);
                        #pragma unroll
                        for (int q = 0; q < 4; ++q)
                            s2[q & 1] = mfma16f(__uint_as_float(cur[q]), __uint_as_float(qf[r][q]), s2[q & 1]);
                    }
                    __builtin_amdgcn_sched_group_barrier(kSgDsRd, KW, 0);
                    #pragma unroll
                    for (int r = 0; r < KR - KW; ++r) {
                        __builtin_amdgcn_sched_group_barrier(kSgMfma, 4, 0);
                        __builtin_amdgcn_sched_group_barrier(kSgDsRd, 1, 0);
                    }
                    __builtin_amdgcn_sched_group_barrier(kSgMfma, 4 * KW, 0);
                    __builtin_amdgcn_sched_barrier(0);
                    v4f sc = s2[0] + s2[1];
                    // element i of lane l is key kb + 4g + i of row l%16
                    const int kb = k_lo + k32Keys * j;
                    if (kb + k32Keys - 1 > lim_wave) {
                        #pragma unroll
                        for (int i = 0; i < 4; ++i) sc[i] = kb + 4 * g + i <= lim ? sc[i] : -INFINITY;
                    }
                    const float smax = fmaxf(fmaxf(sc[0], sc[1]), fmaxf(sc[2], sc[3]));
                    // a row's first visible keys set its reference (O is still zero for it);
                    // a row whose maximum passes reference + headroom flags a repeat (rows
                    // are uniform over their 4 lanes after the reduction; NaN scores take
                    // this path too)
                    if (__builtin_amdgcn_ballot_w64(!(smax * a.c <= thr))) {
                        const float bm = row4_reduce(smax, OpMax{}) * a.c;
                        const bool over = pass < k32MaxPasses && m_ref != -INFINITY && bm > thr;
                        overflow |= __builtin_amdgcn_ballot_w64(over) != 0;
                        if (m_ref == -INFINITY || over) {
                            m_ref = bm;
                            m_neg = bm == -INFINITY ? 0.f : -bm;
                            thr = bm + k32Headroom;
                        }
                    }
                    v4f p;
                    #pragma unroll
                    for (int i = 0; i < 4; ++i) p[i] = __builtin_amdgcn_exp2f(__builtin_fmaf(sc[i], a.c, m_neg));
                    l_run += (p[0] + p[1]) + (p[2] + p[3]);
                    *reinterpret_cast<v4f*>(smem + pslot + (uint32_t)(j & 1) * k32XPStage) = p;
                }
            }
            lds_barrier();   // B1: every wave is done with the ring
            if (lane == 0) flags[wave] = overflow ? 1 : 0;
            lds_barrier();   // B2
            const bool again = (flags[0] | flags[1] | flags[2] | flags[3]) != 0;
            lds_barrier();   // B3: the flags are read before they are written again
            if (!again) break;
        }
        l_run = row4_reduce(l_run, OpSum{});
        if (g == 0) {
            xm[16 * pw + l16] = m_ref;
            xl[16 * pw + l16] = l_run;
        }
        lds_barrier();   // F: references and row sums are in LDS
        return;
    }

    // ==================================== P.V waves
    // staging: P.V wave 4 + w loads keys 4w .. 4w+3 of a block (flash32_kernel's layout),
    // block j+2 during step j; blocks past the end load zeros
    const uint64_t ck_base = reinterpret_cast<uint64_t>(a.ckv);
    const uint64_t pe_base = reinterpret_cast<uint64_t>(a.pe);
    const uint32_t lds0 = lds_addr(smem);
    const int k_hi_s = __builtin_amdgcn_readfirstlane(k_hi);
    uint32_t lat_lane[4];
    #pragma unroll
    for (int k = 0; k < 4; ++k) lat_lane[k] = 16u * lane + (uint32_t)k * (kFR * 4);
    const uint32_t pe_lane = (uint32_t)(lane >> 4) * k32PeBytes +
                             16u * ((lane & 15) ^ swz((4 * pw + (lane >> 4)) & 15));
    struct Loads { v4i rk, rp; uint32_t st, st_pe; };
    auto loads_of = [&](int j) __attribute__((always_inline)) {
        const int stage = j % NS;
        const int kb = __builtin_amdgcn_readfirstlane(k_lo + k32Keys * j + 4 * pw);
        const uint32_t left = (uint32_t)max(0, min(4, k_hi_s - kb));
        const uint64_t row0 = (uint64_t)flash_key_row(a, b, kb, k_hi_s);
        Loads d;
        d.rk = rsrc_span(ck_base + row0 * (kFR * 4), 0, left * (kFR * 4));
        d.rp = rsrc_span(pe_base + row0 * k32PeBytes, 0, left * k32PeBytes);
        d.st = __builtin_amdgcn_readfirstlane(lds0 + NS * k32PeStage + stage * k32LatStage + 4 * pw * k32Pitch);
        d.st_pe = __builtin_amdgcn_readfirstlane(lds0 + stage * k32PeStage + 4 * pw * k32PeBytes);
        return d;
    };
    // load q < 8: half q % 2 of key q / 2's latent row; load 8: the four keys' rope rows
    auto issue_one = [&](const Loads& d, int q) __attribute__((always_inline)) {
        if (q < 8) {
            if (q & 1) dma16_imm<1024>(d.rk, d.st + (q >> 1) * k32Pitch, lat_lane[q >> 1]);
            else dma16_imm<0>(d.rk, d.st + (q >> 1) * k32Pitch, lat_lane[q >> 1]);
        } else {
            dma16_imm<0>(d.rp, d.st_pe, pe_lane);
        }
    };
    uint32_t v_base = lat0 + 4 * g * k32Pitch + 8u * l16;   // + stage * k32LatStage
    typedef uint32_t v2u __attribute__((ext_vector_type(2)));
    v4f O[2 * 16];   // [mh][r]
    for (int pass = 1;; ++pass) {
        #pragma unroll
        for (int i = 0; i < 32; ++i) O[i] = v4f{};
        if (nb == 0) break;
        #pragma unroll
        for (int j = 0; j < 2; ++j) {
            const Loads d = loads_of(j);
            #pragma unroll
            for (int q = 0; q < k32Loads; ++q) issue_one(d, q);
        }
        wait_vm<k32Loads>();               // block 0 has landed; block 1 may be in flight
        lds_barrier();                     // A_0
        {
            const Loads d = loads_of(2);   // stage 2 is free from the pass's start
            #pragma unroll
            for (int q = 0; q < k32Loads; ++q) issue_one(d, q);
        }
        #pragma unroll 1
        for (int j = 1; j <= nb; ++j) {
            const Loads next = loads_of(j + 2);
            wait_vm<k32Loads>();           // block j has landed; block j+1 may be in flight
            lds_barrier();                 // A_j: block j-1's P^T is in its slot
            // Wave priority: the first 96 of the step's 128 MFMAs go ahead of the score
            // wave's on the SIMD, the last 32 behind them, so they run under the score
            // wave's softmax and P^T write.  cfg2, the same bits: equal priorities 1,331-1,342
            // us, priority 1 for the whole step 1,280-1,293 us, this 1,259-1,270 us.  (The
            // 16-bit passes measured 5-8% slower with their P.V waves first, so they keep
            // equal priorities.)
            __builtin_amdgcn_s_setprio(1);
            constexpr int VW = 8;          // V reads in flight
            asm volatile("" : "+v"(v_base));
            const uint32_t vbs = v_base + (uint32_t)((j - 1) % NS) * k32LatStage;
            // V read t: K step i = t / 16 (keys 4g + i), column pair 32mh + 2*l16, mh = t % 16
            auto v_read = [&](int t) __attribute__((always_inline)) {
                return *reinterpret_cast<const v2u*>(smem + vbs + (t >> 4) * k32Pitch + 128u * (t & 15));
            };
            v2u vq[VW];
            #pragma unroll
            for (int t = 0; t < VW; ++t) vq[t] = v_read(t);
            const v4f p = *reinterpret_cast<const v4f*>(smem + pslot + (uint32_t)((j - 1) & 1) * k32XPStage);
            #pragma unroll
            for (int t = 0; t < 64; ++t) {
                const v2u cur = vq[t % VW];
                if (t + VW < 64) vq[t % VW] = v_read(t + VW);
                const int mh = t & 15, i = t >> 4;
                O[2 * mh] = mfma16f(__uint_as_float(cur[0]), p[i], O[2 * mh]);
                O[2 * mh + 1] = mfma16f(__uint_as_float(cur[1]), p[i], O[2 * mh + 1]);
                // block j+2 into stage (j+2) % 4, which block j-2 left at barrier A_j
                if (t % 7 == 3 && t / 7 < k32Loads) issue_one(next, t / 7);
                if (t == 47) __builtin_amdgcn_s_setprio(0);
            }
        }
        wait_vm<0>();    // the zero loads of the blocks past the end have landed
        lds_barrier();   // B1
        lds_barrier();   // B2
        const bool again = (flags[0] | flags[1] | flags[2] | flags[3]) != 0;
        lds_barrier();   // B3
        if (!again) break;
    }
    lds_barrier();       // F
    // ---- partial state: lane l holds row l%16, columns 32mh + 8g + 2i + r of O[mh][r][i]
    if (row < rows_b) {
        const int64_t slot = (work.direct ? (int64_t)b : work.slot) * rows_b + row;
        if (g == 0) {
            if (!work.direct) a.m[slot] = xm[16 * pw + l16];
            (work.direct ? a.l_direct : a.l)[slot] = xl[16 * pw + l16];
        }
        float* orow = (work.direct ? a.o_direct : a.o) + slot * kFR;
        #pragma unroll
        for (int mh = 0; mh < 16; ++mh) {
            const v4f lo = {O[2 * mh][0], O[2 * mh + 1][0], O[2 * mh][1], O[2 * mh + 1][1]};
            const v4f hi = {O[2 * mh][2], O[2 * mh + 1][2], O[2 * mh][3], O[2 * mh + 1][3]};
            *reinterpret_cast<v4f*>(orow + 32 * mh + 8 * g) = lo;
            *reinterpret_cast<v4f*>(orow + 32 * mh + 8 * g + 4) = hi;
        }
    }
}

// ------------------------------------------------------------------ fp32: key-split waves
// The fp32 pass for batches too small to fill the chip with flash32_kernel's 64-row
// workgroups.  Those need many key splits there, and their split partials outgrow the
// cache (B=1, Sk=4989: 104 splits of 48 keys write 27 MB of partials, merged by a second
// kernel, for an 11.5 MB cache).  Here a workgroup is 16 rows and its four waves split the
// workgroup's keys (wave w: the w-th quarter of its 16-key blocks), so the same number of
// workgroups needs a quarter of the splits.  Each wave runs on its own until its keys are
// done: no LDS ring and no barrier in the loop, the cache read straight into registers.
// At fp32 a block's MFMA work (144 + 128 16x16x4 MFMAs, ~8,700 cycles per wave) is long
// against its 68 16-byte loads per lane (the 16 keys' K rows and V^T fragments, mostly L2
// hits: the row tiles of one split are neighbours on one XCD), so 17 loads in flight hide
// the latency.
//   S^T[16 keys x 16 rows] = K . Q^T: load r < 32 of lane (l16, g) is key l16's latent
//     floats 16r + 4g .. +3 (4 MFMAs, one per float), loads 32..35 its rope floats 16r' +
//     4g .. +3; the Q^T fragment of step r is the same depths of row l16, read from the
//     workgroup's copy of its 16 query rows in LDS (the four waves share the rows), so the
//     MFMAs sum the same products as a plain dot product.  Accumulator element v of lane l
//     is key 4g + v of row l16.
//   softmax as in flash32_kernel (fixed reference, 2^64 headroom); a wave whose row
//     outgrows its reference repeats its own keys, the other waves are not involved
//   O^T[512 x 16 rows] += V^T . P^T: load 36 + 8i + c is key 4g + i's columns 64c + 4 l16
//     .. +3, four MFMAs with B = p[i] (A row l16 <-> column 64c + 4 l16 + q for O[c][q]);
//     accumulator element v of O[c][q] is column 64c + 16g + 4v + q of row l16.
// Load n of a block always lands in register slot n % 34 (68 = 2 x 34), and the first 34
// loads of block j+1 are issued under block j's P.V MFMAs; loads past the wave's keys
// read zeros (each block's buffer resource spans only the keys it has).  After the last
// block the four waves' (m, l, O) merge through LDS (rescaled by 2^(m_w - max_w m_w), in
// wave order), and the workgroup writes ctx / row_sum (one split) or its split's partial
// slot, in flash32_kernel's layout, for flash_merge_kernel.
template <int... I, class F>
__device__ __forceinline__ void static_for_seq(std::integer_sequence<int, I...>, F&& f) {
    (f(std::integral_constant<int, I>{}), ...);
}
// f(std::integral_constant<int, i>) for i = 0 .. N-1, unrolled at compile time
template <int N, class F>
__device__ __forceinline__ void static_for(F&& f) {
    static_for_seq(std::make_integer_sequence<int, N>{}, f);
}

constexpr int kWRows = 16;
constexpr int kWKeys = 16;
constexpr int kWLoads = 68;               // 16-byte loads per lane and block: 36 K, 32 V
constexpr int kWWin = 34;                 // loads in flight
constexpr int kWPitch = kFR + 4;          // floats per row of the LDS merge buffer
// Q rows in LDS: 584 floats (2,336 bytes) apart, so that the 16-byte slot of lane (l16, g)'s
// read is 2 l16 + g (mod 16) plus a constant: distinct within each 16-lane LDS cycle
constexpr int kWQPitch = kFR + kFD + 8;
constexpr int kWQWin = 4;                 // Q^T fragment reads in flight
static_assert(kWLoads % kWWin == 0, "a load's register slot is the same in every block");

__global__ void __launch_bounds__(kFThreads, 1) flash32w_kernel(FlashArgs a) {
    // the workgroup's 16 query rows during the pass, the four waves' states after it
    __shared__ __attribute__((aligned(16))) float mo[4 * kWRows * kWPitch];
    __shared__ float mm[4 * kWRows], ml[4 * kWRows];
    static_assert(kWRows * kWQPitch <= 4 * kWRows * kWPitch, "Q rows fit the merge buffer");
    const int tid = threadIdx.x, lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int l16 = lane & 15, g = lane >> 4;

    // workgroup -> (batch, split, 16-row tile); the row tiles of a split are consecutive
    // logical workgroups, i.e. on one XCD
    const int wg = xcd_logical_block(blockIdx.x, gridDim.x);
    const int rt = wg % a.row_tiles;
    const int sp = (wg / a.row_tiles) % a.n_split;
    const int b = wg / (a.row_tiles * a.n_split);
    const int rows_b = a.Sq * a.H;
    const int r0 = rt * kWRows;
    const int row = r0 + l16;

    // the batch's keys (its length when ragged); a split past them has no keys
    const int skb = flash_batch_keys(a, b);
    const int k_lo = sp * a.keys_per_split;
    int k_hi = min(skb, k_lo + a.keys_per_split);
    int lim = k_hi - 1;
    if (a.causal) {
        lim = min(lim, skb - a.Sq + min(row, rows_b - 1) / a.H);
        k_hi = min(k_hi, skb - a.Sq + min(r0 + kWRows - 1, rows_b - 1) / a.H + 1);
    }
    // this wave's blocks: a quarter of the workgroup's, contiguous
    const int nblk = k_hi > k_lo ? (k_hi - k_lo + kWKeys - 1) / kWKeys : 0;
    const int per = (nblk + 3) >> 2;
    const int jw = min(nblk, wave * per);
    const int nb = min(nblk, jw + per) - jw;
    const int kw0 = k_lo + kWKeys * jw;
    const int kw1 = min(k_hi, kw0 + kWKeys * nb);

    // ---- the 16 query rows into LDS (latent then rope, kWQPitch floats apart): thread t
    // copies 16-byte chunks t, t + 256, .. of the 16 x 144; rows past the batch are zeros
    {
        const __amdgpu_buffer_rsrc_t rq =
            make_rsrc(reinterpret_cast<const float*>(a.qa) + (int64_t)b * rows_b * kFR);
        const __amdgpu_buffer_rsrc_t rr =
            make_rsrc(reinterpret_cast<const float*>(a.qr) + (int64_t)b * rows_b * kFD);
        // (one descriptor per loop: a per-lane choice of descriptor would make the
        // compiler loop over the lanes' distinct descriptors)
        constexpr int kLatCh = kFR / 4, kPeCh = kFD / 4;   // 128 + 16 chunks per row
        static_assert(kWRows * kLatCh % kFThreads == 0 && kWRows * kPeCh == kFThreads,
                      "whole chunks per thread");
        #pragma unroll
        for (int i = 0; i < kWRows * kLatCh / kFThreads; ++i) {
            const int e = tid + kFThreads * i;
            const int qrow = e / kLatCh, ch = e % kLatCh;
            const uint32_t mask = oob_mask(r0 + qrow, rows_b);
            *reinterpret_cast<v4u*>(mo + qrow * kWQPitch + 4 * ch) =
                load16(rq, ((uint32_t)(r0 + qrow) * (kFR * 4) + 16u * ch) | mask);
        }
        {
            const int qrow = tid / kPeCh, ch = tid % kPeCh;
            const uint32_t mask = oob_mask(r0 + qrow, rows_b);
            *reinterpret_cast<v4u*>(mo + qrow * kWQPitch + kFR + 4 * ch) =
                load16(rr, ((uint32_t)(r0 + qrow) * (kFD * 4) + 16u * ch) | mask);
        }
    }
    __syncthreads();
    // Q^T fragment of K step r: row l16's floats 16r + 4g .. +3 (rope at 512 + 16(r - 32))
    const float* q_lane = mo + l16 * kWQPitch + 4 * g;
    auto q_read = [&](int r) __attribute__((always_inline)) {
        return *reinterpret_cast<const v4u*>(q_lane + 16 * r);
    };

    // ---- the cache: block jj's buffer resources span its keys inside [kw0, kw1), from the
    // cache row of its first key (a paged cache's 16-key blocks never straddle a page)
    const char* ck_b = reinterpret_cast<const char*>(a.ckv);
    const char* pe_b = reinterpret_cast<const char*>(a.pe);
    // (readfirstlane: the values are wave-uniform, and the compiler must know it, or it
    // wraps every load in a loop over the lanes' distinct descriptors)
    auto rsrc_u = [](const char* ptr, int bytes) __attribute__((always_inline)) {
        const uint64_t v = reinterpret_cast<uint64_t>(ptr);
        const uint32_t lo = __builtin_amdgcn_readfirstlane((uint32_t)v);
        const uint32_t hi = __builtin_amdgcn_readfirstlane((uint32_t)(v >> 32));
        return __builtin_amdgcn_make_buffer_rsrc(
            reinterpret_cast<void*>(((uint64_t)hi << 32) | lo), (short)0,
            __builtin_amdgcn_readfirstlane(bytes), 0x00020000);
    };
    auto rs_kp = [&](int jj, __amdgpu_buffer_rsrc_t* rk, __amdgpu_buffer_rsrc_t* rp)
        __attribute__((always_inline)) {
        const int kb = kw0 + kWKeys * jj;
        const int left = max(0, min(kWKeys, kw1 - kb));
        const int64_t row0 = flash_key_row(a, b, kb, kw1);
        *rk = rsrc_u(ck_b + row0 * (kFR * 4), left * (kFR * 4));
        *rp = rsrc_u(pe_b + row0 * (kFD * 4), left * (kFD * 4));
    };
    const uint32_t k_off = (uint32_t)l16 * (kFR * 4) + 16u * g;
    const uint32_t p_off = (uint32_t)l16 * (kFD * 4) + 16u * g;
    const uint32_t v_off = (uint32_t)(4 * g) * (kFR * 4) + 16u * l16;
    auto load_n = [&](auto n_tag, __amdgpu_buffer_rsrc_t rk, __amdgpu_buffer_rsrc_t rp)
        __attribute__((always_inline)) {
        constexpr int n = decltype(n_tag)::value;
        if constexpr (n < k32LatReads) return load16(rk, k_off + 64u * n);
        else if constexpr (n < k32LatReads + k32PeReads)
            return load16(rp, p_off + 64u * (n - k32LatReads));
        else {
            constexpr int i = (n - 36) >> 3, c = (n - 36) & 7;
            return load16(rk, v_off + (uint32_t)(i * kFR * 4 + 256 * c));
        }
    };

    v4f O[8][4];   // [c][q]
    v4u buf[kWWin];
    float m_ref = -INFINITY, m_neg = 0.f, thr = -INFINITY, l_run = 0.f;
    for (int pass = 1;; ++pass) {
        #pragma unroll
        for (int c = 0; c < 8; ++c)
            #pragma unroll
            for (int q = 0; q < 4; ++q) O[c][q] = v4f{};
        l_run = 0.f;
        {
            __amdgpu_buffer_rsrc_t rk, rp;
            rs_kp(0, &rk, &rp);
            static_for<kWWin>([&](auto n) { buf[n] = load_n(n, rk, rp); });
        }
        bool again = false;
        for (int jj = 0; jj < nb; ++jj) {
            __amdgpu_buffer_rsrc_t rk, rp, rk1, rp1;
            rs_kp(jj, &rk, &rp);
            rs_kp(jj + 1, &rk1, &rp1);
            v4f s2[2] = {v4f{}, v4f{}};
            float p[4];
            v4u qb[kWQWin];
            #pragma unroll
            for (int r = 0; r < kWQWin; ++r) qb[r] = q_read(r);
            static_for<kWLoads>([&](auto n_tag) {
                constexpr int n = decltype(n_tag)::value;
                constexpr int slot = n % kWWin;
                const v4u cur = buf[slot];
                if constexpr (n < k32LatReads + k32PeReads) {
                    const v4u qv = qb[n % kWQWin];
                    if constexpr (n + kWQWin < k32LatReads + k32PeReads) qb[n % kWQWin] = q_read(n + kWQWin);
                    #pragma unroll
                    for (int q = 0; q < 4; ++q)
                        s2[q & 1] = mfma16f(__uint_as_float(cur[q]), __uint_as_float(qv[q]), s2[q & 1]);
                } else {
                    constexpr int i = (n - 36) >> 3, c = (n - 36) & 7;
                    #pragma unroll
                    for (int q = 0; q < 4; ++q)
                        O[c][q] = mfma16f(__uint_as_float(cur[q]), p[i], O[c][q]);
                }
                if constexpr (n + kWWin < kWLoads)
                    buf[slot] = load_n(std::integral_constant<int, n + kWWin>{}, rk, rp);
                else
                    buf[slot] = load_n(std::integral_constant<int, n + kWWin - kWLoads>{}, rk1, rp1);
                // each step in program order: its four MFMAs, then the load kWWin ahead and
                // the Q^T read kWQWin ahead (left alone, the scheduler sinks loads and reads
                // to their uses and exposes their latency)
                __builtin_amdgcn_sched_barrier(0);
                if constexpr (n == k32LatReads + k32PeReads - 1) {
                    // softmax numerators of the block: element v of lane l is key kb + 4g + v
                    // of row l16 (the mask is branch-free, so the score part stays one
                    // scheduling region)
                    v4f sc = s2[0] + s2[1];
                    const int kb = kw0 + kWKeys * jj;
                    #pragma unroll
                    for (int v = 0; v < 4; ++v) sc[v] = kb + 4 * g + v <= lim ? sc[v] : -INFINITY;
                    const float smax = fmaxf(fmaxf(sc[0], sc[1]), fmaxf(sc[2], sc[3]));
                    if (__builtin_amdgcn_ballot_w64(!(smax * a.c <= thr))) {
                        const float bm = row4_reduce(smax, OpMax{}) * a.c;
                        const bool over = pass < k32MaxPasses && m_ref != -INFINITY && bm > thr;
                        if (__builtin_amdgcn_ballot_w64(over)) again = true;
                        if (m_ref == -INFINITY || over) {
                            m_ref = bm;
                            m_neg = bm == -INFINITY ? 0.f : -bm;
                            thr = bm + k32Headroom;
                        }
                    }
                    #pragma unroll
                    for (int v = 0; v < 4; ++v)
                        p[v] = __builtin_amdgcn_exp2f(__builtin_fmaf(sc[v], a.c, m_neg));
                    l_run += (p[0] + p[1]) + (p[2] + p[3]);
                }
            });
            if (again) break;
        }
        if (!again) break;
    }

    // ---- the four waves' states merge through LDS (over the query rows: every wave is
    // past its last Q^T read first)
    l_run = row4_reduce(l_run, OpSum{});
    __syncthreads();
    float* mow = mo + (wave * kWRows + l16) * kWPitch;
    #pragma unroll
    for (int c = 0; c < 8; ++c)
        #pragma unroll
        for (int v = 0; v < 4; ++v)
            *reinterpret_cast<v4f*>(mow + 64 * c + 16 * g + 4 * v) =
                v4f{O[c][0][v], O[c][1][v], O[c][2][v], O[c][3][v]};
    if (g == 0) {
        mm[wave * kWRows + l16] = m_ref;
        ml[wave * kWRows + l16] = l_run;
    }
    __syncthreads();
    // wave w writes columns 128w .. 128w+127: lane l has row l/4, 32 columns from 32 (l%4)
    const int rr_ = lane >> 2;
    const int cb = 128 * wave + 32 * (lane & 3);
    float M = -INFINITY;
    #pragma unroll
    for (int w = 0; w < 4; ++w) M = fmaxf(M, mm[w * kWRows + rr_]);
    float f[4];
    #pragma unroll
    for (int w = 0; w < 4; ++w) {
        const float mw = mm[w * kWRows + rr_];
        f[w] = mw == -INFINITY ? 0.f : __builtin_amdgcn_exp2f(mw - M);
    }
    v4f acc[8];
    float L = 0.f;
    #pragma unroll
    for (int w = 0; w < 4; ++w) {
        const float* src = mo + (w * kWRows + rr_) * kWPitch + cb;
        #pragma unroll
        for (int k = 0; k < 8; ++k) {
            const v4f x = *reinterpret_cast<const v4f*>(src + 4 * k);
            acc[k] = w == 0 ? f[0] * x : acc[k] + f[w] * x;
        }
        L = w == 0 ? f[0] * ml[rr_] : L + f[w] * ml[w * kWRows + rr_];
    }
    const int orow = r0 + rr_;
    if (orow < rows_b) {
        const bool direct = a.n_split == 1;
        const int64_t slot = (direct ? (int64_t)b : (int64_t)sp * a.B + b) * rows_b + orow;
        float* dst = (direct ? a.o_direct : a.o) + slot * kFR + cb;
        #pragma unroll
        for (int k = 0; k < 8; ++k) *reinterpret_cast<v4f*>(dst + 4 * k) = acc[k];
        if (wave == 0 && (lane & 3) == 0) {
            if (!direct) a.m[slot] = M;
            (direct ? a.l_direct : a.l)[slot] = L;
        }
    }
}

constexpr int kFStages = 4;   // LDS ring depth

// ctx = sum_s w_s O_s, row_sum = sum_s w_s l_s, w_s = 2^(m_s - max_s m_s).  One workgroup
// per row: its threads take the row maximum over the splits, then wave w sums splits
// w, w+4, ... (lane: 8 columns), and the four waves' sums are added in wave order -- a
// fixed order, so the merge is deterministic.  Each wave keeps a split's 2 KB row in
// flight per iteration, so many splits (small batches) do not serialise on latency.
// Split s of row r (batch b, row i of the batch) is partial slot unit(s) * rows_b + i:
// unit(s) = s * B + b for the uniform splits, first[b] + s for a work list (whose batches
// of one chunk were written straight to ctx / row_sum and are skipped here).
__global__ void __launch_bounds__(256) flash_merge_kernel(const float* __restrict__ o,
                                                          const float* __restrict__ m,
                                                          const float* __restrict__ l,
                                                          float* __restrict__ ctx,
                                                          float* __restrict__ row_sum, int B,
                                                          int rows_b, int n_split,
                                                          const int* __restrict__ wl) {
    __shared__ float red[256];
    __shared__ v4f part[4][64][2];
    __shared__ float lpart[4];
    const int r = blockIdx.x, tid = threadIdx.x, wave = tid >> 6, lane = tid & 63;
    const int b = r / rows_b, i = r - b * rows_b;
    int64_t unit0 = b, unit_step = B;
    if (wl) {
        n_split = load_uniform(wl + kWlHead + B + b);
        if (n_split == 1) return;
        unit0 = load_uniform(wl + kWlHead + b);
        unit_step = 1;
    }
    auto slot_of = [&](int s) { return (unit0 + s * unit_step) * rows_b + i; };
    float mx = -INFINITY;
    for (int s = tid; s < n_split; s += 256) mx = fmaxf(mx, m[slot_of(s)]);
    red[tid] = mx;
    __syncthreads();
    #pragma unroll
    for (int w = 128; w > 0; w >>= 1) {
        if (tid < w) red[tid] = fmaxf(red[tid], red[tid + w]);
        __syncthreads();
    }
    mx = red[0];
    v4f acc0 = {0.f, 0.f, 0.f, 0.f}, acc1 = acc0;
    float ls = 0.f;
    for (int s = wave; s < n_split; s += 4) {
        const int64_t slot = slot_of(s);
        const float ms = m[slot];
        const float w = ms == -INFINITY ? 0.f : __builtin_amdgcn_exp2f(ms - mx);
        const v4f* src = reinterpret_cast<const v4f*>(o + slot * kFR) + 2 * lane;
        acc0 += w * src[0];
        acc1 += w * src[1];
        ls += w * l[slot];
    }
    part[wave][lane][0] = acc0;
    part[wave][lane][1] = acc1;
    if (lane == 0) lpart[wave] = ls;
    __syncthreads();
    if (wave == 0) {
        #pragma unroll
        for (int w = 1; w < 4; ++w) {
            acc0 += part[w][lane][0];
            acc1 += part[w][lane][1];
        }
        v4f* dst = reinterpret_cast<v4f*>(ctx + (int64_t)r * kFR) + 2 * lane;
        dst[0] = acc0;
        dst[1] = acc1;
        if (lane == 0) row_sum[r] = ((lpart[0] + lpart[1]) + lpart[2]) + lpart[3];
    }
}

// Work list of a ragged batch (one workgroup; key counts are device data).  The chunk rule,
// the fit check, each batch's chunk counts and the order of the items are the functions of
// worklist.h; this kernel spreads them over its threads (thread tid owns batches
// [wl_thread_first(tid), wl_thread_first(tid + 1))) and turns the sums they need into
// wave-level reductions and scans.
__global__ void __launch_bounds__(kWlThreads) flash_worklist_kernel(const int* __restrict__ seq_lens,
                                                                    int B, int Sk, int row_tiles,
                                                                    int block_keys, int max_items,
                                                                    int* __restrict__ wl) {
    // reductions and scans run within each wave (__shfl_*), then over the four waves'
    // totals in LDS: a handful of barriers, since this one-workgroup kernel sits on the
    // decode step's critical path
    static_assert(kWlThreads == 256 && kWlBuckets == 256, "one bucket per thread, four waves");
    __shared__ long long w_tot[4];
    __shared__ int w_min[4], w_max[4], w_cnt[4], w_full[4], w_rem[4];
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int b0 = wl_thread_first(tid, B), b1 = wl_thread_first(tid + 1, B);
    // a thread's lengths stay in registers (up to 8 batches per thread, B <= 2048); past
    // that they are read again
    constexpr int kRegLens = 8;
    int lens_r[kRegLens];
    #pragma unroll
    for (int i = 0; i < kRegLens; ++i) lens_r[i] = b0 + i < b1 ? wl_len(seq_lens[b0 + i], Sk) : 0;
    auto len_of = [&](int b) {
        const int i = b - b0;
        if (i < kRegLens) {
            int v = 0;
            #pragma unroll
            for (int j = 0; j < kRegLens; ++j) v = j == i ? lens_r[j] : v;
            return v;
        }
        return wl_len(seq_lens[b], Sk);
    };
    long long tot = 0;
    int mn = 0x7fffffff, mx = 0;
    for (int b = b0; b < b1; ++b) {
        const int L = len_of(b);
        tot += L;
        mn = min(mn, L);
        mx = max(mx, L);
    }
    for (int d = 32; d > 0; d >>= 1) {
        tot += __shfl_xor(tot, d);
        mn = min(mn, __shfl_xor(mn, d));
        mx = max(mx, __shfl_xor(mx, d));
    }
    if (lane == 0) { w_tot[wave] = tot; w_min[wave] = mn; w_max[wave] = mx; }
    __syncthreads();
    tot = ((w_tot[0] + w_tot[1]) + w_tot[2]) + w_tot[3];
    mn = min(min(w_min[0], w_min[1]), min(w_min[2], w_min[3]));
    mx = max(max(w_max[0], w_max[1]), max(w_max[2], w_max[3]));
    int chunk = wl_initial_chunk(tot, mn, mx, B, Sk, row_tiles, block_keys);
    int cnt, full;
    for (;;) {
        cnt = 0; full = 0;
        for (int b = b0; b < b1; ++b) {
            const int L = len_of(b);
            cnt += wl_chunk_count(L, chunk);
            full += wl_full_count(L, chunk);
        }
        int c = cnt;
        for (int d = 32; d > 0; d >>= 1) c += __shfl_xor(c, d);
        __syncthreads();   // every thread has read the previous round's w_cnt
        if (lane == 0) w_cnt[wave] = c;
        __syncthreads();
        const int total = ((w_cnt[0] + w_cnt[1]) + w_cnt[2]) + w_cnt[3];
        if (wl_fits(total, max_items, chunk, Sk)) break;
        chunk *= 2;
    }
    // exclusive prefix sums over the threads: inclusive scans within each wave, then the
    // totals of the waves before
    int ic = cnt, ifl = full;
    for (int d = 1; d < 64; d <<= 1) {
        const int c = __shfl_up(ic, d), f = __shfl_up(ifl, d);
        if (lane >= d) { ic += c; ifl += f; }
    }
    __syncthreads();   // w_cnt of the loop above has been read by every thread
    if (lane == 63) { w_cnt[wave] = ic; w_full[wave] = ifl; }
    __syncthreads();
    int pc = 0, pf = 0, n_full = 0, n_all = 0;
    for (int w = 0; w < 4; ++w) {
        if (w < wave) { pc += w_cnt[w]; pf += w_full[w]; }
        n_full += w_full[w];
        n_all += w_cnt[w];
    }
    int slot = pc + ic - cnt, fi = pf + ifl - full;
    int* first = wl + kWlHead;
    int* count = first + B;
    int* items = count + B;
    const int n_items = min(n_all, max_items);
    if (mn == mx) {
        // equal lengths: every batch has the same chunks, so item t is computed directly
        // (all threads write; at B=1 one thread would otherwise write every item)
        const int n = wl_chunk_count(mx, chunk), nf = wl_full_count(mx, chunk);
        for (int b = tid; b < B; b += kWlThreads) {
            first[b] = b * n;
            count[b] = n;
        }
        for (int it = tid; it < n_items; it += kWlThreads)
            wl_equal_item(it, B, nf, &items[2 * it], &items[2 * it + 1]);
        if (tid == 0) {
            wl[0] = n_items;
            wl[1] = chunk;
        }
        return;
    }
    // Ragged: the shorter last chunks follow the full ones longest first (a counting sort
    // over the length buckets), so the dispatcher hands out the longest remaining pieces
    // first; the order inside a bucket is the LDS atomics' and does not matter, since an
    // item's partial slot (first[b] + c) and so the merge order depend on b and c only.
    // (Simulated in-order dispatch at B=128, lengths uniform in [1, 4989]: the makespan
    // drops from 2916 to 2621 key-times against a 2571 lower bound.)
    __shared__ int hist[kWlBuckets], cursor[kWlBuckets];
    hist[tid] = 0;
    cursor[tid] = 0;
    __syncthreads();
    for (int b = b0; b < b1; ++b) {
        const int L = len_of(b);
        if (wl_has_short(L, chunk)) atomicAdd(&hist[wl_bucket(L, chunk)], 1);
    }
    __syncthreads();
    int hb = hist[tid], hs = hb;   // exclusive scan of the buckets in order
    for (int d = 1; d < 64; d <<= 1) {
        const int v = __shfl_up(hs, d);
        if (lane >= d) hs += v;
    }
    if (lane == 63) w_rem[wave] = hs;
    __syncthreads();
    for (int w = 0; w < wave; ++w) hs += w_rem[w];
    hist[tid] = hs - hb;              // bucket start among the last chunks
    __syncthreads();
    for (int b = b0; b < b1; ++b) {
        const int L = len_of(b);
        const int n = wl_chunk_count(L, chunk);
        first[b] = slot;
        count[b] = n;
        slot += n;
        for (int c = 0; c < n; ++c) {
            const bool is_full = (long long)(c + 1) * chunk <= L;
            const int q = wl_bucket(L, chunk);
            const int it = is_full ? fi++ : n_full + hist[q] + atomicAdd(&cursor[q], 1);
            if (it < max_items) {   // always (the fit check above); a guard
                items[2 * it] = b;
                items[2 * it + 1] = c;
            }
        }
    }
    if (tid == 0) {
        wl[0] = n_items;
        wl[1] = chunk;
    }
}

}  // namespace

bool flash_supported(const FlashProblem& p) {
    if (p.fp8_kv && !(p.half && !p.f16 && p.kv_scale > 0.f && std::isfinite(p.kv_scale)))
        return false;   // an fp8 cache is read with bf16 queries and a positive scale
    return p.R == kFR && p.D == kFD && p.B > 0 && p.Sq > 0 && p.H > 0 && p.Sk > 0;
}

FlashPlan plan_flash(const FlashProblem& p) {
    FlashPlan f;
    f.row_tiles = (p.Sq * p.H + kFRows - 1) / kFRows;
    const int base = p.B * f.row_tiles;
    const int block_keys = p.half ? kFKeys : k32Keys;
    const int blocks = (p.Sk + block_keys - 1) / block_keys;
    const size_t rows = (size_t)p.B * p.Sq * p.H;
    const size_t rows_b = (size_t)p.Sq * p.H;
    // fp32 batches that would need key splits to fill the chip with 64-row workgroups may
    // run on 16-row workgroups of key-split waves (flash32w_kernel): a quarter of the
    // splits for as many workgroups.  Splits for about one workgroup per CU; each wave gets
    // the same whole number of 16-key blocks, and the fewest splits that keep that number.
    // Its fixed cost per launch is lower (less Q to load, a quarter of the split partials
    // to write and merge) but a block costs it ~5.4 us against ~4.2 in the 64-row kernel,
    // so it is taken up to 12 blocks per wave (measured at B=1: Sk 512 / 4989 / 16384 20.0 /
    // 35.4 / 64.6 us against 25.2 / 46.8 / 75.4; B=2..4, Sk=4989: 47.2 / 63.5 / 75.0
    // against 58.2 / 67.7 / 77.0; B=8: 129.9 against 119.0, 20 blocks per wave; with 3d:
    // B=4, 10 blocks: 83.0 against 88.3, and at 16 blocks B=6 121.5 against 108.2, B=4 with
    // Sk=8192 116.5 against 113.0, B=2 with Sk=16384 116.6 against 115.9).
    // MLA_FLASH32_WAVE=0 / 1 forces the choice (both kernels give the same results to
    // rounding).
    const char* wave_env = std::getenv("MLA_FLASH32_WAVE");
    // (ragged and paged batches too, on uniform splits of the table's span: a short
    // sequence's later splits are empty workgroups -- at these batch sizes that costs less
    // than the balanced work list's 64-row pass)
    const bool wave_ok = !p.half && !p.fp8_kv && !p.want_list;
    const int base16 = p.B * ((p.Sq * p.H + kWRows - 1) / kWRows);
    const int wblocks = (p.Sk + kWKeys - 1) / kWKeys;
    const int target = std::max(1, kNumCUs / base16);   // splits that fit one round
    const int bpw = std::max(1, (wblocks + 4 * target - 1) / (4 * target));
    constexpr int kWaveMaxBlocks = 12;
    if (wave_ok && (wave_env ? wave_env[0] == '1' : base < kNumCUs && bpw <= kWaveMaxBlocks)) {
        f.wave = true;
        f.row_tiles = (p.Sq * p.H + kWRows - 1) / kWRows;
        f.n_split = (wblocks + 4 * bpw - 1) / (4 * bpw);
        f.keys_per_split = 4 * bpw * kWKeys;
        f.partial_bytes = f.n_split > 1 ? rows * f.n_split * (kFR + 2) * sizeof(float)
                                        : rows * sizeof(float);
        return f;
    }
    if (p.seq_lens || p.ragged) {
        // ragged keys: a work list built on the device from the key counts balances the
        // grid (flash_worklist_kernel); the partial slots, the list and its grid are sized
        // for its largest case
        f.balanced = true;
        f.max_items = wl_max_items(p.B, f.row_tiles);
        f.n_split = 0;
        f.keys_per_split = 0;
        const size_t wl_bytes = ((size_t)wl_ints(p.B, f.max_items) * sizeof(int) + 255) / 256 * 256;
        f.partial_bytes = wl_bytes + (size_t)f.max_items * rows_b * (kFR + 2) * sizeof(float);
        return f;
    }
    // about one workgroup per CU (the LDS ring admits one per CU), at least one key block
    // per split; MLA_FLASH_SPLITS=n forces n splits (for measurements)
    f.keys_per_split = dense_keys_per_split(p.Sk, base, block_keys);
    if (const char* sp_env = std::getenv("MLA_FLASH_SPLITS")) {
        const int n = std::atoi(sp_env);
        if (n >= 1) f.keys_per_split = (blocks + std::min(n, blocks) - 1) / std::min(n, blocks) * block_keys;
    }
    const int per = f.keys_per_split / block_keys;
    f.n_split = (blocks + per - 1) / per;
    // split partials (O, m, l); with one split O and l go straight to ctx / row_sum and
    // only the row maxima need a scratch row
    f.partial_bytes = f.n_split > 1 ? rows * f.n_split * (kFR + 2) * sizeof(float)
                                    : rows * sizeof(float);
    return f;
}

int flash_worklist_ints(const FlashProblem& p, const FlashPlan& f) {
    return f.balanced ? wl_ints(p.B, f.max_items) : 0;
}

hipError_t launch_flash_worklist(const FlashProblem& p, const FlashPlan& f, int* wl,
                                 hipStream_t stream) {
    if (!f.balanced || !p.seq_lens) return hipErrorInvalidValue;
    hipLaunchKernelGGL(flash_worklist_kernel, dim3(1), dim3(kWlThreads), 0, stream, p.seq_lens,
                       p.B, p.Sk, f.row_tiles, p.half ? kFKeys : k32Keys, f.max_items, wl);
    return hipGetLastError();
}

FlashPartials flash_partials(const FlashProblem& p, const FlashPlan& f, const float* partials) {
    const size_t rows = (size_t)p.B * p.Sq * p.H;
    FlashPartials r{nullptr, nullptr, nullptr, f.balanced ? 0 : f.n_split};
    if (!f.balanced && f.n_split > 1) {
        r.o = partials;
        r.m = partials + (size_t)f.n_split * rows * kFR;
        r.l = r.m + (size_t)f.n_split * rows;
    }
    return r;
}

namespace {
// The 16-bit and fp8-cache kernel the launcher takes for p (the switches below).
enum class Flash16 { kCodeRing, kSpecPv64, kSpecPv32, kKeySplit };
Flash16 flash16_choice(const FlashProblem& p) {
    const char* spec_env = std::getenv("MLA_FLASH16_SPEC");
    const bool spec = !(spec_env && spec_env[0] == '0');
    const char* pv_env = std::getenv("MLA_FLASH16_PV");
    const bool pv64 = !(pv_env && std::strcmp(pv_env, "32") == 0);
    const char* f8_env = std::getenv("MLA_FLASH16_FP8");
    const bool f8_convert = f8_env && std::strcmp(f8_env, "convert") == 0;
    if (!spec) return Flash16::kKeySplit;
    if (p.fp8_kv && !f8_convert) return Flash16::kCodeRing;
    return pv64 ? Flash16::kSpecPv64 : Flash16::kSpecPv32;
}
}  // namespace

bool flash_ctx16_ok(const FlashProblem& p, const FlashPlan& f) {
    const char* env = std::getenv("MLA_CTX16");
    if (env && env[0] == '0') return false;
    const Flash16 k = flash16_choice(p);
    return (p.half || p.fp8_kv) && !f.balanced && !f.wave && f.n_split == 1 &&
           (k == Flash16::kCodeRing || k == Flash16::kSpecPv64);
}

hipError_t launch_flash(const FlashProblem& p, const FlashPlan& f, float* ctx, float* row_sum,
                        float* partials, hipStream_t stream, bool merge, void* ctx16) {
    if (ctx16 && !flash_ctx16_ok(p, f)) return hipErrorInvalidValue;
    const int rows = p.B * p.Sq * p.H;
    const int rows_b = p.Sq * p.H;
    FlashArgs a;
    a.qa = static_cast<const uint16_t*>(p.qa);
    a.qr = static_cast<const uint16_t*>(p.qr);
    a.ckv = static_cast<const uint16_t*>(p.ckv);
    a.pe = static_cast<const uint16_t*>(p.pe);
    a.wl = nullptr;
    a.o_direct = ctx;
    a.l_direct = row_sum;
    a.ctx16 = ctx16;
    int grid;
    int* wl = nullptr;
    if (f.balanced) {
        if (!p.seq_lens) return hipErrorInvalidValue;
        wl = reinterpret_cast<int*>(partials);
        const size_t wl_bytes =
            ((size_t)wl_ints(p.B, f.max_items) * sizeof(int) + 255) / 256 * 256;
        float* slots = reinterpret_cast<float*>(reinterpret_cast<char*>(partials) + wl_bytes);
        a.wl = wl;
        a.o = slots;
        a.m = slots + (size_t)f.max_items * rows_b * kFR;
        a.l = a.m + (size_t)f.max_items * rows_b;
        grid = f.max_items * f.row_tiles;
    } else if (f.wave) {
        // the wave kernel writes ctx / row_sum itself with one split
        a.o = partials;
        a.m = partials + (size_t)f.n_split * rows * kFR;
        a.l = a.m + (size_t)f.n_split * rows;
        if (f.n_split == 1) a.m = a.l = a.o = nullptr;
        grid = p.B * f.row_tiles * f.n_split;
    } else if (f.n_split > 1) {
        a.o = partials;
        a.m = partials + (size_t)f.n_split * rows * kFR;
        a.l = a.m + (size_t)f.n_split * rows;
        grid = p.B * f.row_tiles * f.n_split;
    } else {
        a.o = ctx;
        a.l = row_sum;
        a.m = partials;   // the row maxima are not needed: a small scratch row
        grid = p.B * f.row_tiles;
    }
    a.B = p.B; a.Sq = p.Sq; a.Sk = p.Sk; a.H = p.H;
    a.n_split = f.balanced ? 1 : f.n_split;
    a.keys_per_split = f.keys_per_split;
    a.row_tiles = f.row_tiles;
    a.key_stride = p.key_stride > 0 ? p.key_stride : p.Sk;
    a.c = 1.4426950408889634f / p.scale;
    a.o_scale = 1.f;
    if (p.fp8_kv) {   // scores and ctx take the cache scale (the codes enter the MFMAs)
        a.c *= p.kv_scale;
        a.o_scale = p.kv_scale;
    }
    a.causal = p.causal ? 1 : 0;
    a.seq_lens = p.seq_lens;
    a.block_table = p.block_table;
    a.page_size = p.page_size;
    a.max_pages = p.page_size > 0 ? p.Sk / p.page_size : 0;
    if (p.block_table && (p.page_size <= 0 || p.page_size % 64 != 0 || p.Sk % p.page_size != 0))
        return hipErrorInvalidValue;
    if (f.balanced) {
        hipError_t e = launch_flash_worklist(p, f, wl, stream);
        if (e != hipSuccess) return e;
    }
    // 16-bit: the specialised-wave pass unless MLA_FLASH16_SPEC=0 asks for the key-split one
    const Flash16 k16 = flash16_choice(p);
    const bool spec = k16 != Flash16::kKeySplit;
    // fp32, 64-row workgroups: the specialised-wave pass unless MLA_FLASH32_SPEC=0 asks for
    // flash32_kernel
    const char* spec32_env = std::getenv("MLA_FLASH32_SPEC");
    const bool spec32 = !(spec32_env && spec32_env[0] == '0');
    // 16-bit specialised waves: the P.V waves over 64 rows x 128 columns (measured at cfg4,
    // bf16: 177-179 us against 178-186 us, and the same results bit for bit), or over 32 rows
    // x 256 columns with MLA_FLASH16_PV=32
    const bool pv64 = k16 != Flash16::kSpecPv32;
    // an fp8 cache: the code-ring pass (flash16x8_kernel; cfg4 shape, attention with 3d:
    // 171 us against 220-240 us) unless MLA_FLASH16_FP8=convert asks for the pass that
    // converts each block into a bf16 ring
    if (p.fp8_kv && k16 == Flash16::kCodeRing)
        hipLaunchKernelGGL(flash16x8_kernel, dim3(grid), dim3(kXThreads), 0, stream, a);
    else if (p.fp8_kv && spec && pv64)
        hipLaunchKernelGGL((flash16x_kernel<bf16_t, true, true>), dim3(grid), dim3(kXThreads), 0, stream, a);
    else if (p.half && spec && pv64 && p.f16)
        hipLaunchKernelGGL((flash16x_kernel<f16_t, false, true>), dim3(grid), dim3(kXThreads), 0, stream, a);
    else if (p.half && spec && pv64)
        hipLaunchKernelGGL((flash16x_kernel<bf16_t, false, true>), dim3(grid), dim3(kXThreads), 0, stream, a);
    else if (p.fp8_kv && spec)
        hipLaunchKernelGGL((flash16x_kernel<bf16_t, true>), dim3(grid), dim3(kXThreads), 0, stream, a);
    else if (p.fp8_kv)
        hipLaunchKernelGGL((flash16_kernel<3, bf16_t, true>), dim3(grid), dim3(kFThreads), 0, stream, a);
    else if (p.half && spec && p.f16)
        hipLaunchKernelGGL((flash16x_kernel<f16_t, false>), dim3(grid), dim3(kXThreads), 0, stream, a);
    else if (p.half && spec)
        hipLaunchKernelGGL((flash16x_kernel<bf16_t, false>), dim3(grid), dim3(kXThreads), 0, stream, a);
    else if (p.half && p.f16)
        hipLaunchKernelGGL((flash16_kernel<kFStages, f16_t, false>), dim3(grid), dim3(kFThreads), 0, stream, a);
    else if (p.half)
        hipLaunchKernelGGL((flash16_kernel<kFStages, bf16_t, false>), dim3(grid), dim3(kFThreads), 0, stream, a);
    else if (f.wave)
        hipLaunchKernelGGL(flash32w_kernel, dim3(grid), dim3(kFThreads), 0, stream, a);
    else if (spec32)
        hipLaunchKernelGGL(flash32x_kernel<kFStages>, dim3(grid), dim3(kXThreads), 0, stream, a);
    else
        hipLaunchKernelGGL(flash32_kernel<kFStages>, dim3(grid), dim3(kFThreads), 0, stream, a);
    hipError_t e = hipGetLastError();
    if (e != hipSuccess || (!f.balanced && f.n_split == 1)) return e;
    if (!merge && !f.balanced) return e;   // the caller folds the merge in
    hipLaunchKernelGGL(flash_merge_kernel, dim3((unsigned)rows), dim3(256), 0, stream, a.o,
                       a.m, a.l, ctx, row_sum, p.B, rows_b, f.n_split, a.wl);
    return hipGetLastError();
}

}  // namespace mla
