// Weight-streaming GEMM for the 16-bit (bf16 / fp16) products whose A operand is a small
// batch of activation rows (M <= 128 per tile) and whose B operand is a weight matrix
// streamed once from HBM: 2a1 (x @ W_q_a) and 2a2 (q_lat @ W_q_b) of the Q path, 3d from
// the fused pass's 16-bit ctx (NT, G = heads) and the output projection beside the layer;
// fp32 output, output in the storage format or split-K partials, and for 2a2 the fused
// epilogues that also do 2b and 2c.  It replaces gemm_kernel for those shapes
// (gemm.hip: plan_gemm picks it), whose staging round-trips every operand byte through
// registers and transposes the N-contiguous weights on the way into LDS.
//
// Workgroup = 4 wave64s over a 128-row x BN-column tile (BN = 256, 128 or 64), 2 x 2 waves of
// 64 x BN/2, on the 32x32x16 16-bit MFMA.  K is walked in 64-deep slices through an LDS
// ring of NS stages (3, 4 or 6), and both operands go global -> LDS with direct-to-LDS
// loads (no registers):
//   A: 128 rows x 128 bytes per slice, read back as K-contiguous fragments (ds_read_b128);
//   W: 64 rows x 2*BN bytes per slice, N-contiguous as in memory, read back as the MFMA's
//      K-contiguous B fragments with the transposing ds_read_b64_tr_b16 (two per fragment:
//      within each 16-lane group lanes 4q .. 4q+3 address row q and lane j receives
//      column j of the four rows); NT (W rows K-contiguous): BN rows x 128 bytes per slice,
//      staged and read exactly like A.
// NS - 1 slices are in flight while one feeds the MFMAs, and one barrier per slice orders
// the ring.  Chunk permutations keep every LDS read free of bank conflicts: 16-byte chunk c
// of A row r sits at c ^ ((r >> 1) & 7), and chunk c of W row r at c ^ (4 (r & 3)) for
// BN = 128 and 256 (16 or 32 chunks a row; the XOR stays inside each 256-byte window),
// c ^ (4 ((r >> 1) & 1)) for BN = 64 (8 chunks); the loads
// write chunk positions in order and take the permutation in their global offsets.
// Rows past M and slices past the workgroup's K range load zeros (out-of-range buffer
// offsets), so every slice issues the same loads and one wait count serves them all.
//
// 2a2's fused epilogues (QUP modes): kQupRope writes the nope columns as the 16-bit q_nope
// that 2c reads and rotates the rope columns into q_rope (2b).  kQupAbsorb also does 2c: its
// 128-column tiles are, in threes, head 2j's nope columns, head 2j+1's, and both heads' rope
// columns (64 each; the W loads take that column map in their offsets), so a nope tile holds
// the head's whole q_nope block.  W_uk[h] comes in as 64 x 128 slices in the W layout while
// the main loop runs: the first two into the RoPE table's space (a nope tile has no rope
// columns), the others in place of the ring's slices past the K range.  After the loop the
// block is rounded to the storage format into LDS in the A layout, and 2c's MFMAs run on the
// same fragment reads, in the K order of the tiled engine's 2c, so q_abs gets the same bits
// as 2a2 + 2c as separate launches.
#include "kernels.h"
#include "mma.h"
#include "stage.h"

namespace mla {

namespace {

typedef float v2f __attribute__((ext_vector_type(2)));

constexpr int kWBM = 128;                     // rows per workgroup
constexpr int kWKS = 64;                      // K per slice
constexpr int kWThreads = 256;
constexpr int kWAStage = kWBM * kWKS * 2;     // 16 KB of A per slice
constexpr int kWLoadsA = kWAStage / 1024 / 4; // 1 KB loads per wave and slice: 4

struct WArgs {
    const uint16_t* A; int64_t lda, sAg;      // elements
    const uint16_t* B; int64_t ldb, sBg;
    float* C; int64_t ldc, sCg;               // split == 1: fp32 C, or with C16 set
    uint16_t* C16;                            // C in the storage format (split == 1)
    float* ws; int64_t ws_split;              // split > 1: partials [split][G][M][N]
    int M, N, K, G, split, k_chunk, tiles_m, tiles_n;
    QUpEpilogue q;                            // the fused 2a2 epilogue (QUP kernels)
};

constexpr int kQupNone = 0, kQupRope = 1, kQupAbsorb = 2;

template <typename TL, int BN, int NS, int MINB, int QUP, bool NT = false>
__global__ void __launch_bounds__(kWThreads, MINB) wgemm_kernel(WArgs a) {
    static_assert(!NT || QUP == kQupNone, "the fused epilogues read N-contiguous W");
    constexpr int kBRow = 2 * BN;                        // bytes per W row of a slice
    constexpr int kBStage = kWKS * kBRow;                // 16 KB / 8 KB
    constexpr int kStage = kWAStage + kBStage;
    constexpr int kLoadsB = kBStage / 1024 / 4;          // 8 / 4 / 2 per wave and slice
    constexpr int kLoads = kWLoadsA + kLoadsB;
    constexpr int kRowsPerLoadB = 1024 / kBRow;          // 2 / 4 / 8 W rows per 1 KB load
    constexpr int CB = BN / 64;                          // 32-column blocks per wave
    // QUP: the tile rows' RoPE table (rows x 32 pairs x (cos, sin)) after the ring
    constexpr int kTab = QUP ? kWBM * 32 * 8 : 0;
    static_assert(QUP != kQupAbsorb || (BN == 128 && NS == 4),
                  "the absorb tail's LDS plan: A2 32 KB + W_uk 96 KB in the ring, 32 KB in the table");
    __shared__ __attribute__((aligned(1024))) uint8_t smem[NS * kStage + kTab];

    const int tid = threadIdx.x, lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    int t = xcd_logical_block(blockIdx.x, gridDim.x);
    const int tn = t % a.tiles_n; t /= a.tiles_n;
    const int tm = t % a.tiles_m; t /= a.tiles_m;
    const int sp = t % a.split;
    const int g = t / a.split;
    const int m0 = tm * kWBM, n0 = tn * BN;
    // kQupAbsorb: tile tn = 3j + r is head 2j + r's nope columns (r < 2) or the rope columns
    // of heads 2j and 2j + 1 (r = 2)
    bool rope_tile = false;
    int head0 = 0;
    if constexpr (QUP == kQupAbsorb) {
        const int trip = tn / 3, r3 = tn - 3 * trip;
        rope_tile = r3 == 2;
        head0 = 2 * trip + (rope_tile ? 0 : r3);
    }
    // global column of the tile's column L
    auto tile_col = [&](int L) __attribute__((always_inline)) -> int {
        if constexpr (QUP == kQupAbsorb) {
            const int qk = a.q.nope + a.q.rope;
            return rope_tile ? (head0 + (L >> 6)) * qk + a.q.nope + (L & 63) : head0 * qk + L;
        } else {
            return n0 + L;
        }
    };
    const int k_begin = sp * a.k_chunk;
    const int nsl = (min(a.K, k_begin + a.k_chunk) - k_begin) / kWKS;   // whole slices
    const int rows_a = min(kWBM, a.M - m0);

    // ---- staging: wave w loads A rows 32w .. 32w+31 (four loads of 8 rows x 128 B) and W
    // rows w*kLoadsB*kRowsPerLoadB .. of each slice (loads of kRowsPerLoadB rows)
    const uint32_t lds0 = lds_addr(smem);
    const uint64_t a_base = reinterpret_cast<uint64_t>(a.A + g * a.sAg + (int64_t)m0 * a.lda);
    const uint64_t b_base = reinterpret_cast<uint64_t>(
        a.B + g * a.sBg + (QUP == kQupAbsorb ? 0 : NT ? (int64_t)n0 * a.ldb : n0));
    uint32_t a_voff[kWLoadsA], b_voff[kLoadsB];
    #pragma unroll
    for (int q = 0; q < kWLoadsA; ++q) {
        const int row = 32 * wave + 8 * q + (lane >> 3);
        a_voff[q] = (uint32_t)row * (uint32_t)a.lda * 2u + 16u * ((lane & 7) ^ ((row >> 1) & 7));
    }
    #pragma unroll
    for (int q = 0; q < kLoadsB; ++q) {
        const int r = (wave * kLoadsB + q) * kRowsPerLoadB + lane / (kBRow / 16);
        const int pos = lane % (kBRow / 16);
        const int sw = BN >= 128 ? 4 * (r & 3) : 4 * ((r >> 1) & 1);
        if constexpr (NT) {
            // NT: W row n (K-contiguous) staged like an A row: 8 rows x 128 bytes per load,
            // chunk c of row n at c ^ ((n >> 1) & 7)
            const int n = (BN / 4) * wave + 8 * q + (lane >> 3);
            b_voff[q] = (uint32_t)n * (uint32_t)a.ldb * 2u + 16u * ((lane & 7) ^ ((n >> 1) & 7));
        } else if constexpr (QUP == kQupAbsorb)
            b_voff[q] = (uint32_t)r * (uint32_t)a.ldb * 2u + 2u * (uint32_t)tile_col(8 * (pos ^ sw));
        else
            b_voff[q] = (uint32_t)r * (uint32_t)a.ldb * 2u + 16u * (pos ^ sw);
    }
    // valid bytes of a slice: A rows below rows_a, all 64 W rows (whole slices)
    const uint32_t a_bytes = (uint32_t)(rows_a - 1) * (uint32_t)a.lda * 2u + 128u;
    const uint32_t b_bytes = NT ? (uint32_t)(BN - 1) * (uint32_t)a.ldb * 2u + 128u
                                : (uint32_t)(kWKS - 1) * (uint32_t)a.ldb * 2u +
                                      (QUP == kQupAbsorb ? 2u * (uint32_t)a.N : (uint32_t)kBRow);
    // kQupAbsorb, nope tiles: W_uk[head0] (nope = 128 rows x kv, rows kv apart) in slices of
    // 64 rows x 128 columns in the W layout of a ring stage, pass p's two K halves kh.  Pass 0
    // goes into the table's space before the ring starts; pass p >= 1 takes the place of the
    // ring's slice nsl + p - 1, past the K range (a stage the ring has just freed: its A
    // part holds kh 0, its W part kh 1), which keeps the per-slice load count.  Passes past
    // kv / 128 load zeros.  The tile's q_nope block goes into the stage of the last slice.
    auto wuk_slot = [&](int p, int kh) __attribute__((always_inline)) -> uint32_t {
        return (p == 0 ? (uint32_t)(NS * kStage) : (uint32_t)((nsl + p - 1) % NS) * kStage) +
               (uint32_t)kBStage * kh;
    };
    auto issue_wuk = [&](int p, int kh) __attribute__((always_inline)) {
        if constexpr (QUP == kQupAbsorb) {
            const int kv = a.q.kv;
            const bool live = p < (kv >> 7);
            const v4i rw = rsrc_span(reinterpret_cast<uint64_t>(
                                         static_cast<const uint16_t*>(a.q.w_uk) +
                                         (int64_t)head0 * a.q.nope * kv),
                                     0, live ? (uint32_t)(a.q.nope * kv * 2) : 0u);
            #pragma unroll
            for (int q = 0; q < kLoadsB; ++q) {
                const int r = (wave * kLoadsB + q) * kRowsPerLoadB + lane / (kBRow / 16);
                const int pos = lane % (kBRow / 16);
                const uint32_t voff = (uint32_t)r * (uint32_t)kv * 2u + 16u * (pos ^ (4 * (r & 3)));
                dma16(rw, __builtin_amdgcn_readfirstlane(
                              lds0 + wuk_slot(p, kh) + (uint32_t)((wave * kLoadsB + q) * kRowsPerLoadB) * kBRow),
                      voff, live ? (uint32_t)(kh * kWKS * kv * 2 + 256 * p) : 0u);
            }
        }
    };
    auto issue_slice = [&](int s) __attribute__((always_inline)) {
        if constexpr (QUP == kQupAbsorb) {
            static_assert(2 * kLoadsB == kLoads, "a W_uk pass issues a slice's load count");
            if (!rope_tile && s >= nsl) {
                issue_wuk(s - nsl + 1, 0);
                issue_wuk(s - nsl + 1, 1);
                return;
            }
        }
        const uint32_t st = lds0 + (uint32_t)(s % NS) * kStage;
        const int k = k_begin + s * kWKS;
        const bool live = s < nsl;
        const v4i ra = rsrc_span(a_base + 2ull * (uint64_t)k, 0, live ? a_bytes : 0u);
        const v4i rb = rsrc_span(b_base + 2ull * (uint64_t)k * (NT ? 1ull : (uint64_t)a.ldb), 0,
                                 live ? b_bytes : 0u);
        #pragma unroll
        for (int q = 0; q < kWLoadsA; ++q)
            dma16(ra, __builtin_amdgcn_readfirstlane(st + (uint32_t)(32 * wave + 8 * q) * 128u),
                  a_voff[q], 0);
        #pragma unroll
        for (int q = 0; q < kLoadsB; ++q)
            dma16(rb, __builtin_amdgcn_readfirstlane(
                          NT ? st + kWAStage + (uint32_t)((BN / 4) * wave + 8 * q) * 128u
                             : st + kWAStage + (uint32_t)((wave * kLoadsB + q) * kRowsPerLoadB) * kBRow),
                  b_voff[q], 0);
    };

    // ---- fragments: wave (wm, wn) covers rows 64wm .. +63 and columns (BN/2)wn .. +BN/2-1
    const int wm = wave >> 1, wn = wave & 1;
    // A fragment of row block rb, K step kt: row 64wm + 32rb + l%32, bytes 32kt + 16(l/32)
    uint32_t a_rd[2];
    #pragma unroll
    for (int rb = 0; rb < 2; ++rb) {
        const int row = 64 * wm + 32 * rb + (lane & 31);
        a_rd[rb] = (uint32_t)row * 128u + 16u * ((lane >> 5) ^ ((row >> 1) & 7));
    }
    // W fragment half p of column block cb, K step kt: lane 16G + 4q + i reads row
    // 16kt + 8(G/2) + 4p + q, columns (BN/2)wn + 32cb + 16(G%2) + 4i .. +3
    const int G = lane >> 4, q4 = (lane >> 2) & 3, i4 = lane & 3;
    // (NT: W row n = (BN/2)wn + 32cb + l%32 is read like an A row, bytes 32kt + 16(l/32))
    uint32_t b_rd[CB];
    #pragma unroll
    for (int cb = 0; cb < CB; ++cb) {
        if constexpr (NT) {
            const int n = (BN / 2) * wn + 32 * cb + (lane & 31);
            b_rd[cb] = kWAStage + (uint32_t)n * 128u + 16u * ((lane >> 5) ^ ((n >> 1) & 7));
        } else {
            const int chunk = ((BN / 2) * wn + 32 * cb + 16 * (G & 1) + 4 * i4) / 8;
            const int sw = BN >= 128 ? 4 * q4 : 4 * (q4 >> 1);
            b_rd[cb] = kWAStage + (uint32_t)(8 * (G >> 1) + q4) * kBRow + 16u * (chunk ^ sw) + 8u * (i4 & 1);
        }
    }
    typedef short v4s __attribute__((ext_vector_type(4)));
    typedef __attribute__((address_space(3))) v4s lds_v4s;
    auto b_frag = [&](uint32_t st, int kt, int cb) __attribute__((always_inline)) {
        if constexpr (NT) {
            return *reinterpret_cast<const v4u*>(smem + st + (b_rd[cb] ^ (32u * kt)));
        } else {
            const uint32_t o = st + b_rd[cb] + (uint32_t)(16 * kt) * kBRow;
            const v4s lo = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_v4s*)(smem + o));
            const v4s hi = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_v4s*)(smem + o + 4 * kBRow));
            return __builtin_bit_cast(v4u, __builtin_shufflevector(lo, hi, 0, 1, 2, 3, 4, 5, 6, 7));
        }
    };
    auto a_frag = [&](uint32_t st, int kt, int rb) __attribute__((always_inline)) {
        // chunk 2kt + l/32 at (2kt + l/32) ^ s: a_rd holds (l/32) ^ s, and 2kt ^ s = 2kt ^
        // (s & 6) ^ (s & 1) -- the XOR with 32kt only touches bits 5-6 of the offset
        return *reinterpret_cast<const v4u*>(smem + st + (a_rd[rb] ^ (32u * kt)));
    };

    v16f acc[2][CB];
    #pragma unroll
    for (int rb = 0; rb < 2; ++rb)
        #pragma unroll
        for (int cb = 0; cb < CB; ++cb) acc[rb][cb] = v16f{};

    // QUP: a tile with rope columns loads its rows' cos / sin table (2a-n wrote it) into LDS
    // ahead of the ring, 1 KB = 1024 / (8 half) rows per load; rows past M read zeros.  The
    // first slice's wait covers these loads too (vmcnt retires in order).
    bool has_rope = false;
    if constexpr (QUP) {
        const int qk = a.q.nope + a.q.rope, half = a.q.rope >> 1;
        if constexpr (QUP == kQupAbsorb) {
            has_rope = rope_tile;
        } else {
            #pragma unroll
            for (int c = 0; c < BN; c += 32) has_rope |= (n0 + c) % qk >= a.q.nope;
        }
        if (has_rope) {
            const v4i rt = rsrc_span(reinterpret_cast<uint64_t>(a.q.cos_sin + 2 * (int64_t)m0 * half),
                                     0, (uint32_t)(rows_a * half * 8));
            for (int b = wave; b < half; b += 4)   // kWBM * half * 8 bytes = half KB
                dma16(rt, __builtin_amdgcn_readfirstlane(lds0 + NS * kStage + 1024u * b),
                      1024u * b + 16u * lane, 0);
        }
    }
    if constexpr (QUP == kQupAbsorb) {
        if (!rope_tile) {
            issue_wuk(0, 0);
            issue_wuk(0, 1);
        }
    }
    #pragma unroll
    for (int s = 0; s < NS - 1; ++s) issue_slice(s);

    #pragma unroll 1
    for (int s = 0; s < nsl; ++s) {
        wait_vm<(NS - 2) * kLoads>();   // slice s has landed (the NS - 2 after it may not)
        lds_barrier();                    // every wave's part of it; slice s-1 is consumed
        issue_slice(s + NS - 1);          // into stage (s - 1) % NS
        const uint32_t st = (uint32_t)(s % NS) * kStage;
        #pragma unroll
        for (int kt = 0; kt < kWKS / 16; ++kt) {
            v4u af[2], bf[CB];
            #pragma unroll
            for (int rb = 0; rb < 2; ++rb) af[rb] = a_frag(st, kt, rb);
            #pragma unroll
            for (int cb = 0; cb < CB; ++cb) bf[cb] = b_frag(st, kt, cb);
            #pragma unroll
            for (int rb = 0; rb < 2; ++rb)
                #pragma unroll
                for (int cb = 0; cb < CB; ++cb) acc[rb][cb] = Mma<TL>::sub(af[rb], bf[cb], 0, acc[rb][cb]);
        }
    }
    wait_vm<0>();   // the zero loads past the range have landed

    if constexpr (QUP == kQupAbsorb) {
        if (!rope_tile) {
            // ---- 2c for head0 on this tile's rows: q_abs = q_nope16 @ W_uk[head0]
            const int kv = a.q.kv, passes = kv >> 7;
            __syncthreads();   // every wave is done with the ring; W_uk has landed
            // A2: the 16-bit q_nope block, K slice kh = columns 64 kh .. at 16 KB kh of the
            // last slice's stage, in the A layout of the ring.  Lane pairs (c, c ^ 1) swap
            // values (DPP) so that each lane writes one dword: the even lane row R(e), the
            // odd lane row R(e + 1).
            const uint32_t a2 = (uint32_t)((nsl + NS - 1) % NS) * kStage;
            const bool odd = lane & 1;
            #pragma unroll
            for (int rb = 0; rb < 2; ++rb)
                #pragma unroll
                for (int cb = 0; cb < CB; ++cb) {
                    const int k = (32 * cb + (lane & 31)) & ~1;
                    #pragma unroll
                    for (int e = 0; e < 16; e += 2) {
                        const float x0 = acc[rb][cb][e], x1 = acc[rb][cb][e + 1];
                        const float p0 = dpp_move<0xB1>(x0), p1 = dpp_move<0xB1>(x1);
                        const int row = 64 * wm + 32 * rb + acc_row(odd ? e + 1 : e, lane);
                        const uint32_t w = odd ? Half<TL>::pack2(p1, x1) : Half<TL>::pack2(x0, p0);
                        const uint32_t off = a2 + (uint32_t)kWAStage * wn + (uint32_t)row * 128u +
                                             16u * ((k >> 3) ^ ((row >> 1) & 7)) + 2u * (k & 7);
                        *reinterpret_cast<uint32_t*>(smem + off) = w;
                    }
                }
            __syncthreads();
            uint16_t* const qabs = static_cast<uint16_t*>(a.q.q_abs) + (int64_t)head0 * kv;
            const int64_t ld_abs = (int64_t)a.q.H * kv;
            #pragma unroll 1
            for (int p = 0; p < passes; ++p) {
                v16f acc2[2][CB];
                #pragma unroll
                for (int rb = 0; rb < 2; ++rb)
                    #pragma unroll
                    for (int cb = 0; cb < CB; ++cb) acc2[rb][cb] = v16f{};
                #pragma unroll
                for (int kh = 0; kh < 2; ++kh)
                    #pragma unroll
                    for (int kt = 0; kt < kWKS / 16; ++kt) {
                        v4u af[2], bf[CB];
                        #pragma unroll
                        for (int rb = 0; rb < 2; ++rb) af[rb] = a_frag(a2 + (uint32_t)kWAStage * kh, kt, rb);
                        #pragma unroll
                        for (int cb = 0; cb < CB; ++cb) bf[cb] = b_frag(wuk_slot(p, kh) - kWAStage, kt, cb);
                        #pragma unroll
                        for (int rb = 0; rb < 2; ++rb)
                            #pragma unroll
                            for (int cb = 0; cb < CB; ++cb)
                                acc2[rb][cb] = Mma<TL>::sub(af[rb], bf[cb], 0, acc2[rb][cb]);
                    }
                #pragma unroll
                for (int rb = 0; rb < 2; ++rb)
                    #pragma unroll
                    for (int cb = 0; cb < CB; ++cb) {
                        uint16_t* const dst = qabs + 128 * p + (BN / 2) * wn + 32 * cb + ((lane & 31) & ~1);
                        #pragma unroll
                        for (int e = 0; e < 16; e += 2) {
                            const float x0 = acc2[rb][cb][e], x1 = acc2[rb][cb][e + 1];
                            const float p0 = dpp_move<0xB1>(x0), p1 = dpp_move<0xB1>(x1);
                            const int row = 64 * wm + 32 * rb + acc_row(odd ? e + 1 : e, lane);
                            const uint32_t w = odd ? Half<TL>::pack2(p1, x1) : Half<TL>::pack2(x0, p0);
                            if (row < rows_a)
                                *reinterpret_cast<uint32_t*>(dst + (int64_t)(m0 + row) * ld_abs) = w;
                        }
                    }
            }
            return;
        }
    }

    if constexpr (QUP) {
        // ---- fused 2a2 epilogue: nope blocks to q_nope, rope blocks rotated to q_rope.
        // Every 32-column block lies inside one head's nope or rope part (nope, rope and
        // the block start are multiples of 32); the pair partner of column c is column c ^ 1,
        // the neighbouring lane.  cos / sin come from the table 2a-n wrote for these rows,
        // staged in LDS at the start.
        const int half = a.q.rope >> 1;
        const int qk = a.q.nope + a.q.rope;
        if (has_rope) __syncthreads();   // every wave's table loads (uniform per workgroup)
        const int64_t ld_nope = (int64_t)a.q.H * a.q.nope, ld_rope = (int64_t)a.q.H * a.q.rope;
        #pragma unroll
        for (int rb = 0; rb < 2; ++rb)
            #pragma unroll
            for (int cb = 0; cb < CB; ++cb) {
                const int c0 = tile_col((BN / 2) * wn + 32 * cb);
                const int h = c0 / qk, j0 = c0 - h * qk;
                if (j0 < a.q.nope) {
                    uint16_t* dst = static_cast<uint16_t*>(a.q.q_nope) + (int64_t)h * a.q.nope + j0 + (lane & 31);
                    #pragma unroll
                    for (int e = 0; e < 16; ++e) {
                        const int row = 64 * wm + 32 * rb + acc_row(e, lane);
                        if (row < rows_a)
                            dst[(int64_t)(m0 + row) * ld_nope] = (uint16_t)Half<TL>::bits(acc[rb][cb][e]);
                    }
                } else {
                    const int r = j0 - a.q.nope + (lane & 31);   // rope column of the head
                    const int i = r >> 1;
                    uint16_t* dst = static_cast<uint16_t*>(a.q.q_rope) + (int64_t)h * a.q.rope + r;
                    #pragma unroll
                    for (int e = 0; e < 16; ++e) {
                        const float own = acc[rb][cb][e];
                        const float other = dpp_move<0xB1>(own);   // lane ^ 1
                        const int row = 64 * wm + 32 * rb + acc_row(e, lane);
                        if (row < rows_a) {
                            const v2f t = *reinterpret_cast<const v2f*>(
                                smem + NS * kStage + 8 * (row * half + i));
                            const float c = t[0], sn = t[1];
                            const float v = (lane & 1) ? rope_odd(other, own, c, sn) : rope_even(own, other, c, sn);
                            dst[(int64_t)(m0 + row) * ld_rope] = (uint16_t)Half<TL>::bits(v);
                        }
                    }
                }
            }
        return;
    }

    // ---- epilogue: fp32 C, C in the storage format, or this split's partials
    if (a.C16) {   // split == 1; lane pairs (c, c ^ 1) swap values so each lane stores a dword
        uint16_t* const c16 = a.C16 + (int64_t)g * a.sCg;
        const bool odd = lane & 1;
        #pragma unroll
        for (int rb = 0; rb < 2; ++rb)
            #pragma unroll
            for (int cb = 0; cb < CB; ++cb) {
                uint16_t* const dst = c16 + n0 + (BN / 2) * wn + 32 * cb + ((lane & 31) & ~1);
                #pragma unroll
                for (int e = 0; e < 16; e += 2) {
                    const float x0 = acc[rb][cb][e], x1 = acc[rb][cb][e + 1];
                    const float p0 = dpp_move<0xB1>(x0), p1 = dpp_move<0xB1>(x1);
                    const int row = 64 * wm + 32 * rb + acc_row(odd ? e + 1 : e, lane);
                    const uint32_t w = odd ? Half<TL>::pack2(p1, x1) : Half<TL>::pack2(x0, p0);
                    if (row < rows_a) *reinterpret_cast<uint32_t*>(dst + (int64_t)(m0 + row) * a.ldc) = w;
                }
            }
        return;
    }
    float* out;
    int64_t ld;
    if (a.split > 1) {
        out = a.ws + (int64_t)sp * a.ws_split + (int64_t)g * a.M * a.N;
        ld = a.N;
    } else {
        out = a.C + (int64_t)g * a.sCg;
        ld = a.ldc;
    }
    #pragma unroll
    for (int rb = 0; rb < 2; ++rb)
        #pragma unroll
        for (int cb = 0; cb < CB; ++cb)
            #pragma unroll
            for (int e = 0; e < 16; ++e) {
                const int row = 64 * wm + 32 * rb + acc_row(e, lane);
                if (row < rows_a)
                    out[(int64_t)(m0 + row) * ld + n0 + (BN / 2) * wn + 32 * cb + (lane & 31)] =
                        acc[rb][cb][e];
            }
}

// Stage counts per column tile: 256 columns x 3 stages (144 KB of LDS); 128 columns x 4
// stages (128 KB, one workgroup per CU) or 3 (96 KB); 64 columns x 3 (72 KB, two per CU), 4
// or 6 stages (96 / 144 KB).  The fused 2a2 epilogues add 32 KB for the RoPE table (160 KB
// at 128 x 4; not with 64 x 6 or 256 x 3); the one that also does 2c runs at 128 x 4 only.
template <typename TL, int QUP>
hipError_t launch_wgemm_t(const WArgs& a, const GemmPlan& plan, dim3 grid, dim3 block,
                          hipStream_t stream) {
    if constexpr (QUP == kQupAbsorb) {
        if (plan.bn == 128 && plan.stages == 4)
            hipLaunchKernelGGL((wgemm_kernel<TL, 128, 4, 1, kQupAbsorb>), grid, block, 0, stream, a);
        else
            return hipErrorInvalidValue;
    } else if (plan.bn == 256 && plan.stages == 3 && !QUP) {   // 144 KB: no room for the table
        hipLaunchKernelGGL((wgemm_kernel<TL, 256, 3, 1, kQupNone>), grid, block, 0, stream, a);
    } else if (plan.bn == 128 && plan.stages == 4) {
        hipLaunchKernelGGL((wgemm_kernel<TL, 128, 4, 1, QUP>), grid, block, 0, stream, a);
    } else if (plan.bn == 128 && plan.stages == 3) {
        hipLaunchKernelGGL((wgemm_kernel<TL, 128, 3, 1, QUP>), grid, block, 0, stream, a);
    } else if (plan.bn == 64 && plan.stages == 3) {
        hipLaunchKernelGGL((wgemm_kernel<TL, 64, 3, 2, QUP>), grid, block, 0, stream, a);
    } else if (plan.bn == 64 && plan.stages == 4) {
        hipLaunchKernelGGL((wgemm_kernel<TL, 64, 4, 1, QUP>), grid, block, 0, stream, a);
    } else if (plan.bn == 64 && plan.stages == 6 && !QUP) {   // no room for the table
        hipLaunchKernelGGL((wgemm_kernel<TL, 64, 6, 1, kQupNone>), grid, block, 0, stream, a);
    } else {
        return hipErrorInvalidValue;
    }
    return hipGetLastError();
}

// NT (W rows K-contiguous): 128 or 64 columns, 3 or 4 stages, no fused epilogue.
template <typename TL>
hipError_t launch_wgemm_nt(const WArgs& a, const GemmPlan& plan, dim3 grid, dim3 block,
                           hipStream_t stream) {
    if (plan.bn == 128 && plan.stages == 4)
        hipLaunchKernelGGL((wgemm_kernel<TL, 128, 4, 1, kQupNone, true>), grid, block, 0, stream, a);
    else if (plan.bn == 128 && plan.stages == 3)
        hipLaunchKernelGGL((wgemm_kernel<TL, 128, 3, 1, kQupNone, true>), grid, block, 0, stream, a);
    else if (plan.bn == 64 && plan.stages == 4)
        hipLaunchKernelGGL((wgemm_kernel<TL, 64, 4, 1, kQupNone, true>), grid, block, 0, stream, a);
    else if (plan.bn == 64 && plan.stages == 3)
        hipLaunchKernelGGL((wgemm_kernel<TL, 64, 3, 2, kQupNone, true>), grid, block, 0, stream, a);
    else
        return hipErrorInvalidValue;
    return hipGetLastError();
}

}  // namespace

bool wgemm_supported(const GemmProblem& p, int bn, int split) {
    const OutType own16 = p.f16 ? kOutF16 : kOutBF16;
    return p.half && !p.a_f32 && p.amode == kAPlain &&
           (p.out_type == kOutF32 || split > 1 || p.out_type == own16) && split >= 1 &&
           !p.k_len && !p.b_pages && (bn == 64 || bn == 128 || (bn == 256 && !p.b_nt)) &&
           p.N % bn == 0 && p.K % kWKS == 0 && p.lda >= kWKS &&
           (p.b_nt ? p.ldb >= p.K : p.ldb >= bn) && p.M > 0 && p.G >= 1 &&
           // 16-byte aligned rows and groups for the 16-byte loads; 4-byte 16-bit C rows
           p.lda % 8 == 0 && p.ldb % 8 == 0 && p.sAg % 8 == 0 && p.sBg % 8 == 0 &&
           (p.out_type == kOutF32 || split > 1 || (p.ldc % 2 == 0 && p.sCg % 2 == 0)) &&
           // 32-bit buffer offsets within a tile: 128 A rows, 64 W rows (NT: bn W rows)
           (int64_t)kWBM * p.lda * 2 < kRsrcRange &&
           (int64_t)(p.b_nt ? bn : kWKS) * p.ldb * 2 < kRsrcRange;
}

bool qup_supported(const GemmProblem& p, const QUpEpilogue& q, const GemmPlan& plan) {
    const bool rope_ok = p.half && p.G == 1 && !p.b_nt && p.out_type == kOutF32 && q.H > 0 && q.nope > 0 && q.nope % 32 == 0 &&
                         q.rope > 0 && q.rope % 32 == 0 && q.rope <= 64 &&
                         (int64_t)p.N == (int64_t)q.H * (q.nope + q.rope) && q.q_rope && q.cos_sin;
    if (!q.w_uk) return rope_ok && q.q_nope;
    // with 2c: one head's nope columns per 128-column tile, two heads' rope columns per
    // tile, W_uk rows and q_abs rows 16-byte / 4-byte aligned, kv / 128 passes of 32 KB
    return rope_ok && q.q_abs && plan.bn == 128 && plan.stages == 4 && q.nope == 128 &&
           q.rope == 64 && q.H % 2 == 0 && q.kv > 0 && q.kv % 128 == 0 && q.kv <= 512 &&
           (reinterpret_cast<uintptr_t>(q.w_uk) & 15) == 0 &&
           (reinterpret_cast<uintptr_t>(q.q_abs) & 3) == 0;
}

bool wgemm_aligned(const GemmProblem& p) {
    return (reinterpret_cast<uintptr_t>(p.A) & 15) == 0 && (reinterpret_cast<uintptr_t>(p.B) & 15) == 0 &&
           (reinterpret_cast<uintptr_t>(p.C) & 3) == 0;
}

hipError_t launch_wgemm(const GemmProblem& p, const GemmPlan& plan, float* partials,
                        hipStream_t stream) {
    if (!wgemm_supported(p, plan.bn, plan.split) || !wgemm_aligned(p) || plan.k_chunk <= 0 ||
        plan.k_chunk % kWKS != 0 || (int64_t)plan.k_chunk * plan.split < p.K)
        return hipErrorInvalidValue;
    WArgs a;
    a.A = static_cast<const uint16_t*>(p.A); a.lda = p.lda; a.sAg = p.sAg;
    a.B = static_cast<const uint16_t*>(p.B); a.ldb = p.ldb; a.sBg = p.sBg;
    const bool c16 = p.out_type != kOutF32 && plan.split == 1;
    a.C = c16 ? nullptr : static_cast<float*>(p.C); a.ldc = p.ldc; a.sCg = p.sCg;
    a.C16 = c16 ? static_cast<uint16_t*>(p.C) : nullptr;
    a.ws = partials; a.ws_split = (int64_t)p.G * p.M * p.N;
    a.M = p.M; a.N = p.N; a.K = p.K; a.G = p.G;
    a.split = plan.split; a.k_chunk = plan.k_chunk;
    a.tiles_m = (p.M + kWBM - 1) / kWBM;
    a.tiles_n = p.N / plan.bn;
    if (plan.split > 1 && !partials) return hipErrorInvalidValue;
    const int64_t blocks = (int64_t)a.tiles_m * a.tiles_n * a.split * a.G;
    if (blocks <= 0 || blocks > 0x7fffffff) return hipErrorInvalidValue;
    const dim3 grid((unsigned)blocks), block(kWThreads);
    if (p.qup) {
        if (plan.split != 1 || !qup_supported(p, *p.qup, plan)) return hipErrorInvalidValue;
        a.q = *p.qup;
        if (a.q.w_uk) {
            if (p.f16) return launch_wgemm_t<f16_t, kQupAbsorb>(a, plan, grid, block, stream);
            return launch_wgemm_t<bf16_t, kQupAbsorb>(a, plan, grid, block, stream);
        }
        if (p.f16) return launch_wgemm_t<f16_t, kQupRope>(a, plan, grid, block, stream);
        return launch_wgemm_t<bf16_t, kQupRope>(a, plan, grid, block, stream);
    }
    if (p.b_nt) {
        if (p.f16) return launch_wgemm_nt<f16_t>(a, plan, grid, block, stream);
        return launch_wgemm_nt<bf16_t>(a, plan, grid, block, stream);
    }
    if (p.f16) return launch_wgemm_t<f16_t, kQupNone>(a, plan, grid, block, stream);
    return launch_wgemm_t<bf16_t, kQupNone>(a, plan, grid, block, stream);
}

}  // namespace mla
