// Work list of a ragged batch for the fused attention pass: the rules that cut each
// sequence's keys into chunks and order the chunks for dispatch.
//
// flash_worklist_kernel (flash.hip) builds the list on the device from seq_lens, with one
// workgroup whose threads each own a contiguous run of batches; every per-batch decision
// it makes is one of the functions below.  wl_build_serial() applies the same functions
// in one thread, in batch order: it is what a CPU harness drives over adversarial length
// distributions to check the list's invariants (at most max_items items, every (batch,
// chunk) listed exactly once, partial slots inside the sized range, the keys of every
// sequence covered exactly once).  This header includes no HIP header, so a plain C++
// compiler builds it.
//
// List layout (ints): [0] item count, [1] chunk keys, first partial slot [B], chunk count
// [B], then the items {b, c}: every full-length chunk first (batch order), then the shorter
// last chunks, longest first (a counting sort over kWlBuckets length buckets).
#pragma once

#include <stdint.h>

#include "gpu_shape.h"

#if defined(__HIPCC__)
#define MLA_HD __host__ __device__ inline
#else
#define MLA_HD inline
#endif

namespace mla {

constexpr int kWlHead = 2;
// A ragged list spreads the total key count over kWlPerCu workgroups per CU (fp32) or
// kWlPerCu16 (bf16, fp16 and the fp8 cache).  At B=128 with lengths uniform in [1, 4989],
// fp32: 1 per CU took 1185 us, 2: 950, 3: 901, 4: 870-905, 6: 926, 8: 907 (more pieces
// shorten the tail; each piece costs its Q load and partials).  16-bit: 1 per CU took
// 150.5 us, 2: 165.7, 3: 185.4, 4: 202.4 (fp8 cache 186.3 / 208.1 / 229.9 / 254.2; one
// sequence of 4989 keys per seven of 300: bf16 95.7 us at 1 against 153.9 at 4): a 16-bit
// key block is ~5x shorter than an fp32 one, so a piece's fixed cost weighs ~5x more.
// The list is sized for the larger kWlPerCu.
constexpr int kWlPerCu = 4;
constexpr int kWlPerCu16 = 1;
static_assert(kWlPerCu16 <= kWlPerCu, "the list is sized for kWlPerCu pieces per CU");
constexpr int kWlBuckets = 256;     // length buckets of the last-chunk counting sort
constexpr int kWlThreads = 256;     // threads of the device builder

MLA_HD int wl_min(int a, int b) { return a < b ? a : b; }
MLA_HD int wl_max(int a, int b) { return a > b ? a : b; }

MLA_HD int wl_ints(int B, int max_items) { return kWlHead + 2 * B + 2 * max_items; }

// Items of a balanced list: at most kWlPerCu * CUs / row_tiles + B (either chunk rule of
// wl_initial_chunk), rounded up to a whole number per XCD.
MLA_HD int wl_max_items(int B, int row_tiles) {
    return (kWlPerCu * kNumCUs / row_tiles + B + 1 + kNumXCDs - 1) / kNumXCDs * kNumXCDs;
}

// Keys per split of a dense batch of Sk keys, base = B * row_tiles workgroups per split.
// Below one workgroup per CU: as many splits as fit in one round of CUs (floor(CUs / base)),
// at least one key block per split.  (Measured at B=1: Sk=512 takes 25.0 us in 32 one-block
// splits against 33.0 us in 8 four-block ones; at Sk=4989 the split size leaves the time
// unchanged.  Rounding the split count to nearest instead put B=5, Sk=4989 at 26 splits of
// 12 blocks, 260 workgroups, and the 4 of the second round took the attention from ~100
// to 154 us.)
// From one workgroup per CU up, the rounds of workgroups set the time, and a base just
// past a multiple of the CU count leaves the last round nearly empty (B=132 decode: 264
// workgroups run as two rounds of one).  A split s of 1..4 is taken when its rounds of
// shorter workgroups plus the merge of s partial rows cost less:
//   ceil(base s / CUs) (ceil(blocks / s) + F)   block times,
//   + rows s 2,056 bytes at ~5 TB/s in block times (rows = 64 base),
// with a block ~4.2 us per workgroup and F = 4 in fp32 (16 keys), ~0.9 us and F = 20 in
// 16-bit (32 keys; its queries, ring fill, key-half merge and fp32 partial rows weigh more
// against the short blocks).  Both fitted to measured sweeps of s = 1..4 at B = 128..240,
// Sq = 1 and B = 96, 132 at Sq = 4 (fp32 B = 132: 2,701 -> 1,743 us at s = 4; bf16 B = 200
// stays at s = 1, 325 us against 380 at s = 3).  Integers, so the host planner and the
// device's work list decide alike; a larger split must win by 3%.
MLA_HD int dense_keys_per_split(int Sk, int base, int block_keys) {
    const int blocks = (Sk + block_keys - 1) / block_keys;
    if (base < kNumCUs) {
        int split = kNumCUs / base;
        split = wl_min(wl_max(split, 1), blocks);
        return (blocks + split - 1) / split * block_keys;
    }
    // bytes the merge moves in one block time: 5e12 B/s x 4.2e-6 s (fp32), x 0.9e-6 s (16-bit)
    const long long bytes_per_block = block_keys == 16 ? 21000000LL : 4500000LL;
    const long long fixed = block_keys == 16 ? 4 : 20;
    const long long rows = 64LL * base;
    int best_s = 1;
    long long best = -1;
    for (int s = 1; s <= wl_min(4, blocks); ++s) {
        const long long per = (blocks + s - 1) / s;
        const long long rounds = ((long long)base * s + kNumCUs - 1) / kNumCUs;
        long long cost = rounds * (per + fixed) * 1000;
        if (s > 1) cost += rows * s * 2056LL * 1000 / bytes_per_block;
        if (best < 0 || cost * 100 < best * 97) {
            best = cost;
            best_s = s;
        }
    }
    return (blocks + best_s - 1) / best_s * block_keys;
}

// A sequence's key count as the kernels use it: seq_lens[b] clamped to [0, Sk] (Sk = the
// block table's key span).  A sequence of no keys yields zero output rows.
MLA_HD int wl_len(int v, int Sk) { return v < 0 ? 0 : (v > Sk ? Sk : v); }

// Chunks of a sequence of L keys (a sequence of no keys still gets one, which writes its
// zero rows), its full-length chunks, and whether its last chunk is shorter than `chunk`.
MLA_HD int wl_chunk_count(int L, int chunk) { return wl_max(1, (L + chunk - 1) / chunk); }
MLA_HD int wl_full_count(int L, int chunk) { return L / chunk; }
MLA_HD int wl_has_short(int L, int chunk) { return (L % chunk != 0 || L == 0) ? 1 : 0; }

// Length bucket of a sequence's short last chunk: bucket 0 holds the longest remainders.
MLA_HD int wl_bucket(int L, int chunk) {
    const int r = L % chunk;
    return (int)(((long long)(chunk - 1 - r) * kWlBuckets) / chunk);
}

// Chunk before the fit check, from the batch's total, minimum and maximum key counts:
//   every sequence the same length L -> the dense plan's keys per split for L, so the list
//     reproduces the dense launch exactly (same key ranges, same merge order);
//   otherwise -> the total key count spread over kWlPerCu (fp32, 16-key blocks) or
//     kWlPerCu16 (16-bit, 32-key blocks) workgroups per CU (a multiple of the key block,
//     so a wave's keys never straddle a page; at least 4 blocks; at most the key span
//     rounded up to a block).
MLA_HD int wl_initial_chunk(long long tot, int mn, int mx, int B, int Sk, int row_tiles,
                            int block_keys) {
    if (mn == mx) return dense_keys_per_split(wl_max(1, mx), B * row_tiles, block_keys);
    const long long wgs = (long long)(block_keys == 16 ? kWlPerCu : kWlPerCu16) * kNumCUs;
    const long long want = (tot * row_tiles + wgs - 1) / wgs;
    const long long cap = (long long)(Sk + block_keys - 1) / block_keys * block_keys;
    long long chunk = (want + block_keys - 1) / block_keys * block_keys;
    chunk = chunk < cap ? chunk : cap;
    return wl_max((int)chunk, 4 * block_keys);
}

// The list must fit max_items (the partial slots and the grid are sized for it).  A chunk
// whose list does not is doubled until it does: a chunk of at least Sk keys gives one item
// per sequence, B < max_items.
MLA_HD bool wl_fits(long long total, int max_items, int chunk, int Sk) {
    return total <= max_items || chunk >= Sk;
}

// Equal lengths: every sequence has nf full chunks (and one short chunk when n > nf), so
// item it is computed directly: full items batch-major, then the short chunks.
MLA_HD void wl_equal_item(int it, int B, int nf, int* b, int* c) {
    if (it < B * nf) {
        *b = it / nf;
        *c = it % nf;
    } else {
        *b = it - B * nf;
        *c = nf;
    }
}

// First batch of builder thread tid (batches [first(tid), first(tid + 1)) per thread).
MLA_HD int wl_thread_first(int tid, int B) {
    const int per = (B + kWlThreads - 1) / kWlThreads;
    return wl_min(B, tid * per);
}

// The list in one thread, batch by batch, with the functions above (the device builder's
// order among last chunks of one bucket is its LDS atomics'; here it is batch order).
// Returns the item count.
inline int wl_build_serial(const int* seq_lens, int B, int Sk, int row_tiles, int block_keys,
                           int max_items, int* wl) {
    long long tot = 0;
    int mn = 0x7fffffff, mx = 0;
    for (int b = 0; b < B; ++b) {
        const int L = wl_len(seq_lens[b], Sk);
        tot += L;
        mn = wl_min(mn, L);
        mx = wl_max(mx, L);
    }
    int chunk = wl_initial_chunk(tot, mn, mx, B, Sk, row_tiles, block_keys);
    long long total;
    int n_full;
    for (;;) {
        total = 0;
        n_full = 0;
        for (int b = 0; b < B; ++b) {
            const int L = wl_len(seq_lens[b], Sk);
            total += wl_chunk_count(L, chunk);
            n_full += wl_full_count(L, chunk);
        }
        if (wl_fits(total, max_items, chunk, Sk)) break;
        chunk *= 2;
    }
    int* first = wl + kWlHead;
    int* count = first + B;
    int* items = count + B;
    const int n_items = (int)(total < max_items ? total : max_items);
    wl[0] = n_items;
    wl[1] = chunk;
    if (mn == mx) {
        const int n = wl_chunk_count(mx, chunk), nf = wl_full_count(mx, chunk);
        for (int b = 0; b < B; ++b) {
            first[b] = b * n;
            count[b] = n;
        }
        for (int it = 0; it < n_items; ++it) wl_equal_item(it, B, nf, &items[2 * it], &items[2 * it + 1]);
        return n_items;
    }
    int start[kWlBuckets + 1] = {0};
    for (int b = 0; b < B; ++b) {
        const int L = wl_len(seq_lens[b], Sk);
        if (wl_has_short(L, chunk)) ++start[wl_bucket(L, chunk) + 1];
    }
    for (int q = 0; q < kWlBuckets; ++q) start[q + 1] += start[q];
    int slot = 0, fi = 0;
    for (int b = 0; b < B; ++b) {
        const int L = wl_len(seq_lens[b], Sk);
        const int n = wl_chunk_count(L, chunk);
        first[b] = slot;
        count[b] = n;
        slot += n;
        for (int c = 0; c < n; ++c) {
            const bool full = (long long)(c + 1) * chunk <= L;
            const int it = full ? fi++ : n_full + start[wl_bucket(L, chunk)]++;
            if (it < max_items) {
                items[2 * it] = b;
                items[2 * it + 1] = c;
            }
        }
    }
    return n_items;
}

}  // namespace mla
