// MFMA "K step" abstraction shared by the GEMM engine and the scores kernel.
//
// Every K-contiguous LDS row holds 128 bytes of K per slice (32 fp32 or 64 bf16) plus a
// 16-byte pad.  One K step consumes 32 of those bytes: lane l reads the 16 bytes at
// byte 32*step + 16*(l/32) of its row (one ds_read_b128) and feeds
//   fp32: four v_mfma_f32_32x32x2_f32  (4 k values per lane, K = 8 per step)
//   bf16: one   v_mfma_f32_32x32x16_bf16 (8 k values per lane, K = 16 per step)
//   fp16: one   v_mfma_f32_32x32x16_f16  (the same layout)
// Both instructions take row/column l%32 from lane l and split K between the two
// half-waves, and A and B fragments are always read from the same k offsets, so the
// product is exact whatever order the hardware assigns to the k values inside a lane.
// The 32x32 fp32 accumulator layout is the same for both.
#pragma once

#include "common.h"

namespace mla {

typedef uint32_t v4u __attribute__((ext_vector_type(4)));

template <typename TL> struct Mma;

template <> struct Mma<float> {
    static constexpr int kElems = 4;   // elements per 16-byte chunk
    static constexpr int kSlice = 32;  // K elements per 128-byte LDS row slice
    static constexpr int kSub = 4;     // MFMAs per K step
    // MFMA q of a K step.  Callers loop q outermost over independent accumulators, so
    // consecutive MFMAs never depend on each other.
    __device__ static __forceinline__ v16f sub(v4u a, v4u b, int q, v16f c) {
        return __builtin_amdgcn_mfma_f32_32x32x2f32(__uint_as_float(a[q]), __uint_as_float(b[q]),
                                                    c, 0, 0, 0);
    }
};

template <> struct Mma<bf16_t> {
    static constexpr int kElems = 8;
    static constexpr int kSlice = 64;
    static constexpr int kSub = 1;
    __device__ static __forceinline__ v16f sub(v4u a, v4u b, int, v16f c) {
        return __builtin_amdgcn_mfma_f32_32x32x16_bf16(__builtin_bit_cast(v8bf, a),
                                                       __builtin_bit_cast(v8bf, b), c, 0, 0, 0);
    }
};

template <> struct Mma<f16_t> {
    static constexpr int kElems = 8;
    static constexpr int kSlice = 64;
    static constexpr int kSub = 1;
    __device__ static __forceinline__ v16f sub(v4u a, v4u b, int, v16f c) {
        return __builtin_amdgcn_mfma_f32_32x32x16_f16(__builtin_bit_cast(v8h, a),
                                                      __builtin_bit_cast(v8h, b), c, 0, 0, 0);
    }
};

// ---- buffer-resource staging loads --------------------------------------------------
// Tile staging goes through buffer resources (V#: base address and range in SGPRs) with a
// 32-bit per-lane byte offset.  The hardware range-checks every load: an offset at or
// beyond num_records returns zeros without touching memory.  Rows and columns outside a
// tile get the offset kOob, so the staging code is branch-free, and the per-lane offsets
// stay fixed while the scalar base walks the K slices.  Every offset a kernel forms for a
// valid element is below kRsrcRange; the launchers check the leading dimensions for that.
constexpr uint32_t kOob = 0x80000000u;
constexpr int kRsrcRange = 0x7fffffff;

__device__ __forceinline__ __amdgpu_buffer_rsrc_t make_rsrc(const void* base) {
    // dword3 0x00020000: 32-bit data format, as the gfx9 family requires for raw loads
    return __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(base), (short)0, kRsrcRange,
                                             0x00020000);
}
// kOob when x >= lim, else 0 (x >= 0): the sign of x - lim, moved to bit 31 and inverted.
// Written as arithmetic so the compiler keeps it a VALU op instead of splitting the load
// that consumes it into divergent branches, which it does for a select.
__device__ __forceinline__ uint32_t oob_mask(int x, int lim) {
    return ~(uint32_t)(x - lim) & kOob;
}
// 16 bytes at byte offset `off`.  Callers consume all four words: LLVM narrows a b128
// buffer load whose leading words are unused to a dword load without moving the offset.
__device__ __forceinline__ v4u load16(__amdgpu_buffer_rsrc_t r, uint32_t off) {
    return __builtin_amdgcn_raw_buffer_load_b128(r, (int)off, 0, 0);
}
__device__ __forceinline__ float load_f32(__amdgpu_buffer_rsrc_t r, uint32_t off) {
    return __uint_as_float(__builtin_amdgcn_raw_buffer_load_b32(r, (int)off, 0, 0));
}

// ---- issue order of one staged K slice ------------------------------------------------
// A slice body is one basic block: next-slice global loads, 4 K steps of LDS fragment reads
// + MFMAs, LDS writes of the next slice.  Left alone, the scheduler sinks the global loads
// to the LDS writes (exposing the whole memory latency) and reads each step's fragments
// only after the previous step's MFMAs.  sched_group_barrier fixes the issue order:
//   step-0 reads, global loads, step-1 reads,
//   step-0 MFMAs with step-2 reads spread between them, step-1 MFMAs with step-3 reads,
//   step-2 MFMAs, step-3 MFMAs with the LDS writes spread between them.
// Data dependencies are unchanged; only the order of independent instructions is.
constexpr int kSgMfma = 0x008, kSgVmemRd = 0x020, kSgDsRd = 0x100, kSgDsWr = 0x200;

// NA instructions of class MA and NB of class MB, the B's spread evenly among the A's
template <int MA, int NA, int MB, int NB>
__device__ __forceinline__ void sched_spread() {
    if constexpr (NB == 0) {
        if constexpr (NA > 0) __builtin_amdgcn_sched_group_barrier(MA, NA, 0);
    } else if constexpr (NA == 0) {
        __builtin_amdgcn_sched_group_barrier(MB, NB, 0);
    } else {
        constexpr int a = (NA + NB - 1) / NB;
        __builtin_amdgcn_sched_group_barrier(MA, a, 0);
        __builtin_amdgcn_sched_group_barrier(MB, 1, 0);
        sched_spread<MA, NA - a, MB, NB - 1>();
    }
}

// RD LDS reads and MF MFMAs per K step, VM global loads and WR LDS writes per slice
template <int RD, int MF, int VM, int WR>
__device__ __forceinline__ void sched_slice() {
    __builtin_amdgcn_sched_group_barrier(kSgDsRd, RD, 0);
    if constexpr (VM > 0) __builtin_amdgcn_sched_group_barrier(kSgVmemRd, VM, 0);
    __builtin_amdgcn_sched_group_barrier(kSgDsRd, RD, 0);
    sched_spread<kSgMfma, MF, kSgDsRd, RD>();
    sched_spread<kSgMfma, MF, kSgDsRd, RD>();
    __builtin_amdgcn_sched_group_barrier(kSgMfma, MF, 0);
    sched_spread<kSgMfma, MF, kSgDsWr, WR>();
}

}  // namespace mla
