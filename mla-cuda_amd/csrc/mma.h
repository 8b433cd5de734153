// MFMA "K step" abstraction shared by the GEMM engine and the scores kernel.
//
// Every K-contiguous LDS row holds 128 bytes of K per slice (32 fp32 or 64 bf16) plus a
// 16-byte pad.  One K step consumes 32 of those bytes: lane l reads the 16 bytes at
// byte 32*step + 16*(l/32) of its row (one ds_read_b128) and feeds
//   fp32: four v_mfma_f32_32x32x2_f32  (4 k values per lane, K = 8 per step)
//   bf16: one   v_mfma_f32_32x32x16_bf16 (8 k values per lane, K = 16 per step)
// Both instructions take row/column l%32 from lane l and split K between the two
// half-waves, and A and B fragments are always read from the same k offsets, so the
// product is exact whatever order the hardware assigns to the k values inside a lane.
// The 32x32 fp32 accumulator layout is the same for both.
#pragma once

#include "common.h"

namespace mla {

typedef uint32_t v4u __attribute__((ext_vector_type(4)));

// bf16 storage is raw 16-bit words; conversion rounds to nearest even (as torch does).
typedef uint16_t bf16_t;

__device__ __forceinline__ uint32_t f32_to_bf16_bits(float f) {
    const uint32_t u = __float_as_uint(f);
    if ((u & 0x7fffffffu) > 0x7f800000u) return 0x7fc0u;  // NaN
    return (u + 0x7fffu + ((u >> 16) & 1u)) >> 16;
}
__device__ __forceinline__ float bf16_bits_to_f32(uint32_t h) { return __uint_as_float(h << 16); }

__device__ __forceinline__ uint32_t pack_bf16x2(float lo, float hi) {
    return f32_to_bf16_bits(lo) | (f32_to_bf16_bits(hi) << 16);
}

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

// Load 16 bytes of TL elements [k, k + kElems) of a K-contiguous row, zero beyond k_end.
template <typename TL>
__device__ __forceinline__ v4u load_chunk(const TL* __restrict__ src, int k, int k_end) {
    constexpr int E = Mma<TL>::kElems;
    if (k + E <= k_end) return *reinterpret_cast<const v4u*>(src);
    v4u r = {0u, 0u, 0u, 0u};
    if constexpr (sizeof(TL) == 4) {
        #pragma unroll
        for (int j = 0; j < 4; ++j) r[j] = (k + j < k_end) ? __float_as_uint(src[j]) : 0u;
    } else {
        #pragma unroll
        for (int j = 0; j < 8; ++j) {
            const uint32_t h = (k + j < k_end) ? (uint32_t)src[j] : 0u;
            r[j >> 1] |= h << (16 * (j & 1));
        }
    }
    return r;
}

}  // namespace mla
