// Device-side building blocks shared by every gfx950 kernel of the layer:
// MFMA fragment types, wave64 reductions on DPP / ds_swizzle, XCD-aware block order.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include "gpu_shape.h"

namespace mla {

typedef float v4f __attribute__((ext_vector_type(4)));
typedef float v16f __attribute__((ext_vector_type(16)));
typedef __bf16 v8bf __attribute__((ext_vector_type(8)));

// ----------------------------------------------------------------------------------
// fp32 MFMA: D(32x32) += A(32x2) * B(2x32).  Lane l supplies A[l%32][l/32] and
// B[l/32][l%32]; accumulator i of lane l is D[8*(i/4) + 4*(l/32) + i%4][l%32].
// The kernels drive four of these per 8-deep slice and permute K so that lane l's four
// A (or B) values are k = 4*(l/32) + 0..3: one 128-bit LDS read feeds four MFMAs.
// ----------------------------------------------------------------------------------
__device__ __forceinline__ v16f mfma_32x32x2(float a, float b, v16f c) {
    return __builtin_amdgcn_mfma_f32_32x32x2f32(a, b, c, 0, 0, 0);
}

__device__ __forceinline__ int acc_row(int i, int lane) {
    return 8 * (i >> 2) + 4 * (lane >> 5) + (i & 3);
}

// ----------------------------------------------------------------------------------
// Wave reductions.  Steps 1..8 move data with DPP (quad_perm, row_half_mirror,
// row_mirror); step 16 with gfx950's v_permlane16_swap, which exchanges the odd 16-lane
// rows of one register with the even rows of another -- given the same value twice it
// returns, in every lane, the value of its own row pair's even row and odd row.  The two
// 32-lane halves meet through readlane.  Each step leaves the partial result in every
// lane of its group, and every step combines its two operands in the same order in all
// lanes, so sums are bitwise identical across the group.
// ----------------------------------------------------------------------------------
// bound_ctrl is set: every control used here reads a lane inside the same row, so it
// changes nothing but lets the compiler fold the move into the consuming VALU op (one
// v_max_f32_dpp / v_add_f32_dpp per step).
template <int kCtrl>
__device__ __forceinline__ float dpp_move(float v) {
    return __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), kCtrl, 0xF, 0xF,
                                                      true));
}

struct OpMax {
    __device__ float operator()(float a, float b) const { return fmaxf(a, b); }
};
struct OpSum {
    __device__ float operator()(float a, float b) const { return a + b; }
};

// Reduce across the 32 lanes of each half-wave; every lane gets its half's result.
template <class Op>
__device__ __forceinline__ float half_wave_reduce(float v, Op op) {
    v = op(v, dpp_move<0xB1>(v));   // quad_perm [1,0,3,2]  (lane ^ 1)
    v = op(v, dpp_move<0x4E>(v));   // quad_perm [2,3,0,1]  (lane ^ 2)
    v = op(v, dpp_move<0x141>(v));  // row_half_mirror      (other quad of 8)
    v = op(v, dpp_move<0x140>(v));  // row_mirror           (other half of 16)
    const auto r = __builtin_amdgcn_permlane16_swap(__float_as_uint(v), __float_as_uint(v),
                                                    false, false);
    return op(__uint_as_float(r[0]), __uint_as_float(r[1]));   // (even row, odd row)
}

// Reduce across the whole wave; the result is wave-uniform.
template <class Op>
__device__ __forceinline__ float wave_reduce(float v, Op op) {
    v = half_wave_reduce(v, op);
    const float lo = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), 0));
    const float hi = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), 32));
    return op(lo, hi);
}

// A wave-uniform read of kernel-lifetime read-only data (sequence lengths, page tables):
// through the constant address space it is an s_load into SGPRs, so waiting for it does
// not drain the vector-memory queue the staging pipeline keeps full.
__device__ __forceinline__ int load_uniform(const int* p) {
    typedef const __attribute__((address_space(4))) int ConstInt;
    return *(ConstInt*)p;
}

// ----------------------------------------------------------------------------------
// RoPE rotation of the interleaved pair (x0, x1) = (x[2i], x[2i+1]) by the angle
// pos * inv_freq[i] (exhaustive_benchmark_suite.py:210-232); the angle is formed in fp32
// from the caller's inv_freq table, and cos / sin are the accurate cosf / sinf.  2b
// (rowops.hip), the KV append and 2a2's fused epilogue (wgemm.hip) share these.
// ----------------------------------------------------------------------------------
__device__ __forceinline__ float rope_angle(int64_t pos, float inv_freq) {
    return (float)pos * inv_freq;
}
// cos and sin of the angle, both from one sincosf: every kernel that rotates calls this, so
// the values agree to the bit across kernels (separate cosf / sinf calls may or may not be
// merged into a sincos by the compiler, depending on the context).
__device__ __forceinline__ void rope_cos_sin(float ang, float* c, float* s) { sincosf(ang, s, c); }
// Written with one explicit fma each, and the result pinned to an fp32 register value (the
// empty asm), so that every kernel that inlines them rounds the same way: the compiler can
// neither pick another contraction nor fuse the fma with a following fp16 conversion into
// v_fma_mix, which rounds once to 16 bits instead of to fp32 and then to 16 bits.
__device__ __forceinline__ float fp32_pinned(float v) {
    asm volatile("" : "+v"(v));
    return v;
}
__device__ __forceinline__ float rope_even(float x0, float x1, float c, float s) {
    return fp32_pinned(__builtin_fmaf(x0, c, -(x1 * s)));
}
__device__ __forceinline__ float rope_odd(float x0, float x1, float c, float s) {
    return fp32_pinned(__builtin_fmaf(x0, s, x1 * c));
}

// ----------------------------------------------------------------------------------
// XCD-aware block order.  The dispatcher hands workgroup b to XCD b % 8; this maps the
// hardware id to a logical tile id so that each XCD walks a CONTIGUOUS run of logical
// tiles (and therefore keeps the operands those tiles share in its own L2).
// ----------------------------------------------------------------------------------
__device__ __forceinline__ int xcd_logical_block(int bid, int nblocks) {
    const int q = nblocks / kNumXCDs;
    const int r = nblocks % kNumXCDs;
    const int x = bid % kNumXCDs;
    const int s = bid / kNumXCDs;
    return x * q + (x < r ? x : r) + s;
}

// ----------------------------------------------------------------------------------
// 16-bit storage formats.  Both are raw 16-bit words in memory and in LDS; conversions
// from fp32 round to nearest even, as torch does (a NaN stays a NaN):
//   bfloat16 -- gfx950's v_cvt_pk_bf16_f32, two values per instruction;
//   fp16     -- v_cvt_f16_f32 in the default rounding mode (values past 65504 become
//               infinities, values below 2^-24 flush to zero, as in IEEE binary16).
// Half<TL> gives kernels templated on the format one interface: TL = bf16_t or f16_t.
// Store16<OUT> maps an output-format code (kernels.h OutType: 1 bf16, 2 fp16) to it.
// ----------------------------------------------------------------------------------
typedef uint16_t bf16_t;
typedef _Float16 f16_t;
typedef __bf16 bf16x2_t __attribute__((ext_vector_type(2)));
typedef _Float16 f16x2_t __attribute__((ext_vector_type(2)));
typedef _Float16 v8h __attribute__((ext_vector_type(8)));

__device__ __forceinline__ uint32_t pack_bf16x2(float lo, float hi) {
    const bf16x2_t v = {(__bf16)lo, (__bf16)hi};
    return __builtin_bit_cast(uint32_t, v);
}
__device__ __forceinline__ uint32_t f32_to_bf16_bits(float f) {
    return __builtin_bit_cast(uint16_t, (__bf16)f);
}
__device__ __forceinline__ float bf16_bits_to_f32(uint32_t h) { return __uint_as_float(h << 16); }

__device__ __forceinline__ uint32_t pack_f16x2(float lo, float hi) {
    const f16x2_t v = {(_Float16)lo, (_Float16)hi};
    return __builtin_bit_cast(uint32_t, v);
}
__device__ __forceinline__ uint32_t f32_to_f16_bits(float f) {
    return __builtin_bit_cast(uint16_t, (_Float16)f);
}
__device__ __forceinline__ float f16_bits_to_f32(uint32_t h) {
    return (float)__builtin_bit_cast(_Float16, (uint16_t)h);
}

template <typename TL> struct Half;
template <> struct Half<bf16_t> {
    static constexpr bool kF16 = false;
    __device__ static __forceinline__ uint32_t pack2(float lo, float hi) { return pack_bf16x2(lo, hi); }
    __device__ static __forceinline__ uint32_t bits(float f) { return f32_to_bf16_bits(f); }
    __device__ static __forceinline__ float to_f32(uint32_t h) { return bf16_bits_to_f32(h); }
};
template <> struct Half<f16_t> {
    static constexpr bool kF16 = true;
    __device__ static __forceinline__ uint32_t pack2(float lo, float hi) { return pack_f16x2(lo, hi); }
    __device__ static __forceinline__ uint32_t bits(float f) { return f32_to_f16_bits(f); }
    __device__ static __forceinline__ float to_f32(uint32_t h) { return f16_bits_to_f32(h); }
};

template <int OUT> struct Store16;
template <> struct Store16<1> : Half<bf16_t> {};
template <> struct Store16<2> : Half<f16_t> {};

}  // namespace mla
