// Row-wise steps of the layer: 2a-n RMSNorm, 2b RoPE, 3b softmax-partial combine, the
// streaming merge, and the KV-cache append and wkv_b split beside the layer.
// All three are HBM/latency bound and tiny next to the contractions; they use 128-bit
// loads where the row is contiguous and wave64 DPP reductions.

#include "common.h"
#include "kernels.h"

#include <algorithm>

namespace mla {

namespace {

typedef uint32_t v4u_t __attribute__((ext_vector_type(4)));   // 16 raw bytes

// ---- 2a-n: one 256-thread workgroup per row.  The input may be nsplit fp32 partial
// sums of 2a1 (split-K); they are added here in slice order, which is what makes the
// split-K of 2a1 free of a separate reduction pass.  Each thread keeps its summed
// elements in registers between the sum-of-squares pass and the output pass (rows up to
// 4096 wide), so the partials are read once; the partial loop is unrolled so the loads
// of all slices are in flight together.  The row body is shared with the KV-cache append,
// so both normalise with the same arithmetic and summation order.
constexpr int kNormCache = 4;  // float4 per thread kept in registers (256*4*4 = 4096 wide)

// Sum of nsplit partial rows (slice order) at float4 column c4.  NS > 0: nsplit == NS,
// known at compile time, and all NS loads are issued before the first add (one memory
// latency instead of one per batch); the additions run in the same order either way.
template <int NS = 0>
__device__ __forceinline__ v4f sum_partials4(const float* base, int nsplit, int64_t split_stride,
                                             int c4) {
    if constexpr (NS > 0) {
        v4f p[NS];
        #pragma unroll
        for (int s = 0; s < NS; ++s) p[s] = *reinterpret_cast<const v4f*>(base + s * split_stride + 4 * c4);
        v4f v = p[0];
        #pragma unroll
        for (int s = 1; s < NS; ++s) v += p[s];
        return v;
    }
    v4f v = *reinterpret_cast<const v4f*>(base + 4 * c4);
    int s = 1;
    for (; s + 4 <= nsplit; s += 4) {
        const v4f a = *reinterpret_cast<const v4f*>(base + s * split_stride + 4 * c4);
        const v4f b = *reinterpret_cast<const v4f*>(base + (s + 1) * split_stride + 4 * c4);
        const v4f c = *reinterpret_cast<const v4f*>(base + (s + 2) * split_stride + 4 * c4);
        const v4f d = *reinterpret_cast<const v4f*>(base + (s + 3) * split_stride + 4 * c4);
        v += a; v += b; v += c; v += d;
    }
    for (; s < nsplit; ++s)
        v += *reinterpret_cast<const v4f*>(base + s * split_stride + 4 * c4);
    return v;
}

// out_row[0:N] = row * rsqrt(mean(row^2) + eps) * gain, row = summed partials at `base`.
// Called by all 256 threads of the workgroup (it synchronises through `red`).
template <int OUT, int NS = 0>
__device__ __forceinline__ void rms_row(const float* base, int nsplit, int64_t split_stride,
                                        const void* gain_v, void* out_row, int N, float eps,
                                        float* red) {
    const int tid = threadIdx.x;
    const int n4 = N >> 2;
    v4f cache[kNormCache];
    float ss = 0.f;
    #pragma unroll
    for (int j = 0; j < kNormCache; ++j) {
        const int c4 = tid + 256 * j;
        cache[j] = (c4 < n4) ? sum_partials4<NS>(base, nsplit, split_stride, c4) : v4f{0.f, 0.f, 0.f, 0.f};
        ss += cache[j][0] * cache[j][0] + cache[j][1] * cache[j][1] +
              cache[j][2] * cache[j][2] + cache[j][3] * cache[j][3];
    }
    for (int c4 = tid + 256 * kNormCache; c4 < n4; c4 += 256) {
        const v4f v = sum_partials4<NS>(base, nsplit, split_stride, c4);
        ss += v[0] * v[0] + v[1] * v[1] + v[2] * v[2] + v[3] * v[3];
    }
    ss = wave_reduce(ss, OpSum());
    if ((tid & 63) == 0) red[tid >> 6] = ss;
    __syncthreads();
    const float total = red[0] + red[1] + red[2] + red[3];
    const float inv = rsqrtf(total / (float)N + eps);

    auto emit = [&](int c4, const v4f& v) {
        if constexpr (OUT == kOutF32) {
            const v4f g = *reinterpret_cast<const v4f*>(static_cast<const float*>(gain_v) + 4 * c4);
            v4f o;
            #pragma unroll
            for (int j = 0; j < 4; ++j) o[j] = v[j] * inv * g[j];
            *reinterpret_cast<v4f*>(static_cast<float*>(out_row) + 4 * c4) = o;
        } else {
            const uint16_t* g = static_cast<const uint16_t*>(gain_v) + 4 * c4;
            uint16_t* o = static_cast<uint16_t*>(out_row) + 4 * c4;
            #pragma unroll
            for (int j = 0; j < 4; ++j)
                o[j] = (uint16_t)Store16<OUT>::bits(v[j] * inv * Store16<OUT>::to_f32(g[j]));
        }
    };
    #pragma unroll
    for (int j = 0; j < kNormCache; ++j) {
        const int c4 = tid + 256 * j;
        if (c4 < n4) emit(c4, cache[j]);
    }
    for (int c4 = tid + 256 * kNormCache; c4 < n4; c4 += 256)
        emit(c4, sum_partials4<NS>(base, nsplit, split_stride, c4));
}

template <int OUT, int NS>
__global__ void __launch_bounds__(256) rmsnorm_kernel(const float* __restrict__ in, int nsplit,
                                                      int64_t split_stride, const void* gain_v,
                                                      void* out_v, int N, float eps,
                                                      RopeTable rt) {
    __shared__ float red[4];
    const int row = blockIdx.x;
    // the row's RoPE angle table for 2a2's fused epilogue, when asked for
    if (rt.cos_sin && (int)threadIdx.x < rt.half) {
        const int i = threadIdx.x;
        const int64_t pos = rt.positions[rt.per_batch ? row : row % rt.Sq];
        float c, s;
        rope_cos_sin(rope_angle(pos, rt.inv_freq[i]), &c, &s);
        float* t = rt.cos_sin + 2 * ((int64_t)row * rt.half + i);
        t[0] = c;
        t[1] = s;
    }
    void* out_row = OUT == kOutF32
                        ? static_cast<void*>(static_cast<float*>(out_v) + (int64_t)row * N)
                        : static_cast<void*>(static_cast<uint16_t*>(out_v) + (int64_t)row * N);
    rms_row<OUT, NS>(in + (int64_t)row * N, nsplit, split_stride, gain_v, out_row, N, eps, red);
}

// ---- 2b: one workgroup per (query row bq, chunk of 32 heads; 4 when it also sums 2a2's
// split partials, below).  Every head of a row uses
// the same rope/2 angles, so the workgroup evaluates them once into LDS: angle =
// float(pos) * inv_freq[i] in fp32 with the caller's inv_freq table, then the accurate
// sincosf (not the fast intrinsics: at positions ~5e3 an angle ulp is ~5e-4 rad and
// large arguments need full range reduction).  Threads then rotate the (head, pair)
// elements of the chunk with 64-bit loads and stores.
// When 2a2 ran split-K, q_raw is its partials ([nsplit][rows][H*qk], split_stride apart)
// and this kernel also does the split sum (in split order from 0, as split_reduce_kernel
// does, so the result is the same to the bit): the nope columns of its heads go to
// nope_out (for 2c), the rope columns are summed before the rotation.  That saves 2a2's
// reduction launch at small batches.
constexpr int kRopeHeads = 32;
constexpr int kRopeSumHeads = 4;   // heads per workgroup when it also sums 2a2's partials
constexpr int kRopeMaxHalf = 256;


template <int OUT>
__global__ void __launch_bounds__(256) rope_kernel(const float* __restrict__ q_raw,
                                                   int nsplit, int64_t split_stride,
                                                   float* __restrict__ nope_out,
                                                   const int64_t* __restrict__ positions,
                                                   const float* __restrict__ inv_freq,
                                                   void* out_v, int Sq, int H, int nope,
                                                   int rope, int pos_per_batch) {
    __shared__ float cs[kRopeMaxHalf], sn[kRopeMaxHalf];
    const int half = rope >> 1;
    const int qk = nope + rope;
    const int bq = blockIdx.x;
    const int hpw = nope_out ? kRopeSumHeads : kRopeHeads;
    const int h0 = blockIdx.y * hpw;
    const int nh = min(hpw, H - h0);
    const int64_t pos = positions[pos_per_batch ? bq : bq % Sq];
    for (int i = threadIdx.x; i < half; i += blockDim.x) {
        const float ang = rope_angle(pos, inv_freq[i]);
        rope_cos_sin(ang, &cs[i], &sn[i]);
    }
    const int64_t row0 = (int64_t)bq * H * qk;
    if (nope_out) {
        const int nq = nope >> 2;
        for (int idx = threadIdx.x; idx < nh * nq; idx += blockDim.x) {
            const int64_t off = row0 + (int64_t)(h0 + idx / nq) * qk + 4 * (idx % nq);
            float4 acc = make_float4(0.f, 0.f, 0.f, 0.f);
            for (int q = 0; q < nsplit; ++q) {
                const float4 v = *reinterpret_cast<const float4*>(q_raw + q * split_stride + off);
                acc.x += v.x; acc.y += v.y; acc.z += v.z; acc.w += v.w;
            }
            *reinterpret_cast<float4*>(nope_out + off) = acc;
        }
    }
    __syncthreads();
    const float* src = q_raw + row0 + nope;
    for (int idx = threadIdx.x; idx < nh * half; idx += blockDim.x) {
        const int h = h0 + idx / half;
        const int i = idx % half;
        float2 x = make_float2(0.f, 0.f);
        for (int q = 0; q < nsplit; ++q) {
            const float2 v = *reinterpret_cast<const float2*>(src + q * split_stride + (int64_t)h * qk + 2 * i);
            x.x += v.x;
            x.y += v.y;
        }
        const float e = rope_even(x.x, x.y, cs[i], sn[i]);
        const float o = rope_odd(x.x, x.y, cs[i], sn[i]);
        const int64_t dst = ((int64_t)bq * H + h) * rope + 2 * i;
        if constexpr (OUT == kOutF32) {
            *reinterpret_cast<float2*>(static_cast<float*>(out_v) + dst) = make_float2(e, o);
        } else {
            *reinterpret_cast<uint32_t*>(static_cast<uint16_t*>(out_v) + dst) = Store16<OUT>::pack2(e, o);
        }
    }
}

// ---- 3b: one wave per row.  M = max_j m_j; alpha_j = exp(m_j - M), exactly 1 where
// m_j == M (which also keeps an all-masked partial at -inf from producing NaN);
// row_sum = sum_j l_j alpha_j.  Rows are contiguous, so the lanes' loads coalesce.
__global__ void __launch_bounds__(256) combine_kernel(const float* __restrict__ m_part,
                                                      const float* __restrict__ l_part,
                                                      float* __restrict__ alpha,
                                                      float* __restrict__ row_sum,
                                                      float* __restrict__ row_max, int rows,
                                                      int P) {
    const int lane = threadIdx.x & 63;
    const int row = blockIdx.x * 4 + (threadIdx.x >> 6);
    if (row >= rows) return;  // wave-uniform
    const float* mr = m_part + (int64_t)row * P;
    const float* lr = l_part + (int64_t)row * P;
    float* ar = alpha + (int64_t)row * P;
    float m = -INFINITY;
    for (int j = lane; j < P; j += 64) m = fmaxf(m, mr[j]);
    const float M = wave_reduce(m, OpMax());
    float l = 0.f;
    for (int j = lane; j < P; j += 64) {
        const float mj = mr[j];
        const float aj = (mj == M) ? 1.f : expf(mj - M);
        ar[j] = aj;
        l += lr[j] * aj;
    }
    l = wave_reduce(l, OpSum());
    if (lane == 0) {
        row_sum[row] = l;
        if (row_max) row_max[row] = M;
    }
}

// ---- streaming merge: one wave per row; lanes walk the row's R ctx values as float4.
// Exact when both maxima are equal; a fully masked state (M = -inf, L = 0) contributes 0.
__global__ void __launch_bounds__(256) stream_merge_kernel(float* __restrict__ ctx,
                                                           float* __restrict__ run_max,
                                                           float* __restrict__ run_sum,
                                                           const float* __restrict__ ctx_c,
                                                           const float* __restrict__ max_c,
                                                           const float* __restrict__ sum_c,
                                                           int rows, int R, int first) {
    const int lane = threadIdx.x & 63;
    const int row = blockIdx.x * 4 + (threadIdx.x >> 6);
    if (row >= rows) return;  // wave-uniform
    const float mc = max_c[row];
    float a = 0.f, b = 1.f, mn = mc;
    if (!first) {
        const float mo = run_max[row];
        mn = fmaxf(mo, mc);
        a = (mo == mn) ? 1.f : expf(mo - mn);
        b = (mc == mn) ? 1.f : expf(mc - mn);
    }
    v4f* dst = reinterpret_cast<v4f*>(ctx + (int64_t)row * R);
    const v4f* src = reinterpret_cast<const v4f*>(ctx_c + (int64_t)row * R);
    for (int c = lane; c < R / 4; c += 64) dst[c] = first ? src[c] : dst[c] * a + src[c] * b;
    if (lane == 0) {
        run_sum[row] = first ? sum_c[row] : run_sum[row] * a + sum_c[row] * b;
        run_max[row] = mn;
    }
}

// ---- KV-cache append: one 256-thread workgroup per new token row (b, s).  The row's
// kv_rank latent columns are normalised exactly as 2a-n normalises (rms_row), its rope
// columns rotated exactly as 2b rotates, and both land in cache row start_row + s of
// batch b.  The input is the GEMM output x @ W_kv_a or its nsplit split-K partials, rows
// of ld = kv_rank + rope floats; partials are summed in slice order.
template <int OUT>
__global__ void __launch_bounds__(256) kv_append_kernel(const float* __restrict__ in, int nsplit,
                                                        int64_t split_stride, const void* gain,
                                                        const int64_t* __restrict__ positions,
                                                        const float* __restrict__ inv_freq,
                                                        void* c_kv, void* pe, int Sq, int R, int D,
                                                        int start_row, int cache_rows,
                                                        int pos_per_batch, const int* block_table,
                                                        int page_size, int max_pages, float eps) {
    __shared__ float red[4];
    const int row = blockIdx.x;
    const int b = row / Sq, s = row % Sq;
    const int ld = R + D;
    const float* base = in + (int64_t)row * ld;
    const int64_t pos = positions[pos_per_batch ? row : s];
    // destination row: dense cache row b*cache_rows + start_row + s, or in a paged cache
    // the row of logical slot `pos` (the token's position) through the block table
    int64_t crow;
    if (block_table) {
        if (pos < 0 || pos / page_size >= max_pages) return;   // outside the table: skip
        const int page = block_table[(int64_t)b * max_pages + pos / page_size];
        crow = (int64_t)page * page_size + pos % page_size;
    } else {
        crow = (int64_t)b * cache_rows + start_row + s;
    }
    // rope pairs first (no barrier inside), then the workgroup-wide norm
    for (int i = threadIdx.x; i < D / 2; i += blockDim.x) {
        float x0 = base[R + 2 * i], x1 = base[R + 2 * i + 1];
        for (int q = 1; q < nsplit; ++q) {
            x0 += base[q * split_stride + R + 2 * i];
            x1 += base[q * split_stride + R + 2 * i + 1];
        }
        const float ang = rope_angle(pos, inv_freq[i]);
        float c, sn;
        rope_cos_sin(ang, &c, &sn);
        const float e = rope_even(x0, x1, c, sn), o = rope_odd(x0, x1, c, sn);
        if constexpr (OUT == kOutF32) {
            float* dst = static_cast<float*>(pe) + crow * D + 2 * i;
            dst[0] = e; dst[1] = o;
        } else {
            *reinterpret_cast<uint32_t*>(static_cast<uint16_t*>(pe) + crow * D + 2 * i) =
                Store16<OUT>::pack2(e, o);
        }
    }
    void* out_row = OUT == kOutF32
                        ? static_cast<void*>(static_cast<float*>(c_kv) + crow * R)
                        : static_cast<void*>(static_cast<uint16_t*>(c_kv) + crow * R);
    rms_row<OUT>(base, nsplit, split_stride, gain, out_row, R, eps, red);
}

// ---- fp8 cache decoding: out[i] = code[i] * scale, OCP e4m3 codes, through the same
// conversion the fused attention uses (v_cvt_scalef32_pk_bf16_fp8 with scale 1, exact for
// every code, then bf16 -> fp32, then the fp32 product).  Thread t takes codes 4t .. 4t+3.
__global__ void __launch_bounds__(256) fp8_dequant_kernel(const uint8_t* __restrict__ codes,
                                                          int64_t n, float scale,
                                                          float* __restrict__ out) {
    for (int64_t t = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; 4 * t < n;
         t += (int64_t)gridDim.x * blockDim.x) {
        const int64_t i0 = 4 * t;
        uint32_t w = 0;
        #pragma unroll
        for (int k = 0; k < 4; ++k)
            if (i0 + k < n) w |= (uint32_t)codes[i0 + k] << (8 * k);
        const uint32_t lo = __builtin_bit_cast(uint32_t, __builtin_amdgcn_cvt_scalef32_pk_bf16_fp8(w, 1.f, false));
        const uint32_t hi = __builtin_bit_cast(uint32_t, __builtin_amdgcn_cvt_scalef32_pk_bf16_fp8(w, 1.f, true));
        const float v[4] = {bf16_bits_to_f32(lo & 0xffffu), bf16_bits_to_f32(lo >> 16),
                            bf16_bits_to_f32(hi & 0xffffu), bf16_bits_to_f32(hi >> 16)};
        #pragma unroll
        for (int k = 0; k < 4; ++k)
            if (i0 + k < n) out[i0 + k] = v[k] * scale;
    }
}

// ---- wkv_b split: row r of wkv_b [H, nope + v, R] goes to W_uk (j < nope) or W_uv.
// One thread per 16-byte chunk; rows are whole chunks (R * element size % 16 == 0).
__global__ void __launch_bounds__(256) split_rows_kernel(const v4u_t* __restrict__ src,
                                                         v4u_t* __restrict__ dst_a,
                                                         v4u_t* __restrict__ dst_b, int64_t rows,
                                                         int rows_a, int rows_per_group,
                                                         int chunks_per_row) {
    const int64_t total = rows * chunks_per_row;
    for (int64_t idx = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; idx < total;
         idx += (int64_t)gridDim.x * blockDim.x) {
        const int64_t r = idx / chunks_per_row;
        const int c = (int)(idx - r * chunks_per_row);
        const int64_t h = r / rows_per_group;
        const int j = (int)(r - h * rows_per_group);
        const int rows_b = rows_per_group - rows_a;
        v4u_t* dst = j < rows_a ? dst_a + ((h * rows_a + j) * chunks_per_row + c)
                                : dst_b + ((h * rows_b + (j - rows_a)) * chunks_per_row + c);
        *dst = src[idx];
    }
}


// ---- 2b + 2c for decode-sized fp32 batches (M = B*Sq <= kQSmallRows), from 2a2's split
// partials: one workgroup per (head, 256-column half of q_abs).  At M <= 8 the 2c tile of
// the MFMA engine is 1/4 .. 1/32 full and 2b is a launch of its own; here:
//   1. The head's M q_nope rows, 2a2's partials summed in split order from 0 (rope_kernel's
//      sum, the same bits; one 4-column quad per thread), go to LDS (rows past M as zeros).
//      The half-0 workgroup also rotates the head's rope pairs into q_rope, one (row, pair)
//      per thread, with rope_kernel's angle, sincosf and rotation.
//   2. W_uk[h]'s 128 rows of the workgroup's 256 columns stream once: wave w takes rows
//      32 w .. 32 w + 31 (1 KB per row and instruction), lane l columns 4 l .. 4 l + 3.  The
//      partials' loads go out first (at most kQSmallMaxSplit per thread, in registers),
//      then the 32 W_uk loads, so that step 1 waits for its own loads only and the stream
//      runs under it; then each lane accumulates all eight q_nope rows against its rows
//      (fp32 FMAs, row k ascending).
//   3. The four waves' sums add in wave order through LDS and go to q_abs.
constexpr int kQSmallNope = 128;
constexpr int kQSmallKv = 512;
static_assert(kQSmallRows * kQSmallNope == 4 * 256, "one q_nope quad per thread");

__global__ void __launch_bounds__(256) q_small_kernel(const float* __restrict__ q_parts,
                                                      int nsplit, int64_t split_stride,
                                                      const int64_t* __restrict__ positions,
                                                      const float* __restrict__ inv_freq,
                                                      const float* __restrict__ W_uk,
                                                      float* __restrict__ q_rope,
                                                      float* __restrict__ q_abs, int Sq, int M,
                                                      int H, int rope, int pos_per_batch) {
    __shared__ __attribute__((aligned(16))) float qn[kQSmallRows][kQSmallNope];
    __shared__ __attribute__((aligned(16))) float red[4][kQSmallRows][256];
    const int h = blockIdx.x >> 1, c0 = 256 * (blockIdx.x & 1);
    const int tid = threadIdx.x, wave = tid >> 6, lane = tid & 63;
    const int qk = kQSmallNope + rope, half = rope >> 1;
    // loads in the order they are needed: the partials of this thread's q_nope quad (row
    // tid / 32, columns 4 (tid % 32) ..) and, in half 0, of its rope pair, then the W_uk rows
    const int m = tid >> 5, k4 = 4 * (tid & 31);
    const int64_t off_n = ((int64_t)m * H + h) * qk + k4;
    const bool has_rope = c0 == 0 && tid < M * half;
    const int mr = has_rope ? tid / half : 0, ir = has_rope ? tid % half : 0;
    const int64_t off_r = ((int64_t)mr * H + h) * qk + kQSmallNope + 2 * ir;
    v4f pn[kQSmallMaxSplit];
    float2 pr[kQSmallMaxSplit];
    #pragma unroll
    for (int s = 0; s < kQSmallMaxSplit; ++s) {
        pn[s] = v4f{0.f, 0.f, 0.f, 0.f};
        pr[s] = make_float2(0.f, 0.f);
        if (s < nsplit && m < M) pn[s] = *reinterpret_cast<const v4f*>(q_parts + s * split_stride + off_n);
        if (s < nsplit && has_rope) pr[s] = *reinterpret_cast<const float2*>(q_parts + s * split_stride + off_r);
    }
    const float* w = W_uk + ((int64_t)h * kQSmallNope + 32 * wave) * kQSmallKv + c0 + 4 * lane;
    v4f wr[32];
    #pragma unroll
    for (int r = 0; r < 32; ++r)
        wr[r] = __builtin_nontemporal_load(reinterpret_cast<const v4f*>(w + (int64_t)r * kQSmallKv));
    // 1. q_nope quad: the split sum in split order from 0 (rope_kernel's, the same bits)
    v4f qs = v4f{0.f, 0.f, 0.f, 0.f};
    #pragma unroll
    for (int s = 0; s < kQSmallMaxSplit; ++s)
        if (s < nsplit) qs += pn[s];
    *reinterpret_cast<v4f*>(&qn[m][k4]) = qs;   // rows past M: zeros
    if (has_rope) {
        const int64_t pos = positions[pos_per_batch ? mr : mr % Sq];
        float c, sn;
        rope_cos_sin(rope_angle(pos, inv_freq[ir]), &c, &sn);
        float x0 = 0.f, x1 = 0.f;
        #pragma unroll
        for (int s = 0; s < kQSmallMaxSplit; ++s)
            if (s < nsplit) {
                x0 += pr[s].x;
                x1 += pr[s].y;
            }
        *reinterpret_cast<float2*>(q_rope + ((int64_t)mr * H + h) * rope + 2 * ir) =
            make_float2(rope_even(x0, x1, c, sn), rope_odd(x0, x1, c, sn));
    }
    __syncthreads();
    // 2. this wave's 32 W_uk rows against the eight q_nope rows
    v4f acc[kQSmallRows];
    #pragma unroll
    for (int mm = 0; mm < kQSmallRows; ++mm) acc[mm] = v4f{0.f, 0.f, 0.f, 0.f};
    #pragma unroll
    for (int r4 = 0; r4 < 32; r4 += 4) {
        #pragma unroll
        for (int mm = 0; mm < kQSmallRows; ++mm) {
            const v4f q = *reinterpret_cast<const v4f*>(&qn[mm][32 * wave + r4]);
            #pragma unroll
            for (int t = 0; t < 4; ++t)
                #pragma unroll
                for (int j = 0; j < 4; ++j) acc[mm][j] = __builtin_fmaf(q[t], wr[r4 + t][j], acc[mm][j]);
        }
    }
    // 3. the four waves' sums in wave order
    #pragma unroll
    for (int mm = 0; mm < kQSmallRows; ++mm) *reinterpret_cast<v4f*>(&red[wave][mm][4 * lane]) = acc[mm];
    __syncthreads();
    for (int idx = tid; idx < M * 64; idx += 256) {
        const int mm = idx >> 6, c4 = 4 * (idx & 63);
        const v4f sum = ((*reinterpret_cast<const v4f*>(&red[0][mm][c4]) +
                          *reinterpret_cast<const v4f*>(&red[1][mm][c4])) +
                         *reinterpret_cast<const v4f*>(&red[2][mm][c4])) +
                        *reinterpret_cast<const v4f*>(&red[3][mm][c4]);
        *reinterpret_cast<v4f*>(q_abs + ((int64_t)mm * H + h) * kQSmallKv + c0 + c4) = sum;
    }
}

// ---- 3d for decode-sized fp32 batches (M = B*Sq <= kOutSmallRows), with the fused
// attention's key-split merge folded in.  Two workgroups per head, 64 output columns each.
//   0. The loads go out in the order they are consumed: the rows' split maxima and sums
//      (lane s of a wave: split s), then the W_uv rows of the workgroup's columns (2 KB
//      each, contiguous in K: each 16-lane group of a wave takes four rows, its lanes'
//      16-byte loads covering 256 contiguous bytes per instruction), then the first
//      kOutBatch splits of the partials.  The W_uv stream runs under the merge.
//   1. Weights: wave w takes rows w and w + 4: m = max_s m_s, w_s = 2^(m_s - m),
//      L = sum_s w_s l_s (wave reductions); w_s and 1 / L go to LDS.
//   2. Merge: items are (row, 8 columns), M x 64 of them.  At M = 1 and 2 each item's
//      splits are dealt to 4 or 2 threads (split phases q, q + 4, ..), so that every thread
//      loads; at M > 4 a thread takes two items.  A unit sums its weighted partials in split
//      order, kOutBatch splits of loads in flight; the phases add in phase order through
//      LDS, and ctx_n = sum / L goes to LDS (a row without visible keys gives zeros, as the
//      3d GEMM does).  An unsplit pass gives ctx_n = ctx / row_sum.
//   3. out[m][h][n] = sum_k ctx_n[m][k] W_uv[h][n][k], reduced over the 16 lanes with four
//      DPP steps.
// This replaces flash_merge_kernel plus the 3d GEMM, whose 32-row MFMA tile is 1/32 .. 1/4
// full at M = 1 .. 8 (4.2 MFLOP of tile work per head, ~6.8 us at one CU's fp32 MFMA rate).
constexpr int kOutR = 512;
constexpr int kOutCols = 64;   // output columns per workgroup

template <class Op>
__device__ __forceinline__ float row16_reduce(float v, Op op) {
    v = op(v, dpp_move<0xB1>(v));   // lane ^ 1
    v = op(v, dpp_move<0x4E>(v));   // lane ^ 2
    v = op(v, dpp_move<0x141>(v));  // other quad of 8
    return op(v, dpp_move<0x140>(v));   // other half of 16
}

constexpr int kOutBatch = 8;   // splits of partial loads in flight per item

__global__ void __launch_bounds__(256) out_small_kernel(const float* __restrict__ o,
                                                        const float* __restrict__ mpart,
                                                        const float* __restrict__ lpart,
                                                        int n_split,
                                                        const float* __restrict__ ctx,
                                                        const float* __restrict__ rs,
                                                        const float* __restrict__ W,
                                                        float* __restrict__ out, int B, int Sq,
                                                        int H, int V) {
    __shared__ __attribute__((aligned(16))) float part[kOutSmallRows][kOutR];
    __shared__ float wts[kOutSmallRows][kOutSmallMaxSplit];
    __shared__ float invl[kOutSmallRows];
    __shared__ __attribute__((aligned(16))) float red[4][kOutR];   // split-phase sums
    const int col_blocks = (V + kOutCols - 1) / kOutCols;
    const int h = blockIdx.x / col_blocks, c0 = (blockIdx.x % col_blocks) * kOutCols;
    const int tid = threadIdx.x, wave = tid >> 6, lane = tid & 63;
    const int M = B * Sq, rows_b = Sq * H;
    const int64_t step = (int64_t)B * rows_b;   // between a row's split slots
    auto slot0 = [&](int mi) -> int64_t {
        return (int64_t)(mi / Sq) * rows_b + (int64_t)(mi % Sq) * H + h;
    };
    const bool split = n_split > 1;
    static_assert(kOutSmallRows <= 8, "two rows per wave for the weights, two items per thread");

    // 0a. split maxima and sums of rows wave and wave + 4
    float ms[2], lv[2];
    #pragma unroll
    for (int r = 0; r < 2; ++r) {
        const int mi = wave + 4 * r;
        ms[r] = -INFINITY;
        lv[r] = 0.f;
        if (split && mi < M && lane < n_split) {
            const int64_t sl = slot0(mi) + lane * step;
            ms[r] = mpart[sl];
            lv[r] = lpart[sl];
        }
    }
    // 0b. the W_uv rows: 16-lane group grp of wave w takes columns c0 + 16 w + grp + 4 j,
    // j = 0..3; lane li of the group holds floats 64 q + 4 li .. +3 (q = 0..7) of each row
    const int grp = lane >> 4, li = lane & 15;
    const float* Wh = W + (int64_t)h * V * kOutR;
    v4f wv[4][8];
    int nn[4];
    #pragma unroll
    for (int jr = 0; jr < 4; ++jr) {
        nn[jr] = c0 + 16 * wave + grp + 4 * jr;
        const v4f* wr = reinterpret_cast<const v4f*>(Wh + (int64_t)min(nn[jr], V - 1) * kOutR) + li;
        #pragma unroll
        for (int q = 0; q < 8; ++q) wv[jr][q] = wr[16 * q];
    }
    // 0c. the first splits of the partials of this thread's merge unit: item (row, 8
    // columns) it % items, splits q, q + qn, .. with q = it / items; qn = 4, 2, 1 split
    // phases per item at M = 1, 2, >= 3 so that all 256 threads load, and at M > 4 a second
    // item it + 256
    const int items = M * 64;
    const int qn = split ? max(1, min(4, 256 / items)) : 1;
    const int q = tid / items;   // split phase of the thread's first unit (>= qn: no unit)
    bool live[2];
    int imi[2], ich[2];
    const float* ibase[2];
    v4f pa[2][kOutBatch][2];
    #pragma unroll
    for (int j = 0; j < 2; ++j) {
        const int it = j == 0 ? tid % items : tid + 256;
        live[j] = split && (j == 0 ? q < qn : it < items);
        imi[j] = live[j] ? it >> 6 : 0;
        ich[j] = 8 * (it & 63);
        ibase[j] = o + (slot0(imi[j]) * kOutR + ich[j]);
    }
    const int q0 = live[0] ? q : 0;   // the second item (M > 4) has qn = 1, phase 0
    auto load_batch = [&](int k0) __attribute__((always_inline)) {
        #pragma unroll
        for (int j = 0; j < 2; ++j)
            #pragma unroll
            for (int sb = 0; sb < kOutBatch; ++sb) {
                const int sp = (j == 0 ? q0 : 0) + qn * (k0 + sb);
                if (live[j] && sp < n_split) {
                    const v4f* src = reinterpret_cast<const v4f*>(ibase[j] + sp * step * kOutR);
                    pa[j][sb][0] = src[0];
                    pa[j][sb][1] = src[1];
                }
            }
    };
    load_batch(0);

    // 1. the split weights
    #pragma unroll
    for (int r = 0; r < 2; ++r) {
        const int mi = wave + 4 * r;
        if (split && mi < M) {
            const float mx = wave_reduce(ms[r], OpMax{});
            const float w = (lane < n_split && ms[r] != -INFINITY) ? __builtin_amdgcn_exp2f(ms[r] - mx) : 0.f;
            const float L = wave_reduce(w * lv[r], OpSum{});
            if (lane < n_split) wts[mi][lane] = w;
            if (lane == 0) invl[mi] = L == 0.f ? 0.f : 1.f / L;
        }
    }
    __syncthreads();

    // 2. the merge (each unit's splits in order, the phases added in phase order), or the
    // unsplit pass's ctx / row_sum
    if (split) {
        v4f a[2][2];
        #pragma unroll
        for (int j = 0; j < 2; ++j) a[j][0] = a[j][1] = v4f{0.f, 0.f, 0.f, 0.f};
        const int per = (n_split + qn - 1) / qn;   // splits of a unit, at most
        for (int k0 = 0; k0 < per; k0 += kOutBatch) {
            if (k0 > 0) load_batch(k0);
            #pragma unroll
            for (int j = 0; j < 2; ++j)
                #pragma unroll
                for (int sb = 0; sb < kOutBatch; ++sb) {
                    const int sp = (j == 0 ? q0 : 0) + qn * (k0 + sb);
                    if (live[j] && sp < n_split) {
                        const float w = wts[imi[j]][sp];
                        a[j][0] += w * pa[j][sb][0];
                        a[j][1] += w * pa[j][sb][1];
                    }
                }
        }
        if (qn == 1) {
            #pragma unroll
            for (int j = 0; j < 2; ++j)
                if (live[j]) {
                    const float inv = invl[imi[j]];
                    *reinterpret_cast<v4f*>(&part[imi[j]][ich[j]]) = a[j][0] * inv;
                    *reinterpret_cast<v4f*>(&part[imi[j]][ich[j] + 4]) = a[j][1] * inv;
                }
        } else {
            // phase sums through LDS (qn * M <= 4 rows of red), then added in phase order
            if (live[0]) {
                *reinterpret_cast<v4f*>(&red[q * M + imi[0]][ich[0]]) = a[0][0];
                *reinterpret_cast<v4f*>(&red[q * M + imi[0]][ich[0] + 4]) = a[0][1];
            }
            __syncthreads();
            if (tid < items) {
                const int mi = tid >> 6, c = 8 * (tid & 63);
                v4f x0 = *reinterpret_cast<const v4f*>(&red[mi][c]);
                v4f x1 = *reinterpret_cast<const v4f*>(&red[mi][c + 4]);
                for (int qq = 1; qq < qn; ++qq) {
                    x0 += *reinterpret_cast<const v4f*>(&red[qq * M + mi][c]);
                    x1 += *reinterpret_cast<const v4f*>(&red[qq * M + mi][c + 4]);
                }
                *reinterpret_cast<v4f*>(&part[mi][c]) = x0 * invl[mi];
                *reinterpret_cast<v4f*>(&part[mi][c + 4]) = x1 * invl[mi];
            }
        }
    } else {
        for (int mi = wave; mi < M; mi += 4) {
            const int64_t r = slot0(mi);
            const float inv = rs[r] == 0.f ? 0.f : 1.f / rs[r];
            const v4f* src = reinterpret_cast<const v4f*>(ctx + r * kOutR) + 2 * lane;
            *reinterpret_cast<v4f*>(&part[mi][8 * lane]) = src[0] * inv;
            *reinterpret_cast<v4f*>(&part[mi][8 * lane + 4]) = src[1] * inv;
        }
    }
    __syncthreads();

    // 3. every ctx chunk read from LDS serves the group's four W_uv rows
    #pragma unroll
    for (int mi = 0; mi < kOutSmallRows; ++mi) {
        if (mi < M) {
            v4f acc[4];
            #pragma unroll
            for (int jr = 0; jr < 4; ++jr) acc[jr] = v4f{0.f, 0.f, 0.f, 0.f};
            #pragma unroll
            for (int q = 0; q < 8; ++q) {
                const v4f c = *reinterpret_cast<const v4f*>(&part[mi][64 * q + 4 * li]);
                #pragma unroll
                for (int jr = 0; jr < 4; ++jr) acc[jr] += wv[jr][q] * c;
            }
            #pragma unroll
            for (int jr = 0; jr < 4; ++jr) {
                const float sum = row16_reduce((acc[jr][0] + acc[jr][1]) + (acc[jr][2] + acc[jr][3]),
                                               OpSum{});
                if (li == 0 && nn[jr] < V) out[((int64_t)mi * H + h) * V + nn[jr]] = sum;
            }
        }
    }
}

}  // namespace

namespace {
// the split counts 2a1's plans use get the all-loads-first sum
template <int OUT>
hipError_t launch_rmsnorm_t(const float* in, int nsplit, int64_t split_stride, const void* gain,
                            void* out, int M, int N, float eps, hipStream_t stream,
                            const RopeTable& rt) {
    if (nsplit == 8)
        hipLaunchKernelGGL((rmsnorm_kernel<OUT, 8>), dim3(M), dim3(256), 0, stream, in, nsplit,
                           split_stride, gain, out, N, eps, rt);
    else if (nsplit == 16)
        hipLaunchKernelGGL((rmsnorm_kernel<OUT, 16>), dim3(M), dim3(256), 0, stream, in, nsplit,
                           split_stride, gain, out, N, eps, rt);
    else
        hipLaunchKernelGGL((rmsnorm_kernel<OUT, 0>), dim3(M), dim3(256), 0, stream, in, nsplit,
                           split_stride, gain, out, N, eps, rt);
    return hipGetLastError();
}
}  // namespace

hipError_t launch_rmsnorm(const float* in, int nsplit, int64_t split_stride, const void* gain,
                          void* out, OutType out_type, int M, int N, float eps,
                          hipStream_t stream, const RopeTable& rt) {
    if (M <= 0) return hipSuccess;
    if (rt.cos_sin && (rt.half <= 0 || rt.half > 256 || !rt.positions || !rt.inv_freq || rt.Sq < 1))
        return hipErrorInvalidValue;
    if (out_type == kOutF32) return launch_rmsnorm_t<kOutF32>(in, nsplit, split_stride, gain, out, M, N, eps, stream, rt);
    if (out_type == kOutBF16) return launch_rmsnorm_t<kOutBF16>(in, nsplit, split_stride, gain, out, M, N, eps, stream, rt);
    return launch_rmsnorm_t<kOutF16>(in, nsplit, split_stride, gain, out, M, N, eps, stream, rt);
}

hipError_t launch_rope(const float* q_raw, const int64_t* positions, const float* inv_freq,
                       void* q_rope, OutType out_type, int B, int Sq, int H, int nope, int rope,
                       hipStream_t stream, bool pos_per_batch, int nsplit, int64_t split_stride,
                       float* nope_out) {
    if ((int64_t)B * Sq <= 0 || H <= 0) return hipSuccess;
    if (rope / 2 > kRopeMaxHalf || nsplit < 1) return hipErrorInvalidValue;
    if (nope_out && nope % 4 != 0) return hipErrorInvalidValue;   // float4 nope columns
    // the split sum reads nsplit times the row's bytes: more, smaller workgroups
    const int hpw = nope_out ? kRopeSumHeads : kRopeHeads;
    const dim3 grid(B * Sq, (H + hpw - 1) / hpw);
    if (out_type == kOutF32)
        hipLaunchKernelGGL(rope_kernel<kOutF32>, grid, dim3(256), 0, stream, q_raw, nsplit, split_stride, nope_out, positions,
                           inv_freq, q_rope, Sq, H, nope, rope, pos_per_batch ? 1 : 0);
    else if (out_type == kOutBF16)
        hipLaunchKernelGGL(rope_kernel<kOutBF16>, grid, dim3(256), 0, stream, q_raw, nsplit, split_stride, nope_out, positions,
                           inv_freq, q_rope, Sq, H, nope, rope, pos_per_batch ? 1 : 0);
    else
        hipLaunchKernelGGL(rope_kernel<kOutF16>, grid, dim3(256), 0, stream, q_raw, nsplit, split_stride, nope_out, positions,
                           inv_freq, q_rope, Sq, H, nope, rope, pos_per_batch ? 1 : 0);
    return hipGetLastError();
}

hipError_t launch_combine(const float* m_part, const float* l_part, float* alpha,
                          float* row_sum, float* row_max, int rows, int P, hipStream_t stream) {
    if (rows <= 0) return hipSuccess;
    hipLaunchKernelGGL(combine_kernel, dim3((rows + 3) / 4), dim3(256), 0, stream, m_part,
                       l_part, alpha, row_sum, row_max, rows, P);
    return hipGetLastError();
}

hipError_t launch_stream_merge(float* ctx, float* run_max, float* run_sum, const float* ctx_c,
                               const float* max_c, const float* sum_c, int rows, int R,
                               bool first, hipStream_t stream) {
    if (rows <= 0) return hipSuccess;
    hipLaunchKernelGGL(stream_merge_kernel, dim3((rows + 3) / 4), dim3(256), 0, stream, ctx,
                       run_max, run_sum, ctx_c, max_c, sum_c, rows, R, first ? 1 : 0);
    return hipGetLastError();
}

hipError_t launch_kv_append(const float* in, int nsplit, int64_t split_stride, const void* gain,
                            const int64_t* positions, const float* inv_freq, void* c_kv,
                            void* pe, OutType out_type, int B, int Sq, int R, int D,
                            int start_row, int cache_rows, float eps, hipStream_t stream,
                            bool pos_per_batch, const int* block_table, int page_size,
                            int max_pages) {
    if (block_table && (page_size <= 0 || max_pages <= 0)) return hipErrorInvalidValue;
    const int64_t rows = (int64_t)B * Sq;
    if (rows <= 0) return hipSuccess;
    if (rows > 0x7fffffff) return hipErrorInvalidValue;
    if (out_type == kOutF32)
        hipLaunchKernelGGL(kv_append_kernel<kOutF32>, dim3((unsigned)rows), dim3(256), 0, stream,
                           in, nsplit, split_stride, gain, positions, inv_freq, c_kv, pe, Sq, R,
                           D, start_row, cache_rows, pos_per_batch ? 1 : 0, block_table,
                           page_size, max_pages, eps);
    else if (out_type == kOutBF16)
        hipLaunchKernelGGL(kv_append_kernel<kOutBF16>, dim3((unsigned)rows), dim3(256), 0, stream,
                           in, nsplit, split_stride, gain, positions, inv_freq, c_kv, pe, Sq, R,
                           D, start_row, cache_rows, pos_per_batch ? 1 : 0, block_table,
                           page_size, max_pages, eps);
    else
        hipLaunchKernelGGL(kv_append_kernel<kOutF16>, dim3((unsigned)rows), dim3(256), 0, stream,
                           in, nsplit, split_stride, gain, positions, inv_freq, c_kv, pe, Sq, R,
                           D, start_row, cache_rows, pos_per_batch ? 1 : 0, block_table,
                           page_size, max_pages, eps);
    return hipGetLastError();
}

hipError_t launch_fp8_dequant(const void* codes, int64_t n, float scale, float* out,
                              hipStream_t stream) {
    if (n <= 0) return hipSuccess;
    const int64_t threads = (n + 3) / 4;
    const int blocks = (int)std::min<int64_t>((threads + 255) / 256, 16 * kNumCUs);
    hipLaunchKernelGGL(fp8_dequant_kernel, dim3(blocks), dim3(256), 0, stream,
                       static_cast<const uint8_t*>(codes), n, scale, out);
    return hipGetLastError();
}

hipError_t launch_split_rows(const void* src, void* dst_a, void* dst_b, int64_t groups,
                             int rows_a, int rows_b, int64_t row_bytes, hipStream_t stream) {
    if (groups <= 0 || row_bytes % 16 != 0) return hipErrorInvalidValue;
    const int chunks = (int)(row_bytes / 16);
    const int64_t rows = groups * (rows_a + rows_b);
    const int64_t total = rows * chunks;
    const int blocks = (int)std::min<int64_t>((total + 255) / 256, 16 * kNumCUs);
    hipLaunchKernelGGL(split_rows_kernel, dim3(blocks), dim3(256), 0, stream,
                       static_cast<const v4u_t*>(src), static_cast<v4u_t*>(dst_a),
                       static_cast<v4u_t*>(dst_b), rows, rows_a, rows_a + rows_b, chunks);
    return hipGetLastError();
}


hipError_t launch_q_small(const float* q_parts, int nsplit, int64_t split_stride,
                          const int64_t* positions, const float* inv_freq, const float* W_uk,
                          float* q_rope, float* q_abs, int B, int Sq, int H, int nope, int rope,
                          int kv, bool pos_per_batch, hipStream_t stream) {
    const int M = B * Sq;
    if (M < 1 || M > kQSmallRows || H <= 0 || nope != kQSmallNope || kv != kQSmallKv ||
        rope <= 0 || rope % 2 != 0 || (int64_t)M * (rope / 2) > 256 || nsplit < 1 ||
        nsplit > kQSmallMaxSplit)
        return hipErrorInvalidValue;
    hipLaunchKernelGGL(q_small_kernel, dim3(2 * H), dim3(256), 0, stream, q_parts, nsplit,
                       split_stride, positions, inv_freq, W_uk, q_rope, q_abs, Sq, M, H, rope,
                       pos_per_batch ? 1 : 0);
    return hipGetLastError();
}

hipError_t launch_out_small(const FlashPartials& fp, const float* ctx, const float* row_sum,
                            const float* W_uv, float* out, int B, int Sq, int H, int R, int V,
                            hipStream_t stream) {
    const int M = B * Sq;
    // each workgroup's 4 waves x 4 groups x 4 rows cover its kOutCols columns
    static_assert(kOutCols == 4 * 4 * 4, "column coverage");
    if (M < 1 || M > kOutSmallRows || R != kOutR || H <= 0 || V <= 0 ||
        fp.n_split > kOutSmallMaxSplit)
        return hipErrorInvalidValue;
    if (fp.n_split > 1 ? !(fp.o && fp.m && fp.l) : !(ctx && row_sum)) return hipErrorInvalidValue;
    const int col_blocks = (V + kOutCols - 1) / kOutCols;
    hipLaunchKernelGGL(out_small_kernel, dim3(H * col_blocks), dim3(256), 0, stream, fp.o, fp.m, fp.l,
                       fp.n_split, ctx, row_sum, W_uv, out, B, Sq, H, V);
    return hipGetLastError();
}

}  // namespace mla
