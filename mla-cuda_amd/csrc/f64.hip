// Float64 storage (MLA_DTYPE_F64).  The reference dispatches double through both of its
// launches (mla_kernels.cu:674, 1561: AT_DISPATCH_FLOATING_TYPES_AND_HALF) and keeps every
// intermediate in the accumulate dtype, double for double inputs (mla_kernels.cu:118-120);
// its dtype check holds the double path to 1e-13 of the output's largest element
// (check_dtypes.py:23-38).  Here the double path is the reference's per-step decomposition
// in double throughout:
//
//   Q path      2a1 GEMM -> 2a-n RMSNorm -> 2a2 GEMM -> 2b RoPE -> 2c GEMM (per head)
//   attention   3a scores = q_abs . c_kv^T + q_rope . pe^T (two GEMMs into one buffer)
//               -> row softmax of scores / scale (causal mask applied) -> 3c ctx = P . c_kv
//               -> 3d out = ctx . W_uv^T (per head)
//
// Every contraction runs on one strided-batched GEMM kernel on gfx950's double MFMA,
// v_mfma_f64_16x16x4_f64.  The row kernels reduce on wave64 shuffles.  Throughput is not
// the point of this path (the fp32 and 16-bit paths are): it exists so a caller passing
// double gets the reference's double semantics.
#include "kernels.h"

#include <math.h>

namespace mla {
namespace {

typedef double v4d __attribute__((ext_vector_type(4)));

constexpr int kBM = 64, kBN = 64, kBK = 16;   // workgroup tile, K slice
constexpr int kThreads = 256;                  // four waves, each a 32 x 32 quarter

// D(16x16) += A(16x4) B(4x16) in double.  Lane l supplies A[l%16][l/16] and B[l/16][l%16];
// accumulator r of lane l is D[l/16 + 4*r][l%16] -- rows strided by 4 across the registers,
// unlike the fp32 MFMAs' consecutive rows (measured on gfx950 with random operands).
__device__ __forceinline__ v4d mfma_f64(double a, double b, v4d c) {
    return __builtin_amdgcn_mfma_f64_16x16x4f64(a, b, c, 0, 0, 0);
}

// C[g] = alpha * A[g] . op(B[g]) + beta * C[g]; grid (ceil(N/64), ceil(M/64), G).
// Every global access is guarded by the problem bounds; tiles past them read zeros.
__global__ void __launch_bounds__(kThreads)
gemm64_kernel(Gemm64Problem p) {
    __shared__ double As[kBM][kBK + 1];
    __shared__ double Bs[kBK][kBN + 1];
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int m0 = blockIdx.y * kBM, n0 = blockIdx.x * kBN;
    const int64_t g = blockIdx.z;
    const double* A = p.A + g * p.sA;
    const double* B = p.B + g * p.sB;
    double* C = p.C + g * p.sC;
    const int wm = (wave >> 1) * 32, wn = (wave & 1) * 32;
    v4d acc[2][2];
    for (int i = 0; i < 2; ++i)
        for (int j = 0; j < 2; ++j) acc[i][j] = v4d{0.0, 0.0, 0.0, 0.0};

    for (int k0 = 0; k0 < p.K; k0 += kBK) {
        // A tile: row tid/4, k (tid%4)*4 .. +3
        {
            const int r = tid >> 2, kk = (tid & 3) * 4;
            const int m = m0 + r;
            for (int e = 0; e < 4; ++e) {
                const int k = k0 + kk + e;
                As[r][kk + e] = (m < p.M && k < p.K) ? A[(int64_t)m * p.lda + k] : 0.0;
            }
        }
        if (!p.b_nt) {   // B[k][n]: k row tid/16, columns (tid%16)*4 .. +3
            const int kr = tid >> 4, c = (tid & 15) * 4;
            const int k = k0 + kr;
            for (int e = 0; e < 4; ++e) {
                const int n = n0 + c + e;
                Bs[kr][c + e] = (k < p.K && n < p.N) ? B[(int64_t)k * p.ldb + n] : 0.0;
            }
        } else {         // B[n][k]: column tid/4, k (tid%4)*4 .. +3
            const int c = tid >> 2, kk = (tid & 3) * 4;
            const int n = n0 + c;
            for (int e = 0; e < 4; ++e) {
                const int k = k0 + kk + e;
                Bs[kk + e][c] = (n < p.N && k < p.K) ? B[(int64_t)n * p.ldb + k] : 0.0;
            }
        }
        __syncthreads();
        for (int q = 0; q < kBK / 4; ++q) {
            const int kq = q * 4 + (lane >> 4);
            double a[2], b[2];
            for (int i = 0; i < 2; ++i) a[i] = As[wm + i * 16 + (lane & 15)][kq];
            for (int j = 0; j < 2; ++j) b[j] = Bs[kq][wn + j * 16 + (lane & 15)];
            for (int i = 0; i < 2; ++i)
                for (int j = 0; j < 2; ++j) acc[i][j] = mfma_f64(a[i], b[j], acc[i][j]);
        }
        __syncthreads();
    }
    for (int i = 0; i < 2; ++i)
        for (int j = 0; j < 2; ++j)
            for (int r = 0; r < 4; ++r) {
                const int m = m0 + wm + i * 16 + (lane >> 4) + 4 * r;
                const int n = n0 + wn + j * 16 + (lane & 15);
                if (m < p.M && n < p.N) {
                    double* c = C + (int64_t)m * p.ldc + n;
                    const double v = p.alpha * acc[i][j][r];
                    *c = p.beta != 0.0 ? v + p.beta * *c : v;
                }
            }
}

// Sum and max over a 256-thread workgroup (wave64 shuffles, then the four wave results).
__device__ double block_sum(double v, double* red) {
    for (int o = 32; o > 0; o >>= 1) v += __shfl_xor(v, o);
    const int wave = threadIdx.x >> 6;
    __syncthreads();
    if ((threadIdx.x & 63) == 0) red[wave] = v;
    __syncthreads();
    return (red[0] + red[1]) + (red[2] + red[3]);
}
__device__ double block_max(double v, double* red) {
    for (int o = 32; o > 0; o >>= 1) v = fmax(v, __shfl_xor(v, o));
    const int wave = threadIdx.x >> 6;
    __syncthreads();
    if ((threadIdx.x & 63) == 0) red[wave] = v;
    __syncthreads();
    return fmax(fmax(red[0], red[1]), fmax(red[2], red[3]));
}

// 2a-n, one workgroup per row, in place: x = (x * (1 / sqrt(mean(x^2) + eps))) * gain
// (exhaustive_benchmark_suite.py:252-258; double needs no rounding between the factors).
__global__ void __launch_bounds__(kThreads)
rmsnorm64_kernel(double* x, const double* gain, int N, double eps) {
    __shared__ double red[4];
    double* row = x + (int64_t)blockIdx.x * N;
    double ss = 0.0;
    for (int i = threadIdx.x; i < N; i += kThreads) ss += row[i] * row[i];
    ss = block_sum(ss, red);
    const double inv = 1.0 / sqrt(ss / N + eps);
    for (int i = threadIdx.x; i < N; i += kThreads) row[i] = (row[i] * inv) * gain[i];
}

// 2b: q_rope[m, h, 2i | 2i+1] from q_raw[m, h*(nope+rope) + nope + 2i | +1], rotated by
// positions[s] (or positions[m] per sequence) * inv_freq[i]
// (exhaustive_benchmark_suite.py:210-232: even' = e cos - o sin, odd' = e sin + o cos).
__global__ void __launch_bounds__(kThreads)
rope64_kernel(const double* q_raw, const int64_t* pos, const double* inv_freq, double* q_rope,
              int64_t n_pairs, int Sq, int H, int nope, int rope, int per_batch) {
    const int64_t t = (int64_t)blockIdx.x * kThreads + threadIdx.x;
    if (t >= n_pairs) return;
    const int half = rope / 2;
    const int i = (int)(t % half);
    const int64_t mh = t / half;            // m * H + h
    const int h = (int)(mh % H);
    const int64_t m = mh / H;
    const int s = (int)(m % Sq);
    const double ang = (double)pos[per_batch ? m : s] * inv_freq[i];
    const double c = cos(ang), sn = sin(ang);
    const double* src = q_raw + m * (int64_t)H * (nope + rope) + (int64_t)h * (nope + rope) + nope;
    const double e = src[2 * i], o = src[2 * i + 1];
    double* dst = q_rope + mh * rope;
    dst[2 * i] = e * c - o * sn;
    dst[2 * i + 1] = e * sn + o * c;
}

// Between 3a and 3c, one workgroup per score row (row = (b*Sq + s)*H + h): t = x / scale,
// softmax over the keys the row sees (all Sk, or j <= Sk - Sq + s with the causal mask),
// written in place; masked keys get 0.
__global__ void __launch_bounds__(kThreads)
softmax64_kernel(double* S, int Sk, int Sq, int H, double scale, int causal) {
    __shared__ double red[4];
    const int64_t row = blockIdx.x;
    const int s = (int)((row / H) % Sq);
    const int lim = causal ? Sk - Sq + s + 1 : Sk;
    double* r = S + row * Sk;
    double mx = -INFINITY;
    for (int j = threadIdx.x; j < lim; j += kThreads) mx = fmax(mx, r[j] / scale);
    mx = block_max(mx, red);
    double sum = 0.0;
    for (int j = threadIdx.x; j < lim; j += kThreads) {
        const double e = exp(r[j] / scale - mx);
        r[j] = e;
        sum += e;
    }
    sum = block_sum(sum, red);
    for (int j = threadIdx.x; j < Sk; j += kThreads) r[j] = j < lim ? r[j] / sum : 0.0;
}

}  // namespace

hipError_t launch_gemm64(const Gemm64Problem& p, hipStream_t stream) {
    if (p.M <= 0 || p.N <= 0 || p.G <= 0) return hipSuccess;
    const dim3 grid((p.N + kBN - 1) / kBN, (p.M + kBM - 1) / kBM, p.G);
    hipLaunchKernelGGL(gemm64_kernel, grid, dim3(kThreads), 0, stream, p);
    return hipGetLastError();
}

hipError_t launch_rmsnorm64(double* x, const double* gain, int M, int N, double eps,
                            hipStream_t stream) {
    hipLaunchKernelGGL(rmsnorm64_kernel, dim3(M), dim3(kThreads), 0, stream, x, gain, N, eps);
    return hipGetLastError();
}

hipError_t launch_rope64(const double* q_raw, const int64_t* pos, const double* inv_freq,
                         double* q_rope, int B, int Sq, int H, int nope, int rope,
                         bool per_batch, hipStream_t stream) {
    const int64_t n_pairs = (int64_t)B * Sq * H * (rope / 2);
    const int64_t blocks = (n_pairs + kThreads - 1) / kThreads;
    hipLaunchKernelGGL(rope64_kernel, dim3((unsigned)blocks), dim3(kThreads), 0, stream, q_raw,
                       pos, inv_freq, q_rope, n_pairs, Sq, H, nope, rope, per_batch ? 1 : 0);
    return hipGetLastError();
}

hipError_t launch_softmax64(double* S, int rows, int Sk, int Sq, int H, double scale,
                            bool causal, hipStream_t stream) {
    hipLaunchKernelGGL(softmax64_kernel, dim3(rows), dim3(kThreads), 0, stream, S, Sk, Sq, H,
                       scale, causal ? 1 : 0);
    return hipGetLastError();
}

}  // namespace mla
