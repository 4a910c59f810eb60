// Dense per-layer projection Z = X W_all with the attention dots
// L[i,h] = Z[i,h,:] . aL[h], R[i,h] = Z[i,h,:] . aR[h].
//
// Reference: projection (baseline/src/baseline_standard.cpp:3-6, one all-head
// GEMM, cblas_sgemm or cblas_gemm_bf16bf16f32), lr_from_z (:7-20) and the
// FP32 -> bf16 RNE convert (baseline/src/common.cpp:80-93).  The reordered
// front end LR = X (W a) of the aggregate-first path follows lr_reordered
// (baseline_standard.cpp:29-43) and prepare_attention
// (implementation/src/gat_tfs_online.cpp:48-73).
#include "internal.hpp"

namespace gatgpu {
namespace {

constexpr int kThreads = 256;

__global__ void __launch_bounds__(kThreads)
k_to_bf16(const float* __restrict__ x, uint16_t* __restrict__ y, uint64_t count) {
    for (uint64_t i = blockIdx.x * uint64_t(kThreads) + threadIdx.x; i < count;
         i += uint64_t(gridDim.x) * kThreads)
        y[i] = bf16_rne(x[i]);
}

// x [n][d] FP32 -> y [n][dp] bf16, columns d..dp-1 zero.
__global__ void __launch_bounds__(kThreads)
k_to_bf16_pad(const float* __restrict__ x, uint16_t* __restrict__ y, uint64_t n, int d, int dp) {
    const uint64_t count = n * uint64_t(dp);
    for (uint64_t i = blockIdx.x * uint64_t(kThreads) + threadIdx.x; i < count;
         i += uint64_t(gridDim.x) * kThreads) {
        const uint64_t r = i / dp;
        const int c = int(i - r * dp);
        y[i] = c < d ? bf16_rne(x[r * d + c]) : uint16_t(0);
    }
}

__global__ void __launch_bounds__(kThreads)
k_widen_bf16(const uint16_t* __restrict__ x, float* __restrict__ y, uint64_t count) {
    for (uint64_t i = blockIdx.x * uint64_t(kThreads) + threadIdx.x; i < count;
         i += uint64_t(gridDim.x) * kThreads)
        y[i] = bf16_widen(x[i]);
}

__device__ inline float ldx(const float* x32, const uint16_t* xbf, uint64_t idx) {
    return xbf ? bf16_widen(xbf[idx]) : x32[idx];
}

// 64x64 output tile per block, 16-deep K steps through LDS, 4x4 per thread.
// X rows index blockIdx.x (2^31 limit), output column tiles blockIdx.y.
__global__ void __launch_bounds__(kThreads)
k_gemm_tiled(const float* __restrict__ x32, const uint16_t* __restrict__ xbf, const float* __restrict__ w,
             float* __restrict__ z, uint64_t n, int D, int W, int zs) {
    __shared__ float As[16][64 + 4];
    __shared__ float Bs[16][64];
    const int tx = threadIdx.x % 16, ty = threadIdx.x / 16;
    const uint64_t row0 = uint64_t(blockIdx.x) * 64;
    const int col0 = blockIdx.y * 64;
    float acc[4][4] = {};
    for (int k0 = 0; k0 < D; k0 += 16) {
#pragma unroll
        for (int u = 0; u < 4; ++u) {
            const int q = threadIdx.x + kThreads * u;
            const int r = q / 16, kk = q % 16;
            const uint64_t gr = row0 + r;
            const int gk = k0 + kk;
            As[kk][r] = (gr < n && gk < D) ? ldx(x32, xbf, gr * D + gk) : 0.0f;
            const int kk2 = q / 64, c = q % 64;
            const int gk2 = k0 + kk2, gc = col0 + c;
            Bs[kk2][c] = (gk2 < D && gc < W) ? w[size_t(gk2) * W + gc] : 0.0f;
        }
        __syncthreads();
#pragma unroll
        for (int kk = 0; kk < 16; ++kk) {
            float av[4], bv[4];
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                av[i] = As[kk][ty * 4 + i];
                bv[i] = Bs[kk][tx * 4 + i];
            }
#pragma unroll
            for (int i = 0; i < 4; ++i)
#pragma unroll
                for (int j = 0; j < 4; ++j) acc[i][j] += av[i] * bv[j];
        }
        __syncthreads();
    }
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        const uint64_t gr = row0 + ty * 4 + i;
        if (gr >= n) continue;
#pragma unroll
        for (int j = 0; j < 4; ++j) {
            const int gc = col0 + tx * 4 + j;
            if (gc < W) z[gr * zs + gc] = acc[i][j];
        }
    }
}

// One thread per (row, head): the dots of lr_from_z, then the optional bf16 store of Z.
__global__ void __launch_bounds__(kThreads)
k_lr_from_z(const float* __restrict__ z, uint64_t n, int K, int dim, int zs, const float* __restrict__ al,
            const float* __restrict__ ar, float* __restrict__ left, float* __restrict__ right) {
    const uint64_t t = blockIdx.x * uint64_t(kThreads) + threadIdx.x;
    if (t >= n * K) return;
    const uint64_t i = t / K;
    const int h = int(t % K);
    const float* zi = z + i * zs + h * dim;
    float l = 0.0f, r = 0.0f;
    for (int d = 0; d < dim; ++d) {
        l += zi[d] * al[h * dim + d];
        r += zi[d] * ar[h * dim + d];
    }
    left[t] = l;
    right[t] = r;
}

// One thread per (row, column of B_LR): LR = X B_LR, B_LR = [b_L | b_R] [D][2K].
__global__ void __launch_bounds__(kThreads)
k_lr_reordered(const float* __restrict__ x32, const uint16_t* __restrict__ xbf,
               const float* __restrict__ blr, uint64_t n, int D, int K, float* __restrict__ left,
               float* __restrict__ right) {
    const uint64_t t = blockIdx.x * uint64_t(kThreads) + threadIdx.x;
    if (t >= n * 2 * K) return;
    const uint64_t i = t / (2 * K);
    const int c = int(t % (2 * K));
    float s = 0.0f;
    for (int k = 0; k < D; ++k) s += ldx(x32, xbf, i * D + k) * blr[size_t(k) * 2 * K + c];
    if (c < K) left[i * K + c] = s;
    else right[i * K + c - K] = s;
}

uint32_t grid_for(uint64_t items, uint32_t cap) {
    uint64_t g = (items + kThreads - 1) / kThreads;
    if (g < 1) g = 1;
    return uint32_t(g > cap ? cap : g);
}

}  // namespace

hipError_t launch_to_bf16(const float* x, uint16_t* y, uint64_t count, hipStream_t s) {
    k_to_bf16<<<grid_for(count, 1u << 16), kThreads, 0, s>>>(x, y, count);
    return hipGetLastError();
}

hipError_t launch_to_bf16_pad(const float* x, uint16_t* y, uint64_t n, int d, int dp, hipStream_t s) {
    if (dp == d) return launch_to_bf16(x, y, n * uint64_t(d), s);
    k_to_bf16_pad<<<grid_for(n * uint64_t(dp), 1u << 16), kThreads, 0, s>>>(x, y, n, d, dp);
    return hipGetLastError();
}

hipError_t launch_widen_bf16(const uint16_t* x, float* y, uint64_t count, hipStream_t s) {
    k_widen_bf16<<<grid_for(count, 1u << 16), kThreads, 0, s>>>(x, y, count);
    return hipGetLastError();
}

hipError_t launch_projection(const float* x32, const uint16_t* xbf, const float* w, uint64_t n,
                             int in, int heads, int dim, const float* al, const float* ar,
                             float* z32, uint16_t* zbf, float* left, float* right, float* zscratch,
                             int zs, hipStream_t s) {
    const int W = heads * dim;
    float* zf = z32 ? z32 : zscratch;
    if (!zf) return hipErrorInvalidValue;
    dim3 grid(uint32_t((n + 63) / 64), uint32_t((W + 63) / 64));
    k_gemm_tiled<<<grid, kThreads, 0, s>>>(x32, xbf, w, zf, n, in, W, zs);
    hipError_t err = hipGetLastError();
    if (err != hipSuccess) return err;
    const uint64_t pairs = n * uint64_t(heads);
    k_lr_from_z<<<dim3(uint32_t((pairs + kThreads - 1) / kThreads)), kThreads, 0, s>>>(zf, n, heads, dim, zs,
                                                                                       al, ar, left, right);
    if ((err = hipGetLastError()) != hipSuccess) return err;
    if (zbf) return launch_to_bf16(zf, zbf, n * uint64_t(zs), s);
    return hipSuccess;
}

hipError_t launch_lr_reordered(const float* x32, const uint16_t* xbf, const float* blr,
                               uint64_t n, int in, int heads, float* left, float* right,
                               hipStream_t s) {
    const uint64_t items = n * 2 * uint64_t(heads);
    k_lr_reordered<<<dim3(uint32_t((items + kThreads - 1) / kThreads)), kThreads, 0, s>>>(
        x32, xbf, blr, n, in, heads, left, right);
    return hipGetLastError();
}

}  // namespace gatgpu
