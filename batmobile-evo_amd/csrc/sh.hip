// Spherical harmonics, L_max = 0..6: forward and backward.
//
// One thread per edge vector, 256 edges per workgroup.  Inputs and outputs are
// staged through LDS so that every global access is a contiguous,
// wave-coalesced stream (the [E,3] and [E,(L+1)^2] row-major rows are 12 B and
// 4*(L+1)^2 B wide, which per-thread row accesses would scatter over many
// cache lines per instruction).  LDS rows are padded to an odd stride, so the
// per-thread row accesses are bank-conflict free.
//
// Replaces reference src/spherical_harmonics/spherical_harmonics.cu:33-314 and
// spherical_harmonics_backward.cu:25-463.
#include "common.h"
#include "batmobile_hip.h"

namespace bmhip {

constexpr int kShBlock = 256;

__host__ __device__ constexpr int odd_stride(int k) { return k | 1; }

template <int L, bool NORM>
__global__ __launch_bounds__(kShBlock) void sh_forward_kernel(const float* __restrict__ v,
                                                                float* __restrict__ Y, int64_t n) {
    constexpr int K = sh_dim(L);
    constexpr int KS = odd_stride(K);
    __shared__ float sv[kShBlock * 3];
    __shared__ float sy[kShBlock * KS];
    const int64_t base = (int64_t)blockIdx.x * kShBlock;
    const int rows = (int)min<int64_t>(kShBlock, n - base);
    const int tid = threadIdx.x;
    for (int i = tid; i < rows * 3; i += kShBlock) sv[i] = v[base * 3 + i];
    __syncthreads();
    if (tid < rows) {
        float x = sv[tid * 3 + 0], y = sv[tid * 3 + 1], z = sv[tid * 3 + 2];
        if constexpr (NORM) normalize3(x, y, z);
        float out[K];
        sh_forward<L>(x, y, z, out);
#pragma unroll
        for (int k = 0; k < K; ++k) sy[tid * KS + k] = out[k];
    }
    __syncthreads();
    float* dst = Y + base * K;
    for (int i = tid; i < rows * K; i += kShBlock) {
        const int r = i / K;
        dst[i] = sy[r * KS + (i - r * K)];
    }
}

// grad_xyz = sum_k g_k dY_k/d(x,y,z).  With NORM the input is the raw vector v,
// Y is taken at u = v/|v| and the result is chained through the normalisation:
// (g_u - u (u . g_u)) / |v|   (reference python/batmobile/autograd.py:62-92).
template <int L, bool NORM>
__global__ __launch_bounds__(kShBlock) void sh_backward_kernel(const float* __restrict__ v,
                                                                 const float* __restrict__ gY,
                                                                 float* __restrict__ gv, int64_t n) {
    constexpr int K = sh_dim(L);
    constexpr int KS = odd_stride(K);
    __shared__ float sv[kShBlock * 3];
    __shared__ float sg[kShBlock * KS];
    const int64_t base = (int64_t)blockIdx.x * kShBlock;
    const int rows = (int)min<int64_t>(kShBlock, n - base);
    const int tid = threadIdx.x;
    for (int i = tid; i < rows * 3; i += kShBlock) sv[i] = v[base * 3 + i];
    const float* src = gY + base * K;
    for (int i = tid; i < rows * K; i += kShBlock) {
        const int r = i / K;
        sg[r * KS + (i - r * K)] = src[i];
    }
    __syncthreads();
    float res[3] = {0.0f, 0.0f, 0.0f};
    if (tid < rows) {
        float x = sv[tid * 3 + 0], y = sv[tid * 3 + 1], z = sv[tid * 3 + 2];
        float r = 1.0f;
        if constexpr (NORM) r = normalize3(x, y, z);
        float Yv[K], g[K];
        sh_forward<L>(x, y, z, Yv);
#pragma unroll
        for (int k = 0; k < K; ++k) g[k] = sg[tid * KS + k];
        float gx, gy, gz;
        sh_backward<L>(x, y, z, Yv, g, gx, gy, gz);
        if constexpr (NORM) {
            const float dot = x * gx + y * gy + z * gz;
            const float inv = 1.0f / r;
            gx = (gx - x * dot) * inv;
            gy = (gy - y * dot) * inv;
            gz = (gz - z * dot) * inv;
        }
        res[0] = gx;
        res[1] = gy;
        res[2] = gz;
    }
    __syncthreads();
    if (tid < rows) {
        sv[tid * 3 + 0] = res[0];
        sv[tid * 3 + 1] = res[1];
        sv[tid * 3 + 2] = res[2];
    }
    __syncthreads();
    for (int i = tid; i < rows * 3; i += kShBlock) gv[base * 3 + i] = sv[i];
}

template <bool NORM>
static int launch_sh_forward(const float* v, float* Y, int64_t n, int L, hipStream_t s) {
    const dim3 grid((unsigned)ceil_div(n, kShBlock));
    switch (L) {
        case 0: sh_forward_kernel<0, NORM><<<grid, kShBlock, 0, s>>>(v, Y, n); break;
        case 1: sh_forward_kernel<1, NORM><<<grid, kShBlock, 0, s>>>(v, Y, n); break;
        case 2: sh_forward_kernel<2, NORM><<<grid, kShBlock, 0, s>>>(v, Y, n); break;
        case 3: sh_forward_kernel<3, NORM><<<grid, kShBlock, 0, s>>>(v, Y, n); break;
        case 4: sh_forward_kernel<4, NORM><<<grid, kShBlock, 0, s>>>(v, Y, n); break;
        case 5: sh_forward_kernel<5, NORM><<<grid, kShBlock, 0, s>>>(v, Y, n); break;
        case 6: sh_forward_kernel<6, NORM><<<grid, kShBlock, 0, s>>>(v, Y, n); break;
        default: return BM_ERR_ARG;
    }
    return (int)hipGetLastError();
}

template <bool NORM>
static int launch_sh_backward(const float* v, const float* g, float* gv, int64_t n, int L,
                              hipStream_t s) {
    const dim3 grid((unsigned)ceil_div(n, kShBlock));
    switch (L) {
        case 0: sh_backward_kernel<0, NORM><<<grid, kShBlock, 0, s>>>(v, g, gv, n); break;
        case 1: sh_backward_kernel<1, NORM><<<grid, kShBlock, 0, s>>>(v, g, gv, n); break;
        case 2: sh_backward_kernel<2, NORM><<<grid, kShBlock, 0, s>>>(v, g, gv, n); break;
        case 3: sh_backward_kernel<3, NORM><<<grid, kShBlock, 0, s>>>(v, g, gv, n); break;
        case 4: sh_backward_kernel<4, NORM><<<grid, kShBlock, 0, s>>>(v, g, gv, n); break;
        case 5: sh_backward_kernel<5, NORM><<<grid, kShBlock, 0, s>>>(v, g, gv, n); break;
        case 6: sh_backward_kernel<6, NORM><<<grid, kShBlock, 0, s>>>(v, g, gv, n); break;
        default: return BM_ERR_ARG;
    }
    return (int)hipGetLastError();
}

}  // namespace bmhip

using namespace bmhip;

extern "C" int batteries_spherical_harmonics(const float* edge_vectors, float* Y_lm, int64_t N,
                                             int L_max, int normalize, hipStream_t stream) {
    if (N < 0 || L_max < 0 || L_max > 6) return BM_ERR_ARG;
    if (N == 0) return BM_OK;
    if (!edge_vectors || !Y_lm) return BM_ERR_ARG;
    return normalize ? launch_sh_forward<true>(edge_vectors, Y_lm, N, L_max, stream)
                     : launch_sh_forward<false>(edge_vectors, Y_lm, N, L_max, stream);
}

extern "C" int batteries_spherical_harmonics_backward(const float* edge_vectors,
                                                      const float* grad_Y_lm, float* grad_xyz,
                                                      int64_t N, int L_max, int normalize,
                                                      hipStream_t stream) {
    if (N < 0 || L_max < 0 || L_max > 6) return BM_ERR_ARG;
    if (N == 0) return BM_OK;
    if (!edge_vectors || !grad_Y_lm || !grad_xyz) return BM_ERR_ARG;
    return normalize
               ? launch_sh_backward<true>(edge_vectors, grad_Y_lm, grad_xyz, N, L_max, stream)
               : launch_sh_backward<false>(edge_vectors, grad_Y_lm, grad_xyz, N, L_max, stream);
}
