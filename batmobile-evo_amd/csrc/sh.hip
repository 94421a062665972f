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

// A block of `rows` consecutive rows of a row-major [n, K] array (rows * K
// contiguous floats from g) to LDS rows of stride KS, and back.  A full block
// (256 rows: 64 K floats) of 16-byte aligned arrays (vec4) moves as float4s,
// every thread issuing all of its loads before its LDS writes; otherwise (the
// grid's last block, or unaligned arrays) float by float.
template <int K, int KS>
__device__ __forceinline__ void block_to_lds(const float* __restrict__ g, float* s, int rows,
                                             bool vec4) {
    const int tid = threadIdx.x;
    if (vec4 && rows == kShBlock) {
        constexpr int NQ = kShBlock * K / 4;  // float4s in the block
        constexpr int PER = (NQ + kShBlock - 1) / kShBlock;
        const float4* g4 = reinterpret_cast<const float4*>(g);
        float4 v[PER];
#pragma unroll
        for (int it = 0; it < PER; ++it) v[it] = g4[min(tid + kShBlock * it, NQ - 1)];
#pragma unroll
        for (int it = 0; it < PER; ++it) {
            const int i = tid + kShBlock * it;
            if (i < NQ) {
                const float vv[4] = {v[it].x, v[it].y, v[it].z, v[it].w};
#pragma unroll
                for (int j = 0; j < 4; ++j) {
                    const int e = 4 * i + j, r = e / K;
                    s[r * KS + (e - r * K)] = vv[j];
                }
            }
        }
    } else {
        for (int i = tid; i < rows * K; i += kShBlock) {
            const int r = i / K;
            s[r * KS + (i - r * K)] = g[i];
        }
    }
}
template <int K, int KS>
__device__ __forceinline__ void lds_to_block(const float* s, float* __restrict__ g, int rows,
                                             bool vec4) {
    const int tid = threadIdx.x;
    if (vec4 && rows == kShBlock) {
        constexpr int NQ = kShBlock * K / 4;
        constexpr int PER = (NQ + kShBlock - 1) / kShBlock;
        float4* g4 = reinterpret_cast<float4*>(g);
#pragma unroll
        for (int it = 0; it < PER; ++it) {
            const int i = tid + kShBlock * it;
            if (i < NQ) {
                float vv[4];
#pragma unroll
                for (int j = 0; j < 4; ++j) {
                    const int e = 4 * i + j, r = e / K;
                    vv[j] = s[r * KS + (e - r * K)];
                }
                g4[i] = make_float4(vv[0], vv[1], vv[2], vv[3]);
            }
        }
    } else {
        for (int i = tid; i < rows * K; i += kShBlock) {
            const int r = i / K;
            g[i] = s[r * KS + (i - r * K)];
        }
    }
}

template <int L, bool NORM>
__global__ __launch_bounds__(kShBlock) void sh_forward_kernel(const float* __restrict__ v,
                                                                float* __restrict__ Y, int64_t n,
                                                                bool vec4) {
    constexpr int K = sh_dim(L);
    constexpr int KS = odd_stride(K);
    __shared__ float sv[kShBlock * 3];
    __shared__ float sy[kShBlock * KS];
    const int64_t base = (int64_t)blockIdx.x * kShBlock;
    const int rows = (int)min<int64_t>(kShBlock, n - base);
    const int tid = threadIdx.x;
    block_to_lds<3, 3>(v + base * 3, sv, rows, vec4);
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
    lds_to_block<K, KS>(sy, Y + base * K, rows, vec4);
}

// Small inputs (at most kShDirectRows rows, one round of workgroups): each lane its own
// vector and row straight from global memory, no LDS and no barriers (with a single
// round there is no other workgroup to cover the staged kernel's barriers).
constexpr int64_t kShDirectRows = 65536;
template <int L, bool NORM>
__global__ __launch_bounds__(kShBlock) void sh_forward_direct_kernel(const float* __restrict__ v,
                                                                       float* __restrict__ Y,
                                                                       int64_t n, bool vec4) {
    constexpr int K = sh_dim(L);
    const int64_t r = (int64_t)blockIdx.x * kShBlock + threadIdx.x;
    if (r >= n) return;
    float x = v[r * 3 + 0], y = v[r * 3 + 1], z = v[r * 3 + 2];
    if constexpr (NORM) normalize3(x, y, z);
    float out[K];
    sh_forward<L>(x, y, z, out);
    if constexpr (K % 4 == 0) {
        if (vec4) {
            float4* y4 = reinterpret_cast<float4*>(Y + r * K);
#pragma unroll
            for (int q = 0; q < K / 4; ++q)
                y4[q] = make_float4(out[4 * q], out[4 * q + 1], out[4 * q + 2], out[4 * q + 3]);
            return;
        }
    }
#pragma unroll
    for (int k = 0; k < K; ++k) Y[r * K + k] = out[k];
}

// grad_xyz = sum_k g_k dY_k/d(x,y,z).  With NORM the input is the raw vector v,
// Y is taken at u = v/|v| and the result is chained through the normalisation:
// (g_u - u (u . g_u)) / |v|   (reference python/batmobile/autograd.py:62-92).
template <int L, bool NORM>
__global__ __launch_bounds__(kShBlock) void sh_backward_kernel(const float* __restrict__ v,
                                                                 const float* __restrict__ gY,
                                                                 float* __restrict__ gv, int64_t n,
                                                                 bool vec4) {
    constexpr int K = sh_dim(L);
    constexpr int KS = odd_stride(K);
    __shared__ float sv[kShBlock * 3];
    __shared__ float sg[kShBlock * KS];
    const int64_t base = (int64_t)blockIdx.x * kShBlock;
    const int rows = (int)min<int64_t>(kShBlock, n - base);
    const int tid = threadIdx.x;
    block_to_lds<3, 3>(v + base * 3, sv, rows, vec4);
    block_to_lds<K, KS>(gY + base * K, sg, rows, vec4);
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
    lds_to_block<3, 3>(sv, gv + base * 3, rows, vec4);
}

static bool al16(const void* p) { return (reinterpret_cast<uintptr_t>(p) & 15) == 0; }

template <bool NORM>
static int launch_sh_forward(const float* v, float* Y, int64_t n, int L, hipStream_t s) {
    const dim3 grid((unsigned)ceil_div(n, kShBlock));
    const bool vec4 = al16(v) && al16(Y);
    if (n <= kShDirectRows) {
        switch (L) {
            case 0: sh_forward_direct_kernel<0, NORM><<<grid, kShBlock, 0, s>>>(v, Y, n, vec4); break;
            case 1: sh_forward_direct_kernel<1, NORM><<<grid, kShBlock, 0, s>>>(v, Y, n, vec4); break;
            case 2: sh_forward_direct_kernel<2, NORM><<<grid, kShBlock, 0, s>>>(v, Y, n, vec4); break;
            case 3: sh_forward_direct_kernel<3, NORM><<<grid, kShBlock, 0, s>>>(v, Y, n, vec4); break;
            case 4: sh_forward_direct_kernel<4, NORM><<<grid, kShBlock, 0, s>>>(v, Y, n, vec4); break;
            case 5: sh_forward_direct_kernel<5, NORM><<<grid, kShBlock, 0, s>>>(v, Y, n, vec4); break;
            case 6: sh_forward_direct_kernel<6, NORM><<<grid, kShBlock, 0, s>>>(v, Y, n, vec4); break;
            default: return BM_ERR_ARG;
        }
        return (int)hipGetLastError();
    }
    switch (L) {
        case 0: sh_forward_kernel<0, NORM><<<grid, kShBlock, 0, s>>>(v, Y, n, vec4); break;
        case 1: sh_forward_kernel<1, NORM><<<grid, kShBlock, 0, s>>>(v, Y, n, vec4); break;
        case 2: sh_forward_kernel<2, NORM><<<grid, kShBlock, 0, s>>>(v, Y, n, vec4); break;
        case 3: sh_forward_kernel<3, NORM><<<grid, kShBlock, 0, s>>>(v, Y, n, vec4); break;
        case 4: sh_forward_kernel<4, NORM><<<grid, kShBlock, 0, s>>>(v, Y, n, vec4); break;
        case 5: sh_forward_kernel<5, NORM><<<grid, kShBlock, 0, s>>>(v, Y, n, vec4); break;
        case 6: sh_forward_kernel<6, NORM><<<grid, kShBlock, 0, s>>>(v, Y, n, vec4); break;
        default: return BM_ERR_ARG;
    }
    return (int)hipGetLastError();
}

template <bool NORM>
static int launch_sh_backward(const float* v, const float* g, float* gv, int64_t n, int L,
                              hipStream_t s) {
    const dim3 grid((unsigned)ceil_div(n, kShBlock));
    const bool vec4 = al16(v) && al16(g) && al16(gv);
    switch (L) {
        case 0: sh_backward_kernel<0, NORM><<<grid, kShBlock, 0, s>>>(v, g, gv, n, vec4); break;
        case 1: sh_backward_kernel<1, NORM><<<grid, kShBlock, 0, s>>>(v, g, gv, n, vec4); break;
        case 2: sh_backward_kernel<2, NORM><<<grid, kShBlock, 0, s>>>(v, g, gv, n, vec4); break;
        case 3: sh_backward_kernel<3, NORM><<<grid, kShBlock, 0, s>>>(v, g, gv, n, vec4); break;
        case 4: sh_backward_kernel<4, NORM><<<grid, kShBlock, 0, s>>>(v, g, gv, n, vec4); break;
        case 5: sh_backward_kernel<5, NORM><<<grid, kShBlock, 0, s>>>(v, g, gv, n, vec4); break;
        case 6: sh_backward_kernel<6, NORM><<<grid, kShBlock, 0, s>>>(v, g, gv, n, vec4); break;
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
