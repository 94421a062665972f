// 34-path L<=3 Clebsch-Gordan tensor products: simple and channel-weighted,
// forward and backward.
//
// Replaces reference src/tensor_product/tensor_product.cu:29-214 and
// src/tensor_product/tensor_product_backward.cu:32-1026.  The weight gradient
// is the exact adjoint of the forward (tensor_product_backward.cu:7-16), not
// the hand-written CG lines of :159-872.
#include "common.h"
#include "batmobile_hip.h"

namespace bmhip {

constexpr int kTpBlock = 256;
constexpr int kRowStride = 17;  // odd LDS stride for 16-float rows

// ---------------------------------------------------------------------------
// simple product: one thread per row, rows staged through LDS
// ---------------------------------------------------------------------------
__device__ __forceinline__ void stage_rows16(float* s, const float* __restrict__ g, int64_t base,
                                             int rows) {
    const float* src = g + base * 16;
    for (int i = threadIdx.x; i < rows * 16; i += kTpBlock) s[(i >> 4) * kRowStride + (i & 15)] = src[i];
}
__device__ __forceinline__ void unstage_rows16(const float* s, float* __restrict__ g, int64_t base,
                                               int rows) {
    float* dst = g + base * 16;
    for (int i = threadIdx.x; i < rows * 16; i += kTpBlock) dst[i] = s[(i >> 4) * kRowStride + (i & 15)];
}

__global__ __launch_bounds__(kTpBlock) void tp_simple_kernel(const float* __restrict__ x,
                                                             const float* __restrict__ y,
                                                             float* __restrict__ out, int64_t n) {
    __shared__ float sx[kTpBlock * kRowStride];
    __shared__ float sy[kTpBlock * kRowStride];
    const int64_t base = (int64_t)blockIdx.x * kTpBlock;
    const int rows = (int)min<int64_t>(kTpBlock, n - base);
    stage_rows16(sx, x, base, rows);
    stage_rows16(sy, y, base, rows);
    __syncthreads();
    const int t = threadIdx.x;
    if (t < rows) {
        float a[16], b[16], o[16];
#pragma unroll
        for (int k = 0; k < 16; ++k) {
            a[k] = sx[t * kRowStride + k];
            b[k] = sy[t * kRowStride + k];
        }
        tp_simple(a, b, o);
#pragma unroll
        for (int k = 0; k < 16; ++k) sx[t * kRowStride + k] = o[k];
    }
    __syncthreads();
    unstage_rows16(sx, out, base, rows);
}

__global__ __launch_bounds__(kTpBlock) void tp_simple_backward_kernel(
    const float* __restrict__ x, const float* __restrict__ y, const float* __restrict__ g,
    float* __restrict__ gx, float* __restrict__ gy, int64_t n) {
    __shared__ float sx[kTpBlock * kRowStride];
    __shared__ float sy[kTpBlock * kRowStride];
    __shared__ float sg[kTpBlock * kRowStride];
    const int64_t base = (int64_t)blockIdx.x * kTpBlock;
    const int rows = (int)min<int64_t>(kTpBlock, n - base);
    stage_rows16(sx, x, base, rows);
    stage_rows16(sy, y, base, rows);
    stage_rows16(sg, g, base, rows);
    __syncthreads();
    const int t = threadIdx.x;
    if (t < rows) {
        float a[16], b[16], c[16], ga[16], gb[16];
#pragma unroll
        for (int k = 0; k < 16; ++k) {
            a[k] = sx[t * kRowStride + k];
            b[k] = sy[t * kRowStride + k];
            c[k] = sg[t * kRowStride + k];
        }
        tp_simple_backward(a, b, c, ga, gb);
#pragma unroll
        for (int k = 0; k < 16; ++k) {
            sx[t * kRowStride + k] = ga[k];
            sy[t * kRowStride + k] = gb[k];
        }
    }
    __syncthreads();
    unstage_rows16(sx, gx, base, rows);
    unstage_rows16(sy, gy, base, rows);
}

// ---------------------------------------------------------------------------
// weighted product
//   out[n,co,o] = sum_q W[path(q), ci, co] * T[n,ci,q] * [out(q) == o]
//   T[n,ci,q]   = sum_{(a,b) in q} c * x[n,ci,a] * y[n,b]     (156 slots)
// ---------------------------------------------------------------------------
constexpr int kWRows = 4;     // rows per workgroup
constexpr int kWChunk = 16;   // input channels per LDS chunk

__global__ __launch_bounds__(kTpBlock) void tp_weighted_forward_kernel(
    const float* __restrict__ x, const float* __restrict__ y, const float* __restrict__ w,
    float* __restrict__ out, int64_t n, int cin, int cout) {
    __shared__ float sT[kWRows * kWChunk * kNumSlots];
    __shared__ float sy[kWRows * 16];
    const int64_t row0 = (int64_t)blockIdx.x * kWRows;
    const int rows = (int)min<int64_t>(kWRows, n - row0);
    const int tid = threadIdx.x;
    for (int i = tid; i < rows * 16; i += kTpBlock) sy[i] = y[row0 * 16 + i];
    // each thread owns (r, co) pairs r = pair / cout, co = pair % cout
    const int npairs = rows * cout;
    const int my_pairs = (npairs + kTpBlock - 1) / kTpBlock;  // usually 1
    for (int pp = 0; pp < my_pairs; ++pp) {
        const int pair = tid + pp * kTpBlock;
        const bool active = pair < npairs;
        const int r = active ? pair / cout : 0;
        const int co = active ? pair - r * cout : 0;
        float acc[16];
#pragma unroll
        for (int k = 0; k < 16; ++k) acc[k] = 0.0f;
        for (int c0 = 0; c0 < cin; c0 += kWChunk) {
            const int cw = min(kWChunk, cin - c0);
            __syncthreads();
            // phase 1: per-path products for (r, ci) of this chunk
            for (int it = tid; it < rows * cw; it += kTpBlock) {
                const int rr = it / cw, ci = it - rr * cw;
                const float* xr = x + ((row0 + rr) * cin + c0 + ci) * 16;
                float a[16], b[16], t[kNumSlots];
#pragma unroll
                for (int k = 0; k < 16; ++k) {
                    a[k] = xr[k];
                    b[k] = sy[rr * 16 + k];
                }
                tp_per_path(a, b, t);
                float* dstT = sT + (rr * kWChunk + ci) * kNumSlots;
#pragma unroll
                for (int q = 0; q < kNumSlots; ++q) dstT[q] = t[q];
            }
            __syncthreads();
            if (active) {
                for (int ci = 0; ci < cw; ++ci) {
                    const float* Tq = sT + (r * kWChunk + ci) * kNumSlots;
                    const float* wc = w + (int64_t)(c0 + ci) * cout + co;
                    static_for<kNumPaths>([&](auto pp2) {
                        constexpr int p = decltype(pp2)::value;
                        const float wp = wc[(int64_t)p * cin * cout];
                        constexpr int s0 = kPathSlot[p];
                        constexpr int lo = kPathL[p][2];
                        static_for<2 * lo + 1>([&](auto mm) {
                            constexpr int m = decltype(mm)::value;
                            acc[lo * lo + m] = fmaf(wp, Tq[s0 + m], acc[lo * lo + m]);
                        });
                    });
                }
            }
        }
        if (active) {
            float* o = out + ((row0 + r) * cout + co) * 16;
#pragma unroll
            for (int k = 0; k < 16; ++k) o[k] = acc[k];
        }
    }
}

// grad_x and grad_y.  h[n,ci,q] = sum_co W[path(q),ci,co] g[n,co,out(q)],
// gx = CG^T(h, y), gy = sum_ci CG^T(h, x).  One thread per (row, ci); the
// per-ci gy partials are reduced in a fixed order.
constexpr int kBRows = 2;
__global__ __launch_bounds__(kTpBlock) void tp_weighted_backward_xy_kernel(
    const float* __restrict__ x, const float* __restrict__ y, const float* __restrict__ w,
    const float* __restrict__ g, float* __restrict__ gx, float* __restrict__ gy, int64_t n, int cin,
    int cout) {
    extern __shared__ float smem[];
    float* sg = smem;                          // [kBRows][cout][16]
    float* sgy = sg + kBRows * cout * 16;      // [kBRows][cin][16]
    float* sy = sgy + kBRows * cin * 16;       // [kBRows][16]
    const int64_t row0 = (int64_t)blockIdx.x * kBRows;
    const int rows = (int)min<int64_t>(kBRows, n - row0);
    const int tid = threadIdx.x;
    for (int i = tid; i < rows * cout * 16; i += kTpBlock) sg[i] = g[row0 * cout * 16 + i];
    for (int i = tid; i < rows * 16; i += kTpBlock) sy[i] = y[row0 * 16 + i];
    __syncthreads();
    for (int it = tid; it < rows * cin; it += kTpBlock) {
        const int r = it / cin, ci = it - r * cin;
        float h[kNumSlots];
#pragma unroll
        for (int q = 0; q < kNumSlots; ++q) h[q] = 0.0f;
        const float* wci = w + (int64_t)ci * cout;
        const float* gr = sg + r * cout * 16;
        for (int co = 0; co < cout; ++co) {
            float gv[16];
#pragma unroll
            for (int k = 0; k < 16; ++k) gv[k] = gr[co * 16 + k];
            static_for<kNumPaths>([&](auto pp) {
                constexpr int p = decltype(pp)::value;
                const float wp = wci[(int64_t)p * cin * cout + co];
                constexpr int s0 = kPathSlot[p];
                constexpr int lo = kPathL[p][2];
                static_for<2 * lo + 1>([&](auto mm) {
                    constexpr int m = decltype(mm)::value;
                    h[s0 + m] = fmaf(wp, gv[lo * lo + m], h[s0 + m]);
                });
            });
        }
        float a[16], b[16], ga[16], gb[16];
        const float* xr = x + ((row0 + r) * cin + ci) * 16;
#pragma unroll
        for (int k = 0; k < 16; ++k) {
            a[k] = xr[k];
            b[k] = sy[r * 16 + k];
            ga[k] = 0.0f;
            gb[k] = 0.0f;
        }
        tp_per_path_backward(a, b, h, ga, gb);
        if (gx) {
            float* o = gx + ((row0 + r) * cin + ci) * 16;
#pragma unroll
            for (int k = 0; k < 16; ++k) o[k] = ga[k];
        }
#pragma unroll
        for (int k = 0; k < 16; ++k) sgy[(r * cin + ci) * 16 + k] = gb[k];
    }
    __syncthreads();
    if (gy) {
        for (int i = tid; i < rows * 16; i += kTpBlock) {
            const int r = i >> 4, k = i & 15;
            float s = 0.0f;
            for (int ci = 0; ci < cin; ++ci) s += sgy[(r * cin + ci) * 16 + k];
            gy[(row0 + r) * 16 + k] = s;
        }
    }
}

// grad_W partials over a segment of rows:
//   part[seg, p, ci, co] = sum_{n in seg} sum_{q in p} T[n,ci,q] * g[n,co,out(q)]
// Block = (ci chunk of 4, segment); thread = (ci_local, co).
constexpr int kGwCi = 4;
__global__ __launch_bounds__(kTpBlock) void tp_weighted_backward_w_partial_kernel(
    const float* __restrict__ x, const float* __restrict__ y, const float* __restrict__ g,
    float* __restrict__ part, int64_t n, int cin, int cout, int64_t rows_per_seg) {
    __shared__ float sT[kGwCi * kNumSlots];
    __shared__ float sx[kGwCi * 16];
    __shared__ float sy[16];
    const int ci0 = blockIdx.x * kGwCi;
    const int seg = blockIdx.y;
    const int64_t r0 = (int64_t)seg * rows_per_seg;
    const int64_t r1 = min<int64_t>(n, r0 + rows_per_seg);
    const int tid = threadIdx.x;
    const int cw = min(kGwCi, cin - ci0);
    // thread -> (ci_local, co) pairs, looping when 4*cout > 256
    const int npairs = cw * cout;
    constexpr int kMaxPairs = 4;  // supports cout <= 256
    float acc[kMaxPairs][kNumPaths];
#pragma unroll
    for (int j = 0; j < kMaxPairs; ++j)
#pragma unroll
        for (int p = 0; p < kNumPaths; ++p) acc[j][p] = 0.0f;
    for (int64_t row = r0; row < r1; ++row) {
        __syncthreads();
        for (int i = tid; i < cw * 16; i += kTpBlock) sx[i] = x[(row * cin + ci0) * 16 + i];
        if (tid < 16) sy[tid] = y[row * 16 + tid];
        __syncthreads();
        if (tid < cw) {
            float a[16], b[16], t[kNumSlots];
#pragma unroll
            for (int k = 0; k < 16; ++k) {
                a[k] = sx[tid * 16 + k];
                b[k] = sy[k];
            }
            tp_per_path(a, b, t);
#pragma unroll
            for (int q = 0; q < kNumSlots; ++q) sT[tid * kNumSlots + q] = t[q];
        }
        __syncthreads();
#pragma unroll
        for (int j = 0; j < kMaxPairs; ++j) {
            const int pair = tid + j * kTpBlock;
            if (pair < npairs) {
                const int cl = pair / cout, co = pair - cl * cout;
                const float* gr = g + (row * cout + co) * 16;
                float gv[16];
#pragma unroll
                for (int k = 0; k < 16; ++k) gv[k] = gr[k];
                const float* Tq = sT + cl * kNumSlots;
                static_for<kNumSlots>([&](auto qq) {
                    constexpr int q = decltype(qq)::value;
                    acc[j][kSlotPath[q]] = fmaf(Tq[q], gv[kSlotOut[q]], acc[j][kSlotPath[q]]);
                });
            }
        }
    }
#pragma unroll
    for (int j = 0; j < kMaxPairs; ++j) {
        const int pair = tid + j * kTpBlock;
        if (pair < npairs) {
            const int cl = pair / cout, co = pair - cl * cout;
            float* dst = part + (int64_t)seg * kNumPaths * cin * cout;
#pragma unroll
            for (int p = 0; p < kNumPaths; ++p)
                dst[((int64_t)p * cin + ci0 + cl) * cout + co] = acc[j][p];
        }
    }
}

// gW[i] = sum_s part[s, i] in ascending s (deterministic).
__global__ __launch_bounds__(kTpBlock) void reduce_segments_kernel(const float* __restrict__ part,
                                                                   float* __restrict__ out,
                                                                   int64_t count, int nseg) {
    const int64_t i = (int64_t)blockIdx.x * kTpBlock + threadIdx.x;
    if (i >= count) return;
    float s = 0.0f;
    for (int k = 0; k < nseg; ++k) s += part[(int64_t)k * count + i];
    out[i] = s;
}

__global__ void fill_zero_kernel(float* __restrict__ p, int64_t count) {
    const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (i < count) p[i] = 0.0f;
}

static int64_t gw_rows_per_seg(int64_t n, int cin) {
    const int64_t cchunks = ceil_div(cin, kGwCi);
    const int64_t segs = std::max<int64_t>(1, 1024 / cchunks);
    const int64_t rps = ceil_div(n, segs);
    return std::max<int64_t>(rps, 32);
}

}  // namespace bmhip

using namespace bmhip;

extern "C" int batteries_get_num_paths_l3(void) { return kNumPaths; }

extern "C" void batteries_get_path_info_l3(int* path_info) {
    for (int p = 0; p < kNumPaths; ++p)
        for (int k = 0; k < 3; ++k) path_info[p * 3 + k] = kPathL[p][k];
}

extern "C" int batteries_tensor_product_simple_l3(const float* input1, const float* input2,
                                                  float* output, int64_t N, hipStream_t stream) {
    if (N < 0) return BM_ERR_ARG;
    if (N == 0) return BM_OK;
    tp_simple_kernel<<<(unsigned)ceil_div(N, kTpBlock), kTpBlock, 0, stream>>>(input1, input2,
                                                                              output, N);
    return (int)hipGetLastError();
}

extern "C" int batteries_tensor_product_simple_backward_l3(const float* input1,
                                                           const float* input2,
                                                           const float* grad_output,
                                                           float* grad_input1, float* grad_input2,
                                                           int64_t N, hipStream_t stream) {
    if (N < 0) return BM_ERR_ARG;
    if (N == 0) return BM_OK;
    tp_simple_backward_kernel<<<(unsigned)ceil_div(N, kTpBlock), kTpBlock, 0, stream>>>(
        input1, input2, grad_output, grad_input1, grad_input2, N);
    return (int)hipGetLastError();
}

extern "C" int batteries_tensor_product_l3(const float* input1, const float* input2,
                                           const float* weights, float* output, int64_t N,
                                           int C_in, int C_out, hipStream_t stream) {
    if (N < 0 || C_in <= 0 || C_out <= 0) return BM_ERR_ARG;
    if (N == 0) return BM_OK;
    tp_weighted_forward_kernel<<<(unsigned)ceil_div(N, kWRows), kTpBlock, 0, stream>>>(
        input1, input2, weights, output, N, C_in, C_out);
    return (int)hipGetLastError();
}

extern "C" size_t batteries_tensor_product_backward_workspace_bytes(int64_t N, int C_in,
                                                                    int C_out) {
    if (N <= 0 || C_in <= 0 || C_out <= 0) return 0;
    const int64_t rps = gw_rows_per_seg(N, C_in);
    const int64_t segs = ceil_div(N, rps);
    return (size_t)(segs * kNumPaths * (int64_t)C_in * C_out) * sizeof(float);
}

extern "C" int batteries_tensor_product_backward_l3(
    const float* input1, const float* input2, const float* weights, const float* grad_output,
    float* grad_input1, float* grad_input2, float* grad_weights, int64_t N, int C_in, int C_out,
    void* workspace, size_t workspace_bytes, hipStream_t stream) {
    if (N < 0 || C_in <= 0 || C_out <= 0 || C_out > 256) return BM_ERR_ARG;
    if (N == 0) {
        if (grad_weights) {
            const int64_t count = (int64_t)kNumPaths * C_in * C_out;
            fill_zero_kernel<<<(unsigned)ceil_div(count, kTpBlock), kTpBlock, 0, stream>>>(
                grad_weights, count);
            return (int)hipGetLastError();
        }
        return BM_OK;
    }
    if (grad_input1 || grad_input2) {
        const size_t smem =
            sizeof(float) * ((size_t)kBRows * C_out * 16 + (size_t)kBRows * C_in * 16 + kBRows * 16);
        if (smem > 64 * 1024) return BM_ERR_ARG;
        tp_weighted_backward_xy_kernel<<<(unsigned)ceil_div(N, kBRows), kTpBlock, smem, stream>>>(
            input1, input2, weights, grad_output, grad_input1, grad_input2, N, C_in, C_out);
        hipError_t e = hipGetLastError();
        if (e != hipSuccess) return (int)e;
    }
    if (grad_weights) {
        const size_t need = batteries_tensor_product_backward_workspace_bytes(N, C_in, C_out);
        if (!workspace || workspace_bytes < need) return BM_ERR_WORKSPACE;
        const int64_t rps = gw_rows_per_seg(N, C_in);
        const int64_t segs = ceil_div(N, rps);
        float* part = static_cast<float*>(workspace);
        dim3 grid((unsigned)ceil_div(C_in, kGwCi), (unsigned)segs);
        tp_weighted_backward_w_partial_kernel<<<grid, kTpBlock, 0, stream>>>(
            input1, input2, grad_output, part, N, C_in, C_out, rps);
        hipError_t e = hipGetLastError();
        if (e != hipSuccess) return (int)e;
        const int64_t count = (int64_t)kNumPaths * C_in * C_out;
        reduce_segments_kernel<<<(unsigned)ceil_div(count, kTpBlock), kTpBlock, 0, stream>>>(
            part, grad_weights, count, (int)segs);
        e = hipGetLastError();
        if (e != hipSuccess) return (int)e;
    }
    return BM_OK;
}
