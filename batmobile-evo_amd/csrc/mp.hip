// Fused spherical harmonics + simple tensor product (+ scatter-add into
// destination nodes), COO->CSR conversion, and the dense-weight variant.
//
// Replaces reference src/message_passing/fused_sh_tp.cu:22-249 and
// src/message_passing/fused_message_passing.cu:23-400.
//
// Kernel design (gfx950, wave64, fp32 MFMA):
//   The simple product of one edge is linear in the source row:
//       TP(X[src, c, :], Y) = M(Y) X[src, c, :],  M[o][a] = sum_b CG[a,b,o] Y[b]
//   with M a dense 16x16 operator built once per edge from the 611 CG entries.
//   For a destination d the scatter-summed output is a GEMM over (edge, a):
//       out[d, c, o] = sum_{e in d} sum_a M_e[o][a] X[src_e, c, a]
//   which runs on v_mfma_f32_16x16x4f32 with A = M_e (o x a) from LDS and
//   B = X[src_e] (a x c) streamed from HBM/L2 as float4 per lane.
//   Phase 1 of every 64-edge batch builds the 64 operators M_e into LDS
//   (wave w builds rows 4w..4w+3, lane = edge, Y_lm kept in registers);
//   phase 2 has wave w own channel tile w (16 channels) of the workgroup's
//   64-channel group and walks the batch edge by edge, accumulating in MFMA
//   registers and flushing one float4 per lane when the destination changes.
//   A workgroup owns whole destinations, so outputs are written exactly once,
//   without atomics, in a fixed order: results are deterministic.
#include "common.h"
#include "batmobile_hip.h"

namespace bmhip {

constexpr int kMpBlock = 256;
constexpr int kBatch = 64;        // edges per LDS batch
constexpr int kMStride = 260;     // floats per edge operator in LDS (256 + pad)
constexpr int kChanGroup = 64;    // channels per workgroup (4 waves x 16)

// Phase 1: lane j of wave w builds rows 4w..4w+3 of M for edge j of the batch.
template <int W>
__device__ __forceinline__ void build_rows(const float* Y, float* sMj) {
    static_for<4>([&](auto rr) {
        constexpr int o = 4 * W + decltype(rr)::value;
        float m[16];
        edge_operator_row<o>(Y, m);
        float4* dst = reinterpret_cast<float4*>(sMj + o * 16);
        dst[0] = make_float4(m[0], m[1], m[2], m[3]);
        dst[1] = make_float4(m[4], m[5], m[6], m[7]);
        dst[2] = make_float4(m[8], m[9], m[10], m[11]);
        dst[3] = make_float4(m[12], m[13], m[14], m[15]);
    });
}

template <bool NORM>
__device__ __forceinline__ void phase1_build(const float* __restrict__ vec,
                                             const int64_t* __restrict__ perm,
                                             const int64_t* __restrict__ src_idx, int64_t k0,
                                             int nb, float* sM, int64_t* sSrc) {
    const int lane = threadIdx.x & 63;
    const int w = threadIdx.x >> 6;
    if (lane < nb) {
        const int64_t k = k0 + lane;
        const int64_t e = perm ? perm[k] : k;
        float x = vec[e * 3 + 0], y = vec[e * 3 + 1], z = vec[e * 3 + 2];
        if constexpr (NORM) normalize3(x, y, z);
        float Y[16];
        sh_forward<3>(x, y, z, Y);
        float* sMj = sM + lane * kMStride;
        switch (w) {
            case 0: build_rows<0>(Y, sMj); break;
            case 1: build_rows<1>(Y, sMj); break;
            case 2: build_rows<2>(Y, sMj); break;
            default: build_rows<3>(Y, sMj); break;
        }
        if (w == 0) sSrc[lane] = src_idx[e];
    }
}

__device__ __forceinline__ v4f mfma4(const float4 m, const float4 xv, v4f acc) {
    acc = __builtin_amdgcn_mfma_f32_16x16x4f32(m.x, xv.x, acc, 0, 0, 0);
    acc = __builtin_amdgcn_mfma_f32_16x16x4f32(m.y, xv.y, acc, 0, 0, 0);
    acc = __builtin_amdgcn_mfma_f32_16x16x4f32(m.z, xv.z, acc, 0, 0, 0);
    acc = __builtin_amdgcn_mfma_f32_16x16x4f32(m.w, xv.w, acc, 0, 0, 0);
    return acc;
}

// One lane's slice of source row src: X[src, c, 4g .. 4g+3]; zero when c >= C.
__device__ __forceinline__ float4 load_x(const float* __restrict__ X, int64_t src, int c, int C,
                                         int g) {
    if (c < C) return *reinterpret_cast<const float4*>(X + (src * C + c) * 16 + 4 * g);
    return make_float4(0.f, 0.f, 0.f, 0.f);
}

constexpr int kPrefetch = 4;

// SCATTER: out[d, c, :] = sum over the CSR row of d.  MESSAGES: out[e, c, :] per edge.
template <bool SCATTER, bool NORM>
__global__ __launch_bounds__(kMpBlock, 2) void mp_simple_mfma_kernel(
    const float* __restrict__ vec, const float* __restrict__ X, const int64_t* __restrict__ src_idx,
    const int64_t* __restrict__ perm, const int64_t* __restrict__ row_ptr,
    float* __restrict__ out, int64_t n_items, int64_t n_edges, int C, int items_per_block,
    int n_logical) {
    __shared__ __attribute__((aligned(16))) float sM[kBatch * kMStride];
    __shared__ int64_t sSrc[kBatch];

    // XCD-aware mapping: consecutive logical blocks land on the same XCD.
    const int per_xcd = (n_logical + 7) / 8;
    const int logical = (blockIdx.x & 7) * per_xcd + (blockIdx.x >> 3);
    if (logical >= n_logical) return;

    const int lane = threadIdx.x & 63;
    const int w = threadIdx.x >> 6;
    const int g = lane >> 4;      // k-group: components a = 4g .. 4g+3
    const int i16 = lane & 15;    // channel within the tile / operator row
    const int c = blockIdx.y * kChanGroup + w * 16 + i16;
    const bool tile_live = blockIdx.y * kChanGroup + w * 16 < C;

    int64_t e0, e1, d0 = 0, d1 = 0;
    if constexpr (SCATTER) {
        d0 = (int64_t)logical * items_per_block;
        d1 = min<int64_t>(n_items, d0 + items_per_block);
        e0 = row_ptr[d0];
        e1 = row_ptr[d1];
    } else {
        e0 = (int64_t)logical * kBatch;
        e1 = min<int64_t>(n_edges, e0 + kBatch);
    }

    v4f acc = {0.f, 0.f, 0.f, 0.f};
    int64_t d_cur = d0;
    int64_t rp_next = SCATTER ? row_ptr[d0 + 1] : 0;

    auto flush = [&](int64_t row) {
        if (c < C) {
            float4* o = reinterpret_cast<float4*>(out + (row * C + c) * 16 + 4 * g);
            *o = make_float4(acc[0], acc[1], acc[2], acc[3]);
        }
        acc = v4f{0.f, 0.f, 0.f, 0.f};
    };

    for (int64_t kb = e0; kb < e1; kb += kBatch) {
        const int nb = (int)min<int64_t>(kBatch, e1 - kb);
        __syncthreads();
        phase1_build<NORM>(vec, perm, src_idx, kb, nb, sM, sSrc);
        __syncthreads();
        if (tile_live) {
            float4 xb[kPrefetch];
#pragma unroll
            for (int u = 0; u < kPrefetch; ++u)
                xb[u] = (u < nb) ? load_x(X, sSrc[u], c, C, g) : make_float4(0.f, 0.f, 0.f, 0.f);
            for (int jj = 0; jj < nb; jj += kPrefetch) {
#pragma unroll
                for (int u = 0; u < kPrefetch; ++u) {
                    const int j = jj + u;
                    if (j < nb) {
                        const float4 xv = xb[u];
                        if (j + kPrefetch < nb) xb[u] = load_x(X, sSrc[j + kPrefetch], c, C, g);
                        const float4 m =
                            *reinterpret_cast<const float4*>(sM + j * kMStride + i16 * 16 + 4 * g);
                        if constexpr (SCATTER) {
                            const int64_t k = kb + j;
                            while (k >= rp_next && d_cur + 1 < d1) {
                                flush(d_cur);
                                ++d_cur;
                                rp_next = row_ptr[d_cur + 1];
                            }
                            acc = mfma4(m, xv, acc);
                        } else {
                            acc = mfma4(m, xv, v4f{0.f, 0.f, 0.f, 0.f});
                            flush(kb + j);
                        }
                    }
                }
            }
        }
    }
    if constexpr (SCATTER) {
        if (tile_live) {
            while (d_cur < d1) {
                flush(d_cur);
                ++d_cur;
            }
        }
    }
}

// ---------------------------------------------------------------------------
// dense channel mix: out[t, co, o] = sum_ci W[ci, co] S[t, ci, o]
// (reference fused_message_passing.cu:359, weights[c_in * C_out + c_out])
// ---------------------------------------------------------------------------
__global__ __launch_bounds__(256) void dense_mix_kernel(const float* __restrict__ S,
                                                        const float* __restrict__ W,
                                                        float* __restrict__ out, int64_t n,
                                                        int cin, int cout) {
    const int64_t t = blockIdx.x;
    for (int co = threadIdx.x; co < cout; co += blockDim.x) {
        float acc[16];
#pragma unroll
        for (int k = 0; k < 16; ++k) acc[k] = 0.f;
        const float* s = S + t * cin * 16;
        for (int ci = 0; ci < cin; ++ci) {
            const float wv = W[(int64_t)ci * cout + co];
#pragma unroll
            for (int k = 0; k < 16; ++k) acc[k] = fmaf(wv, s[ci * 16 + k], acc[k]);
        }
        float* o = out + (t * cout + co) * 16;
#pragma unroll
        for (int k = 0; k < 16; ++k) o[k] = acc[k];
    }
}

// ---------------------------------------------------------------------------
// COO -> CSR by target (edge_index[1]), ascending edge id within each row.
// ---------------------------------------------------------------------------
__global__ void zero_i64_kernel(int64_t* __restrict__ p, int64_t n) {
    const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (i < n) p[i] = 0;
}

__global__ void csr_count_kernel(const int64_t* __restrict__ edge_index, int64_t* __restrict__ counts,
                                 int64_t n_atoms, int64_t n_edges) {
    const int64_t e = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (e >= n_edges) return;
    const int64_t t = edge_index[n_edges + e];
    if (t >= 0 && t < n_atoms)
        atomicAdd(reinterpret_cast<unsigned long long*>(counts + t), 1ULL);
}

__global__ void csr_place_kernel(const int64_t* __restrict__ edge_index,
                                 const int64_t* __restrict__ row_ptr, int64_t* __restrict__ cursor,
                                 int64_t* __restrict__ col_idx, int64_t n_atoms, int64_t n_edges) {
    const int64_t e = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (e >= n_edges) return;
    const int64_t t = edge_index[n_edges + e];
    if (t < 0 || t >= n_atoms) return;
    const unsigned long long pos =
        atomicAdd(reinterpret_cast<unsigned long long*>(cursor + t), 1ULL);
    col_idx[row_ptr[t] + (int64_t)pos] = e;
}

// Ascending order inside each row (insertion sort; rows are short in practice).
__global__ void csr_sort_rows_kernel(const int64_t* __restrict__ row_ptr,
                                     int64_t* __restrict__ col_idx, int64_t n_atoms) {
    const int64_t t = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (t >= n_atoms) return;
    const int64_t s = row_ptr[t], e = row_ptr[t + 1];
    for (int64_t i = s + 1; i < e; ++i) {
        const int64_t v = col_idx[i];
        int64_t j = i - 1;
        while (j >= s && col_idx[j] > v) {
            col_idx[j + 1] = col_idx[j];
            --j;
        }
        col_idx[j + 1] = v;
    }
}

__global__ void selftest_mfma_kernel(const float* __restrict__ A, const float* __restrict__ B,
                                     float* __restrict__ D) {
    const int l = threadIdx.x;
    const float a = A[(l & 15) * 4 + (l >> 4)];   // A[i = l%16][k = l/16]
    const float b = B[(l >> 4) * 16 + (l & 15)];  // B[k = l/16][j = l%16]
    v4f acc = {0.f, 0.f, 0.f, 0.f};
    acc = __builtin_amdgcn_mfma_f32_16x16x4f32(a, b, acc, 0, 0, 0);
#pragma unroll
    for (int r = 0; r < 4; ++r) D[(4 * (l >> 4) + r) * 16 + (l & 15)] = acc[r];
}

}  // namespace bmhip

using namespace bmhip;

extern "C" int batteries_selftest_mfma_16x16x4(const float* A, const float* B, float* D,
                                               hipStream_t stream) {
    if (!A || !B || !D) return BM_ERR_ARG;
    selftest_mfma_kernel<<<1, 64, 0, stream>>>(A, B, D);
    return (int)hipGetLastError();
}

static int launch_mp_simple(bool scatter, bool norm, const float* vec, const float* X,
                            const int64_t* src_idx, const int64_t* perm, const int64_t* row_ptr,
                            float* out, int64_t n_items, int64_t n_edges, int C,
                            int items_per_block, hipStream_t s) {
    if (C <= 0) return BM_ERR_ARG;
    if ((reinterpret_cast<uintptr_t>(X) | reinterpret_cast<uintptr_t>(out)) & 15) return BM_ERR_ARG;
    int n_logical;
    if (scatter) {
        if (items_per_block <= 0) items_per_block = 1;
        n_logical = (int)ceil_div(n_items, items_per_block);
    } else {
        n_logical = (int)ceil_div(n_edges, kBatch);
    }
    if (n_logical == 0) return BM_OK;
    const int per_xcd = (n_logical + 7) / 8;
    dim3 grid((unsigned)(per_xcd * 8), (unsigned)ceil_div(C, kChanGroup));
#define BM_LAUNCH(SC, NO)                                                                      \
    mp_simple_mfma_kernel<SC, NO><<<grid, kMpBlock, 0, s>>>(vec, X, src_idx, perm, row_ptr, out, \
                                                            n_items, n_edges, C,               \
                                                            items_per_block, n_logical)
    if (scatter) {
        if (norm) BM_LAUNCH(true, true); else BM_LAUNCH(true, false);
    } else {
        if (norm) BM_LAUNCH(false, true); else BM_LAUNCH(false, false);
    }
#undef BM_LAUNCH
    return (int)hipGetLastError();
}

extern "C" int batteries_fused_sh_tp_simple(const float* edge_vectors, const float* node_features,
                                            const int64_t* source_idx, float* messages,
                                            int64_t N_edges, int C, int normalize,
                                            hipStream_t stream) {
    if (N_edges < 0 || C <= 0) return BM_ERR_ARG;
    if (N_edges == 0) return BM_OK;
    return launch_mp_simple(false, normalize != 0, edge_vectors, node_features, source_idx, nullptr,
                            nullptr, messages, 0, N_edges, C, 0, stream);
}

extern "C" int batteries_sh_tp_scatter_csr(const float* edge_vectors, const float* node_features,
                                           const int64_t* source_idx, const int64_t* perm,
                                           const int64_t* row_ptr, float* node_output,
                                           int64_t N_dst, int64_t N_edges, int C, int normalize,
                                           hipStream_t stream) {
    if (N_dst < 0 || N_edges < 0 || C <= 0) return BM_ERR_ARG;
    if (N_dst == 0) return BM_OK;
    // about one 64-edge batch of whole destinations per workgroup
    const int64_t avg = N_dst > 0 ? ceil_div(N_edges, N_dst) : 1;
    const int per = (int)std::max<int64_t>(1, kBatch / std::max<int64_t>(1, avg));
    return launch_mp_simple(true, normalize != 0, edge_vectors, node_features, source_idx, perm,
                            row_ptr, node_output, N_dst, N_edges, C, per, stream);
}

extern "C" int batteries_fused_message_passing_simple(const float* node_features,
                                                      const float* edge_vectors,
                                                      const int64_t* edge_index,
                                                      const int64_t* row_ptr,
                                                      const int64_t* col_idx, float* node_output,
                                                      int64_t N_atoms, int64_t N_edges, int C,
                                                      hipStream_t stream) {
    // edge data of CSR slot k: e = col_idx[k], src = edge_index[0, e], vector = edge_vectors[e]
    return batteries_sh_tp_scatter_csr(edge_vectors, node_features, edge_index, col_idx, row_ptr,
                                       node_output, N_atoms, N_edges, C, 0, stream);
}

extern "C" size_t batteries_fused_message_passing_workspace_bytes(int64_t N_atoms, int C_in) {
    return (size_t)(N_atoms > 0 ? N_atoms : 0) * (size_t)C_in * 16 * sizeof(float);
}

extern "C" int batteries_fused_message_passing(const float* node_features,
                                               const float* edge_vectors, const float* weights,
                                               const int64_t* row_ptr, const int64_t* col_idx,
                                               float* node_output, int64_t N_atoms,
                                               int64_t N_edges, int C_in, int C_out,
                                               void* workspace, size_t workspace_bytes,
                                               hipStream_t stream) {
    if (N_atoms < 0 || N_edges < 0 || C_in <= 0 || C_out <= 0) return BM_ERR_ARG;
    if (N_atoms == 0) return BM_OK;
    if (!workspace || workspace_bytes < batteries_fused_message_passing_workspace_bytes(N_atoms, C_in))
        return BM_ERR_WORKSPACE;
    // reference semantics (fused_message_passing.cu:332-337): source atom = col_idx[k],
    // edge vector = edge_vectors[k] for CSR slot k.
    float* S = static_cast<float*>(workspace);
    int rc = batteries_sh_tp_scatter_csr(edge_vectors, node_features, col_idx, nullptr, row_ptr, S,
                                         N_atoms, N_edges, C_in, 0, stream);
    if (rc != BM_OK) return rc;
    dense_mix_kernel<<<(unsigned)N_atoms, 256, 0, stream>>>(S, weights, node_output, N_atoms, C_in,
                                                            C_out);
    return (int)hipGetLastError();
}

extern "C" int batteries_exclusive_scan_i64(const int64_t* in, int64_t* out, int64_t n,
                                            hipStream_t stream);

extern "C" size_t batteries_edge_index_to_csr_workspace_bytes(int64_t N_atoms) {
    return (size_t)(N_atoms > 0 ? N_atoms : 0) * sizeof(int64_t);
}

extern "C" int batteries_edge_index_to_csr(const int64_t* edge_index, int64_t* row_ptr,
                                           int64_t* col_idx, int64_t N_atoms, int64_t N_edges,
                                           void* workspace, size_t workspace_bytes,
                                           hipStream_t stream) {
    if (N_atoms < 0 || N_edges < 0) return BM_ERR_ARG;
    if (workspace_bytes < batteries_edge_index_to_csr_workspace_bytes(N_atoms) ||
        (N_atoms > 0 && !workspace))
        return BM_ERR_WORKSPACE;
    int64_t* counts = static_cast<int64_t*>(workspace);
    const int B = 256;
    if (N_atoms > 0)
        zero_i64_kernel<<<(unsigned)ceil_div(N_atoms, B), B, 0, stream>>>(counts, N_atoms);
    if (N_edges > 0 && N_atoms > 0)
        csr_count_kernel<<<(unsigned)ceil_div(N_edges, B), B, 0, stream>>>(edge_index, counts,
                                                                           N_atoms, N_edges);
    int rc = batteries_exclusive_scan_i64(counts, row_ptr, N_atoms, stream);
    if (rc != BM_OK) return rc;
    if (N_edges > 0 && N_atoms > 0) {
        zero_i64_kernel<<<(unsigned)ceil_div(N_atoms, B), B, 0, stream>>>(counts, N_atoms);
        csr_place_kernel<<<(unsigned)ceil_div(N_edges, B), B, 0, stream>>>(
            edge_index, row_ptr, counts, col_idx, N_atoms, N_edges);
        csr_sort_rows_kernel<<<(unsigned)ceil_div(N_atoms, B), B, 0, stream>>>(row_ptr, col_idx,
                                                                               N_atoms);
    }
    return (int)hipGetLastError();
}
