// MACE-style interaction layer with per-edge radial weights (the baseline's
// configs[4]): Bessel radial basis -> MLP [8 -> 64 -> 34 C] -> channel-wise
// weighted CG product of X[src] with Y(v) -> scatter-add into destinations,
// and its gradient with respect to the positions.
//
// Pattern of reference benchmarks/benchmark_e2e_mace.py:281-434 (SH -> TP ->
// scatter, forces by backward through the edge vectors :412-420); the
// reference's own block shares one W[34, C, C] over edges, the per-edge radial
// weights are this configuration's.  Layer definition (fp32 here):
//   v_e = min_image(pos[dst_e] - pos[src_e]), r = |v|, u = v / r
//   B_k = sqrt(2/rc) sin(k pi r/rc) / r * f(r/rc),  f(d) = 1 - 28 d^6 + 48 d^7 - 21 d^8
//   h = silu(B W1 + b1), R[e, c, p] = (h W2)[p * C + c]
//   out[d, c, o] = sum_{e -> d} sum_p R[e,c,p] sum_{(a,b) in p -> o} CG x[src_e,c,a] Y_e[b]
//
// Work per edge: the MLP's second layer is a GEMM [edges x 64] x [64 x 34C]
// (557 kflop per edge at C = 128) and runs on MFMA over edge chunks; the CG
// work (611 products with a coefficient, 256 bilinear products and 156 path
// weightings per edge and channel) runs on the VALU, thread per
// (destination row, channel), so every output row is written by one thread in
// a fixed edge order (deterministic, no atomics).  Forces are gathered per
// atom from per-edge gradients through the reverse-edge map of the symmetric
// edge list.
#include <mutex>

#include <rocblas/rocblas.h>

#include "common.h"
#include "batmobile_hip.h"

namespace bmhip {

constexpr int kNBasis = 8;
constexpr int kHidden = 64;
// Edges per chunk (R and its gradient live per chunk): up to kMaceChunkMax, and
// all chunks of a graph equally long (multiples of 256, the last one shorter by
// less than 256 per chunk), so the GEMMs run every chunk at one height.  Larger
// chunks run faster on MI355X (configs[4], forward / backward: 8192 edges
// 36.3 / 88.7 ms, 65536 19.3 / 34.5 ms, 131072 16.6 / 32.0 ms, 262144 16.2 /
// 31.3 ms); R is 17 KB per edge at C = 128, 4.6 GB for a chunk of 262144.
constexpr int64_t kMaceChunkMax = 262144;
static int64_t mace_chunk(int64_t E, int C) {
    // R offsets within a chunk stay below 2^31 (32-bit GEMM and kernel offsets)
    const int64_t cap = std::min<int64_t>(kMaceChunkMax, INT32_MAX / ((int64_t)C * 34) / 256 * 256);
    const int64_t e = std::max<int64_t>(E, 1);
    const int64_t n = (e + cap - 1) / cap;
    return ((e + n - 1) / n + 255) / 256 * 256;
}

#pragma clang fp contract(off)
// v = pos[dst] - pos[src] with the minimum image of an orthorhombic box, in the
// neighbor list's operation order (so v equals its vectors negated, exactly)
__device__ __forceinline__ void edge_vector(const float* __restrict__ pos, int64_t s, int64_t d,
                                            const float* box, const float* inv, float* v) {
#pragma unroll
    for (int k = 0; k < 3; ++k) {
        const float t = pos[d * 3 + k] - pos[s * 3 + k];
        const float q = t * inv[k];
        const float rr = rintf(q);
        const float m = rr * box[k];
        v[k] = t - m;
    }
}
#pragma clang fp contract(on)

struct MaceBox {
    float box[3];
    float inv[3];
};

// Bessel basis with envelope, and its derivative with respect to r.
__device__ __forceinline__ void radial_basis(float r, float rc, float* B, float* dB) {
    const float d = r / rc;
    float f = 0.f, df = 0.f;
    if (d < 1.0f) {
        const float d5 = d * d * d * d * d, d6 = d5 * d;
        f = 1.0f - 28.0f * d6 + 48.0f * d6 * d - 21.0f * d6 * d * d;
        const float om = 1.0f - d;
        df = -168.0f * d5 * om * om / rc;  // f'(d) / rc
    }
    const float norm = sqrtf(2.0f / rc);
    const float ir = 1.0f / r;
#pragma unroll
    for (int k = 0; k < kNBasis; ++k) {
        const float w = (float)(k + 1) * 3.14159265358979323846f / rc;
        float sn, cs;
        sincosf(w * r, &sn, &cs);
        const float g = norm * sn * ir;                       // bare Bessel
        const float dg = norm * (w * cs * ir - sn * ir * ir);  // its derivative
        B[k] = g * f;
        if (dB) dB[k] = dg * f + g * df;
    }
}

__device__ __forceinline__ float sigmoidf(float z) { return 1.0f / (1.0f + expf(-z)); }


// ---------------------------------------------------------------------------
// edge vectors from positions (grid over edges)
// ---------------------------------------------------------------------------
__global__ void mace_edge_vectors_kernel(const float* __restrict__ pos, MaceBox bx,
                                         const int64_t* __restrict__ src,
                                         const int64_t* __restrict__ dst, float* __restrict__ vec,
                                         int64_t n_edges) {
    const int64_t e = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (e >= n_edges) return;
    float v[3];
    edge_vector(pos, src[e], dst[e], bx.box, bx.inv, v);
    vec[e * 3 + 0] = v[0];
    vec[e * 3 + 1] = v[1];
    vec[e * 3 + 2] = v[2];
}

// ---------------------------------------------------------------------------
// h[e, :] = silu(B(r_e) W1 + b1), edges [e0, e1) of the chunk (row e - e0 of h)
// ---------------------------------------------------------------------------
__global__ __launch_bounds__(256) void mace_radial_kernel(const float* __restrict__ vec,
                                                          const float* __restrict__ w1,
                                                          const float* __restrict__ b1,
                                                          float* __restrict__ h, int64_t e0,
                                                          int64_t e1, float rc) {
    __shared__ float sW[kNBasis * kHidden + kHidden];
    for (int i = threadIdx.x; i < kNBasis * kHidden + kHidden; i += blockDim.x)
        sW[i] = i < kNBasis * kHidden ? w1[i] : b1[i - kNBasis * kHidden];
    __syncthreads();
    const int64_t e = e0 + (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (e >= e1) return;
    float vx = vec[e * 3], vy = vec[e * 3 + 1], vz = vec[e * 3 + 2];
    const float r = normalize3(vx, vy, vz);
    float B[kNBasis];
    radial_basis(r, rc, B, nullptr);
    float4* out = reinterpret_cast<float4*>(h + (e - e0) * kHidden);
#pragma unroll
    for (int j4 = 0; j4 < kHidden / 4; ++j4) {
        float z[4];
#pragma unroll
        for (int t = 0; t < 4; ++t) {
            const int j = j4 * 4 + t;
            float acc = sW[kNBasis * kHidden + j];
#pragma unroll
            for (int k = 0; k < kNBasis; ++k) acc = fmaf(B[k], sW[k * kHidden + j], acc);
            z[t] = acc * sigmoidf(acc);
        }
        out[j4] = make_float4(z[0], z[1], z[2], z[3]);
    }
}

// ---------------------------------------------------------------------------
// fp32 GEMM on MFMA: C[M, N] = A[M, K] B, with B = [K, N] (row-major) or, when
// TB, given as B^T [N, K] (row-major).  Workgroup tile 128 x BN, K step 16,
// four waves in 2 x 2, each 64 x BN/2 (4 x BN/32 MFMA tiles of 16 x 16).  Both
// operands sit in LDS with k contiguous (sA[m][k], sB[n][k]), so one float4
// read gives a lane its A (or B) values for four k-steps: k-step s of lane
// group g = lane / 16 is k = 4 g + s, the same for A and B.
// ---------------------------------------------------------------------------
template <bool TB, int BN>
__global__ __launch_bounds__(256) void gemm_f32_kernel(const float* __restrict__ A,
                                                       const float* __restrict__ B,
                                                       float* __restrict__ C, int M, int N, int K) {
    constexpr int BM = 128, BK = 16, WN = BN / 2, NT = WN / 16;
    constexpr int LD = BK + 4;  // row stride in floats (keeps float4 alignment)
    __shared__ __attribute__((aligned(16))) float sA[BM * LD];
    __shared__ __attribute__((aligned(16))) float sB[BN * LD];
    const int tid = threadIdx.x, lane = tid & 63, wv = tid >> 6;
    const int wm = wv >> 1, wn = wv & 1;
    const int g4 = lane >> 4, i16 = lane & 15;
    const int64_t m0 = (int64_t)blockIdx.y * BM;
    const int n0 = blockIdx.x * BN;
    const bool k4 = (K & 3) == 0, n4 = (N & 3) == 0;  // float4 global loads possible
    v4f acc[4][NT];
#pragma unroll
    for (int mi = 0; mi < 4; ++mi)
#pragma unroll
        for (int ni = 0; ni < NT; ++ni) acc[mi][ni] = v4f{0.f, 0.f, 0.f, 0.f};
    // one float4 of a row-major [rows, K] matrix (zeros past the edges)
    auto ld_rowk = [&](const float* P, int64_t row, int64_t rows, int k) {
        float4 v = make_float4(0.f, 0.f, 0.f, 0.f);
        if (row < rows) {
            const float* q = P + row * K + k;
            if (k4 && k + 3 < K) {
                v = *reinterpret_cast<const float4*>(q);
            } else {
                v.x = k < K ? q[0] : 0.f;
                v.y = k + 1 < K ? q[1] : 0.f;
                v.z = k + 2 < K ? q[2] : 0.f;
                v.w = k + 3 < K ? q[3] : 0.f;
            }
        }
        return v;
    };
    for (int k0 = 0; k0 < K; k0 += BK) {
        __syncthreads();
#pragma unroll
        for (int it = 0; it < BM * BK / 4 / 256; ++it) {
            const int idx = tid + it * 256, m = idx >> 2, kq = idx & 3;
            *reinterpret_cast<float4*>(sA + m * LD + 4 * kq) = ld_rowk(A, m0 + m, M, k0 + 4 * kq);
        }
        if constexpr (TB) {
#pragma unroll
            for (int it = 0; it < BN * BK / 4 / 256; ++it) {
                const int idx = tid + it * 256, n = idx >> 2, kq = idx & 3;
                *reinterpret_cast<float4*>(sB + n * LD + 4 * kq) = ld_rowk(B, n0 + n, N, k0 + 4 * kq);
            }
        } else {
#pragma unroll
            for (int it = 0; it < BN * BK / 4 / 256; ++it) {
                const int idx = tid + it * 256, k = idx / (BN / 4), nq = idx % (BN / 4);
                const int kk = k0 + k, nn = n0 + 4 * nq;
                float4 v = make_float4(0.f, 0.f, 0.f, 0.f);
                if (kk < K) {
                    const float* q = B + (int64_t)kk * N + nn;
                    if (n4 && nn + 3 < N) {
                        v = *reinterpret_cast<const float4*>(q);
                    } else {
                        v.x = nn < N ? q[0] : 0.f;
                        v.y = nn + 1 < N ? q[1] : 0.f;
                        v.z = nn + 2 < N ? q[2] : 0.f;
                        v.w = nn + 3 < N ? q[3] : 0.f;
                    }
                }
                sB[(4 * nq + 0) * LD + k] = v.x;
                sB[(4 * nq + 1) * LD + k] = v.y;
                sB[(4 * nq + 2) * LD + k] = v.z;
                sB[(4 * nq + 3) * LD + k] = v.w;
            }
        }
        __syncthreads();
        float4 a[4];
#pragma unroll
        for (int mi = 0; mi < 4; ++mi)
            a[mi] = *reinterpret_cast<const float4*>(sA + (wm * 64 + mi * 16 + i16) * LD + 4 * g4);
#pragma unroll
        for (int ni = 0; ni < NT; ++ni) {
            const float4 b =
                *reinterpret_cast<const float4*>(sB + (wn * WN + ni * 16 + i16) * LD + 4 * g4);
#pragma unroll
            for (int mi = 0; mi < 4; ++mi) acc[mi][ni] = mfma4(a[mi], b, acc[mi][ni]);
        }
    }
    // D[4 g4 + r][i16] of tile (mi, ni)
#pragma unroll
    for (int ni = 0; ni < NT; ++ni) {
        const int n = n0 + wn * WN + ni * 16 + i16;
        if (n >= N) continue;
#pragma unroll
        for (int mi = 0; mi < 4; ++mi)
#pragma unroll
            for (int r = 0; r < 4; ++r) {
                const int64_t m = m0 + wm * 64 + mi * 16 + 4 * g4 + r;
                if (m < M) C[m * N + n] = acc[mi][ni][r];
            }
    }
}

// ---------------------------------------------------------------------------
// Product kernels.  Threads are the channels of one edge at a time; a
// workgroup walks the destination rows that have edges in the chunk [e0, e1).
// Per path, T_p[e, c, o] = sum over the path's CG entries of c Y[b] x[a] is
// formed per thread from registers.  (Building K_p[o][a] = sum_b CG Y[b] once
// per edge and reading it as a broadcast operand measured slower here: from
// LDS each broadcast read still moves 1 KB per wave, from memory the scalar
// loads stall.)
// ---------------------------------------------------------------------------
// grid of the product kernels: at most chunk / 4 destination rows hold edges of
// a chunk when every row has 4 or more (grid-stride loop over the rows beyond)
static unsigned mace_row_blocks(int64_t chunk) { return (unsigned)(chunk / 4); }

// rows[2i], rows[2i+1]: first and one-past-last destination with an edge in
// chunk i = [i * chunk, min(E, (i + 1) * chunk)).
__global__ void mace_chunk_rows_kernel(const int64_t* __restrict__ row_ptr, int64_t N, int64_t E,
                                       int64_t chunk, int n_chunks, int64_t* __restrict__ rows) {
    const int i = blockIdx.x * blockDim.x + threadIdx.x;
    if (i >= n_chunks) return;
    const int64_t e0 = (int64_t)i * chunk, e1 = min(E, e0 + chunk);
    auto row_of = [&](int64_t k) {  // the row holding edge k: largest d with row_ptr[d] <= k
        int64_t lo = 0, hi = N - 1;
        while (lo < hi) {
            const int64_t mid = (lo + hi + 1) >> 1;
            if (row_ptr[mid] <= k) lo = mid;
            else hi = mid - 1;
        }
        return lo;
    };
    rows[2 * i] = row_of(e0);
    rows[2 * i + 1] = row_of(e1 - 1) + 1;
}

// One past the last path of the (l1, l2) block that starts at path p0 (the path
// order is l1 outer, l2, l_out inner, so a block's paths are consecutive).
constexpr int block_end(int p0) {
    int p = p0;
    while (p < kNumPaths && kPathL[p][0] == kPathL[p0][0] && kPathL[p][1] == kPathL[p0][1]) ++p;
    return p;
}
constexpr int path_slot(int p) { return p < kNumPaths ? kPathSlot[p] : kNumSlots; }

// Entry e of path p is the first of its path to write its output slot (when the
// entries are taken component a ascending, then in table order): the slot's
// accumulator starts from that term instead of from zero.
constexpr bool first_slot_write(int p, int e) {
    const CGEntry& x = kCG[kPathEntry[p] + e];
    for (int i = kPathEntry[p]; i < kPathEntry[p + 1]; ++i) {
        const CGEntry& y = kCG[i];
        if (y.q == x.q && (y.a < x.a || (y.a == x.a && i < kPathEntry[p] + e))) return false;
    }
    return true;
}
// The same for the input-2 component b (the backward's per-path sums over b).
constexpr bool first_b_write(int p, int e) {
    const CGEntry& x = kCG[kPathEntry[p] + e];
    for (int i = kPathEntry[p]; i < kPathEntry[p + 1]; ++i) {
        const CGEntry& y = kCG[i];
        if (y.b == x.b && (y.a < x.a || (y.a == x.a && i < kPathEntry[p] + e))) return false;
    }
    return true;
}
// every output slot and every component b of every path has an entry (so each
// accumulator is written before it is read)
constexpr bool every_slot_and_b_written() {
    for (int p = 0; p < kNumPaths; ++p) {
        const int lo = kPathL[p][2], l2 = kPathL[p][1];
        for (int o = lo * lo; o < (lo + 1) * (lo + 1); ++o) {
            bool f = false;
            for (int i = kPathEntry[p]; i < kPathEntry[p + 1]; ++i) f = f || kCG[i].o == o;
            if (!f) return false;
        }
        for (int b = l2 * l2; b < (l2 + 1) * (l2 + 1); ++b) {
            bool f = false;
            for (int i = kPathEntry[p]; i < kPathEntry[p + 1]; ++i) f = f || kCG[i].b == b;
            if (!f) return false;
        }
    }
    return true;
}
static_assert(every_slot_and_b_written(), "a path output or input-2 component without entries");

// x * c with c a compile-time coefficient (no multiply for c = 1)
template <int P, int E>
__device__ __forceinline__ float cg_times(float x) {
    constexpr float c = kCG[kPathEntry[P] + E].c;
    if constexpr (c == 1.0f) return x;
    else return c * x;
}

// f(P0, P1) for every (l1, l2) block [P0, P1) of paths, in path order.
template <int P0, typename F>
__device__ __forceinline__ void for_blocks(F&& f) {
    if constexpr (P0 < kNumPaths) {
        constexpr int P1 = block_end(P0);
        f(std::integral_constant<int, P0>{}, std::integral_constant<int, P1>{});
        for_blocks<P1>(f);
    }
}

// T_p[o] = sum over the entries (a, b, o) of p of c x[a] Y[b], for the paths of
// the (l1, l2) block [P0, P1), with each product x[a] Y[b] formed once for the
// block (256 products per edge and channel over all blocks, against one
// product c Y[b] per distinct (c, b) when the paths are taken one by one).
// consume(p, tq) receives T_p (2 l_out + 1 values) of every path of the block.
template <int P0, int P1, typename F>
__device__ __forceinline__ void block_products(const float* Y, const float* xs, F&& consume) {
    constexpr int L1 = kPathL[P0][0], L2 = kPathL[P0][1];
    constexpr int S0 = kPathSlot[P0], NT = path_slot(P1) - S0;
    float t[NT];  // each written first by its slot's first term
    static_for<2 * L1 + 1>([&](auto ia) {
        constexpr int a = L1 * L1 + decltype(ia)::value;
        float xy[2 * L2 + 1];
#pragma unroll
        for (int i = 0; i < 2 * L2 + 1; ++i) xy[i] = xs[a] * Y[L2 * L2 + i];
        static_for<P1 - P0>([&](auto pp) {
            constexpr int p = P0 + decltype(pp)::value;
            static_for<kPathEntry[p + 1] - kPathEntry[p]>([&](auto ee) {
                constexpr int e = decltype(ee)::value;
                constexpr CGEntry en = kCG[kPathEntry[p] + e];
                if constexpr (en.a == a) {
                    if constexpr (first_slot_write(p, e))
                        t[en.q - S0] = cg_times<p, e>(xy[en.b - L2 * L2]);
                    else
                        t[en.q - S0] = fmaf(en.c, xy[en.b - L2 * L2], t[en.q - S0]);
                }
            });
        });
    });
    static_for<P1 - P0>([&](auto pp) {
        constexpr int p = P0 + decltype(pp)::value;
        consume(std::integral_constant<int, p>{}, t + (kPathSlot[p] - S0));
    });
}

// m[o] += sum_p R_p T_p[o] over all paths (the forward's per-edge message).
__device__ __forceinline__ void mace_message(const float* Y, const float* xs, const float* rr,
                                             float* m) {
    for_blocks<0>([&](auto b0, auto b1) {
        block_products<decltype(b0)::value, decltype(b1)::value>(Y, xs, [&](auto pp, const float* tq) {
            constexpr int p = decltype(pp)::value;
            constexpr int lo = kPathL[p][2];
#pragma unroll
            for (int q = 0; q < 2 * lo + 1; ++q) m[lo * lo + q] = fmaf(rr[p], tq[q], m[lo * lo + q]);
        });
    });
}

// gy[b] = sum over the entries (a, b, o) of every path p of c x[a] R_p g[o],
// by (l1, l_out) blocks: each product x[a] g[o] is formed once (256 per edge
// and channel), the block's per-path sums U_p[b] = sum c x[a] g[o] (one path
// per l2 within the block, so U is indexed by b) are scaled by R_p once.
__device__ __forceinline__ void mace_grad_y(const float* xs, const float* g, const float* rr,
                                            float* gy) {
    static_for<4>([&](auto l1c) {
        constexpr int L1 = decltype(l1c)::value;
        static_for<4>([&](auto loc) {
            constexpr int LO = decltype(loc)::value;
            float U[16];  // U[b] written first by its first term (b of the block's paths only)
            static_for<2 * L1 + 1>([&](auto ia) {
                constexpr int a = L1 * L1 + decltype(ia)::value;
                float xg[2 * LO + 1];
#pragma unroll
                for (int i = 0; i < 2 * LO + 1; ++i) xg[i] = xs[a] * g[LO * LO + i];
                static_for<kNumPaths>([&](auto pp) {
                    constexpr int p = decltype(pp)::value;
                    if constexpr (kPathL[p][0] == L1 && kPathL[p][2] == LO)
                        static_for<kPathEntry[p + 1] - kPathEntry[p]>([&](auto ee) {
                            constexpr int e = decltype(ee)::value;
                            constexpr CGEntry en = kCG[kPathEntry[p] + e];
                            if constexpr (en.a == a) {
                                if constexpr (first_b_write(p, e))
                                    U[en.b] = cg_times<p, e>(xg[en.o - LO * LO]);
                                else
                                    U[en.b] = fmaf(en.c, xg[en.o - LO * LO], U[en.b]);
                            }
                        });
                });
            });
            static_for<kNumPaths>([&](auto pp) {
                constexpr int p = decltype(pp)::value;
                if constexpr (kPathL[p][0] == L1 && kPathL[p][2] == LO) {
                    constexpr int l2 = kPathL[p][1];
                    // gy[b] is first written by the l1 = 0 block of l_out = l2
#pragma unroll
                    for (int i = 0; i < 2 * l2 + 1; ++i)
                        gy[l2 * l2 + i] = L1 == 0 ? rr[p] * U[l2 * l2 + i]
                                                  : fmaf(rr[p], U[l2 * l2 + i], gy[l2 * l2 + i]);
                }
            });
        });
    });
}

// Y of edge k (unit vector of vec[k]).
__device__ __forceinline__ void mace_edge_sh(const float* __restrict__ vec, int64_t k, float* Y) {
    float ux = vec[k * 3], uy = vec[k * 3 + 1], uz = vec[k * 3 + 2];
    normalize3(ux, uy, uz);
    sh_forward<3>(ux, uy, uz, Y);
}

__device__ __forceinline__ void load_row16(const float* __restrict__ p, float* v) {
    const float4* q = reinterpret_cast<const float4*>(p);
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        const float4 t = q[i];
        v[4 * i] = t.x;
        v[4 * i + 1] = t.y;
        v[4 * i + 2] = t.z;
        v[4 * i + 3] = t.w;
    }
}

// First row and step of a workgroup's walk over the chunk's destination rows
// [d_lo, d_hi).  Without `order`: rows d_lo + blockIdx.x, + gridDim.x, ...  With
// `order` (n_pos positions, e.g. a spatial order): workgroup b takes position
// (b % 8) * gridDim.x / 8 + b / 8 (consecutive positions on one XCD, whose L2 then
// holds the source rows that neighbouring destinations share) and its row when that
// row is in the chunk; gridDim.x is a multiple of 8.
__device__ __forceinline__ void mace_row_walk(const int64_t* __restrict__ order, int64_t n_pos,
                                              int64_t d_lo, int64_t d_hi, int64_t& first,
                                              int64_t& step) {
    if (!order) {
        first = d_lo + blockIdx.x;
        step = gridDim.x;
        return;
    }
    const int64_t per_xcd = gridDim.x >> 3;
    const int64_t p = (int64_t)(blockIdx.x & 7) * per_xcd + (blockIdx.x >> 3);
    const int64_t d = p < n_pos ? order[p] : -1;
    first = (d >= d_lo && d < d_hi) ? d : d_hi;
    step = d_hi - d_lo + 1;  // one row
}

// Forward: out[d, c, :] += sum over the chunk's edges of row d of
// sum_p R[e, p, c] T_p[e, c, :] (R row e - e0 of the chunk, path-major).
__global__ __launch_bounds__(256) void mace_tp_scatter_kernel(
    const float* __restrict__ vec, const float* __restrict__ x, const int64_t* __restrict__ src,
    const int64_t* __restrict__ row_ptr, const float* __restrict__ R,
    const int64_t* __restrict__ rows, const int64_t* __restrict__ order, int64_t n_pos, int64_t e0,
    int64_t e1, float* __restrict__ out, int C) {
    const int c = blockIdx.y * blockDim.x + threadIdx.x;
    const bool live = c < C;
    const int cc = live ? c : C - 1;
    const int64_t d_lo = rows[0], d_hi = rows[1];
    int64_t d0, dstep;
    mace_row_walk(order, n_pos, d_lo, d_hi, d0, dstep);
    for (int64_t d = d0; d < d_hi; d += dstep) {
        const int64_t s = max(row_ptr[d], e0), e = min(row_ptr[d + 1], e1);
        float m[16];
#pragma unroll
        for (int o = 0; o < 16; ++o) m[o] = 0.0f;
        // operands of edge k: its R row (path offsets in a scalar register, no
        // per-load address math) and the source row
        auto load = [&](int64_t k, float* rr, float* xs) {
            const auto rs = buffer_rsrc(R + (k - e0) * C * kNumPaths, (uint32_t)C * kNumPaths * 4u);
#pragma unroll
            for (int p = 0; p < kNumPaths; ++p) rr[p] = buffer_ld(rs, cc * 4, p * C * 4);
            load_row16(x + (src[k] * C + cc) * 16, xs);
        };
        auto message = [&](int64_t k, const float* rr, const float* xs) {
            float Y[16];
            mace_edge_sh(vec, k, Y);
            mace_message(Y, xs, rr, m);
        };
        // two edges per step, each edge's loads issued one edge ahead (the
        // loads past the row's last edge re-read that edge: always in bounds)
        float rA[kNumPaths], xA[16], rB[kNumPaths], xB[16];
        if (s < e) load(s, rA, xA);
        int64_t k = s;
        for (; k + 1 < e; k += 2) {
            load(k + 1, rB, xB);
            message(k, rA, xA);
            load(min(k + 2, e - 1), rA, xA);
            message(k + 1, rB, xB);
        }
        if (k < e) message(k, rA, xA);
        if (live) {
            float4* op = reinterpret_cast<float4*>(out + (d * C + c) * 16);
#pragma unroll
            for (int q = 0; q < 4; ++q) {
                float4 t = op[q];
                t.x += m[4 * q];
                t.y += m[4 * q + 1];
                t.z += m[4 * q + 2];
                t.w += m[4 * q + 3];
                op[q] = t;
            }
        }
    }
}

// Sum of v[0..15] over the 64 lanes of a wave by recursive halving (each step
// halves the values a lane carries), in a fixed order.  Lane l with
// (l & 3) == 0 returns the total for b = 8 bit5 + 4 bit4 + 2 bit3 + bit2 of l.
__device__ __forceinline__ float wave_sum16(const float* v) {
    const int lane = threadIdx.x & 63;
    float a[8];
    {
        const bool hi = lane & 32;
#pragma unroll
        for (int i = 0; i < 8; ++i) {
            const float keep = hi ? v[8 + i] : v[i], send = hi ? v[i] : v[8 + i];
            a[i] = keep + __shfl_xor(send, 32, 64);
        }
    }
    float b4[4];
    {
        const bool hi = lane & 16;
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            const float keep = hi ? a[4 + i] : a[i], send = hi ? a[i] : a[4 + i];
            b4[i] = keep + __shfl_xor(send, 16, 64);
        }
    }
    float c2[2];
    {
        const bool hi = lane & 8;
#pragma unroll
        for (int i = 0; i < 2; ++i) {
            const float keep = hi ? b4[2 + i] : b4[i], send = hi ? b4[i] : b4[2 + i];
            c2[i] = keep + __shfl_xor(send, 8, 64);
        }
    }
    float t;
    {
        const bool hi = lane & 4;
        const float keep = hi ? c2[1] : c2[0], send = hi ? c2[0] : c2[1];
        t = keep + __shfl_xor(send, 4, 64);
    }
    t += __shfl_xor(t, 2, 64);
    t += __shfl_xor(t, 1, 64);
    return t;
}

// ---------------------------------------------------------------------------
// Backward, per edge of the chunk (threads = channels; the workgroup walks the
// destination rows with edges in the chunk):
//   gR[e, p, c] = sum_{m_out} g[d, c, o] T_p[e, c, m_out]
//   gY[e, b]    = sum_c sum_{(p, o, a)} CG[a, b, o] x[src, c, a] R[e, p, c] g[d, c, o]
// gY is summed over the channels in a fixed order: within a wave by
// recursive halving, then over the waves through LDS once per batch.
// ---------------------------------------------------------------------------
constexpr int kMaceEB = 8;  // edges per gY reduction batch of the backward

__global__ __launch_bounds__(256) void mace_tp_backward_kernel(
    const float* __restrict__ vec, const float* __restrict__ x, const int64_t* __restrict__ src,
    const int64_t* __restrict__ row_ptr, const float* __restrict__ R,
    const float* __restrict__ gout, const int64_t* __restrict__ rows,
    const int64_t* __restrict__ order, int64_t n_pos, int64_t e0, int64_t e1,
    float* __restrict__ gR, float* __restrict__ gY, int C) {
    __shared__ float sRed[4][kMaceEB][16];
    const int c = threadIdx.x;
    const bool live = c < C;
    const int cc = live ? c : C - 1;
    const int lane = threadIdx.x & 63, wv = threadIdx.x >> 6, nw = blockDim.x >> 6;
    const int my_b = 8 * ((lane >> 5) & 1) + 4 * ((lane >> 4) & 1) + 2 * ((lane >> 3) & 1) +
                     ((lane >> 2) & 1);
    const int64_t d_lo = rows[0], d_hi = rows[1];
    int64_t d0, dstep;
    mace_row_walk(order, n_pos, d_lo, d_hi, d0, dstep);
    for (int64_t d = d0; d < d_hi; d += dstep) {
        const int64_t s = max(row_ptr[d], e0), e = min(row_ptr[d + 1], e1);
        float g[16];
        load_row16(gout + (d * C + cc) * 16, g);
        if (!live) {
#pragma unroll
            for (int o = 0; o < 16; ++o) g[o] = 0.0f;
        }
        for (int64_t kb = s; kb < e; kb += kMaceEB) {
            const int nb = (int)min<int64_t>(kMaceEB, e - kb);
            __syncthreads();  // the previous batch's sums have been read from sRed
            for (int j = 0; j < nb; ++j) {
                const int64_t k = kb + j;
                float rr[kNumPaths];
                const auto rs = buffer_rsrc(R + (k - e0) * C * kNumPaths, (uint32_t)C * kNumPaths * 4u);
#pragma unroll
                for (int p = 0; p < kNumPaths; ++p) rr[p] = buffer_ld(rs, cc * 4, p * C * 4);
                float Y[16];
                mace_edge_sh(vec, k, Y);
                float xs[16];
                load_row16(x + (src[k] * C + cc) * 16, xs);
                const auto gs = buffer_rsrc(gR + (k - e0) * C * kNumPaths, (uint32_t)C * kNumPaths * 4u);
                // gR[p] = g . T_p (path-major: lanes write consecutive addresses)
                for_blocks<0>([&](auto b0, auto b1) {
                    block_products<decltype(b0)::value, decltype(b1)::value>(
                        Y, xs, [&](auto pp, const float* tq) {
                            constexpr int p = decltype(pp)::value;
                            constexpr int lo = kPathL[p][2];
                            float gr = 0.0f;
#pragma unroll
                            for (int q = 0; q < 2 * lo + 1; ++q) gr = fmaf(g[lo * lo + q], tq[q], gr);
                            if (live)
                                __builtin_amdgcn_raw_buffer_store_b32(__float_as_int(gr), gs, c * 4,
                                                                      p * C * 4, 0);
                        });
                });
                // gy[b] = sum over the entries (a, b, o) of c x[a] R_p g[o]
                float gy[16];
                mace_grad_y(xs, g, rr, gy);
                const float t = wave_sum16(gy);
                if ((lane & 3) == 0) sRed[wv][j][my_b] = t;
            }
            __syncthreads();
            for (int i = threadIdx.x; i < nb * 16; i += blockDim.x) {
                const int j = i >> 4, b = i & 15;
                float t = 0.0f;
                for (int w = 0; w < nw; ++w) t += sRed[w][j][b];
                gY[(kb + j - e0) * 16 + b] = t;
            }
        }
    }
}

// ---------------------------------------------------------------------------
// Backward through the radial MLP, the normalisation and SH, per edge:
//   g_v = g_r u + (g_u - u (u . g_u)) / r
// with g_r = sum_k (sum_j W1[k, j] g_h[j] silu'(z_j)) dB_k/dr and
// g_u = SH backward of gY at u.
// ---------------------------------------------------------------------------
__global__ __launch_bounds__(256) void mace_radial_backward_kernel(
    const float* __restrict__ vec, const float* __restrict__ w1, const float* __restrict__ b1,
    const float* __restrict__ gh, const float* __restrict__ gY, int64_t e0, int64_t e1, float rc,
    float* __restrict__ gv) {
    __shared__ float sW[kNBasis * kHidden + kHidden];
    for (int i = threadIdx.x; i < kNBasis * kHidden + kHidden; i += blockDim.x)
        sW[i] = i < kNBasis * kHidden ? w1[i] : b1[i - kNBasis * kHidden];
    __syncthreads();
    const int64_t e = e0 + (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (e >= e1) return;
    float ux = vec[e * 3], uy = vec[e * 3 + 1], uz = vec[e * 3 + 2];
    const float r = normalize3(ux, uy, uz);
    float B[kNBasis], dB[kNBasis];
    radial_basis(r, rc, B, dB);
    float gB[kNBasis];
#pragma unroll
    for (int k = 0; k < kNBasis; ++k) gB[k] = 0.0f;
    const float* ghr = gh + (e - e0) * kHidden;
    for (int j = 0; j < kHidden; ++j) {
        float z = sW[kNBasis * kHidden + j];
#pragma unroll
        for (int k = 0; k < kNBasis; ++k) z = fmaf(B[k], sW[k * kHidden + j], z);
        const float sg = sigmoidf(z);
        const float gz = ghr[j] * sg * (1.0f + z * (1.0f - sg));
#pragma unroll
        for (int k = 0; k < kNBasis; ++k) gB[k] = fmaf(sW[k * kHidden + j], gz, gB[k]);
    }
    float gr = 0.0f;
#pragma unroll
    for (int k = 0; k < kNBasis; ++k) gr = fmaf(gB[k], dB[k], gr);
    float Y[16], gyv[16];
    sh_forward<3>(ux, uy, uz, Y);
#pragma unroll
    for (int b = 0; b < 16; ++b) gyv[b] = gY[(e - e0) * 16 + b];
    float gux, guy, guz;
    sh_backward<3>(ux, uy, uz, Y, gyv, gux, guy, guz);
    const float dot = ux * gux + uy * guy + uz * guz;
    const float ir = 1.0f / r;
    gv[e * 3 + 0] = gr * ux + (gux - ux * dot) * ir;
    gv[e * 3 + 1] = gr * uy + (guy - uy * dot) * ir;
    gv[e * 3 + 2] = gr * uz + (guz - uz * dot) * ir;
}

// ---------------------------------------------------------------------------
// grad_pos[a] = sum_{e in row a} (g_v[e] - g_v[rev[e]]): v_e = pos[dst] -
// pos[src], and rev[e] is the edge with the roles of a and src_e swapped.
// ---------------------------------------------------------------------------
__global__ void mace_forces_kernel(const float* __restrict__ gv, const int64_t* __restrict__ row_ptr,
                                   const int64_t* __restrict__ rev, float* __restrict__ gpos,
                                   int64_t n) {
    const int64_t a = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (a >= n) return;
    float f0 = 0.f, f1 = 0.f, f2 = 0.f;
    for (int64_t e = row_ptr[a]; e < row_ptr[a + 1]; ++e) {
        const int64_t t = rev[e];
        if (t < 0) continue;  // edge list not symmetric (reported by the reverse-edge build)
        f0 += gv[e * 3 + 0] - gv[t * 3 + 0];
        f1 += gv[e * 3 + 1] - gv[t * 3 + 1];
        f2 += gv[e * 3 + 2] - gv[t * 3 + 2];
    }
    gpos[a * 3 + 0] = f0;
    gpos[a * 3 + 1] = f1;
    gpos[a * 3 + 2] = f2;
}

// rev[e] for e = (src j -> dst i): the edge (src i -> dst j), found by binary
// search in row j (sources ascending); -1 if the edge list is not symmetric.
__global__ void mace_reverse_edges_kernel(const int64_t* __restrict__ row_ptr,
                                          const int64_t* __restrict__ src,
                                          int64_t* __restrict__ rev, int* __restrict__ missing,
                                          int64_t n, int64_t n_edges) {
    const int64_t e = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (e >= n_edges) return;
    // destination of e: the row containing e
    int64_t lo = 0, hi = n;  // last row with row_ptr[row] <= e
    while (hi - lo > 1) {
        const int64_t mid = (lo + hi) >> 1;
        if (row_ptr[mid] <= e) lo = mid;
        else hi = mid;
    }
    const int64_t i = lo, j = src[e];
    int64_t a = row_ptr[j], b = row_ptr[j + 1];  // first position with src >= i
    while (a < b) {
        const int64_t mid = (a + b) >> 1;
        if (src[mid] < i) a = mid + 1;
        else b = mid;
    }
    const bool ok = a < row_ptr[j + 1] && src[a] == i;
    rev[e] = ok ? a : -1;
    if (!ok) atomicAdd(missing, 1);
}

__global__ void mace_fill_zero_kernel(float* __restrict__ p, int64_t count) {
    const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (i < count) p[i] = 0.0f;
}

__global__ void mace_zero_int_kernel(int* __restrict__ p) { *p = 0; }

struct MaceWs {
    float *vec, *h, *R, *gR, *gh, *gY, *gv;
    int64_t* rows;  // destination range of every chunk
    size_t bytes;
};

static size_t a256(size_t x) { return (x + 255) & ~size_t(255); }

// external: the per-edge weights of all edges live in a caller buffer
// (batteries_mace_edge_weight_rows rows of 34 C), so the workspace holds no R chunk.
static MaceWs mace_ws(void* base, int64_t E, int C, bool backward, bool external = false) {
    const int64_t chunk = mace_chunk(E, C);
    const int64_t eb = std::min<int64_t>(std::max<int64_t>(E, 1), chunk);
    char* p = static_cast<char*>(base);
    size_t o = 0;
    MaceWs w{};
    auto take = [&](size_t bytes) {
        float* r = p ? reinterpret_cast<float*>(p + o) : nullptr;
        o = a256(o + bytes);
        return r;
    };
    w.vec = take(sizeof(float) * 3 * (size_t)E);
    w.rows = reinterpret_cast<int64_t*>(
        take(sizeof(int64_t) * 2 * (size_t)ceil_div(std::max<int64_t>(E, 1), chunk)));
    w.h = take(sizeof(float) * (size_t)eb * kHidden);
    w.R = external ? nullptr : take(sizeof(float) * (size_t)eb * C * kNumPaths);
    if (backward) {
        w.gR = take(sizeof(float) * (size_t)eb * C * kNumPaths);
        w.gh = take(sizeof(float) * (size_t)eb * kHidden);
        w.gY = take(sizeof(float) * (size_t)eb * 16);
        w.gv = take(sizeof(float) * 3 * (size_t)E);
    }
    w.bytes = o;
    return w;
}

static int gemm_launch(const float* A, const float* B, float* Cm, int64_t M, int N, int K, bool tb,
                       hipStream_t s) {
    if (M <= 0 || N <= 0 || K <= 0) return BM_OK;
    const bool narrow = N <= 64;  // 128 x 64 tiles for narrow outputs, else 128 x 128
    const int bn = narrow ? 64 : 128;
    dim3 grid((unsigned)ceil_div(N, bn), (unsigned)ceil_div(M, 128));
    if (grid.y > 65535) return BM_ERR_ARG;
    if (tb) {
        if (narrow) gemm_f32_kernel<true, 64><<<grid, 256, 0, s>>>(A, B, Cm, (int)M, N, K);
        else gemm_f32_kernel<true, 128><<<grid, 256, 0, s>>>(A, B, Cm, (int)M, N, K);
    } else {
        if (narrow) gemm_f32_kernel<false, 64><<<grid, 256, 0, s>>>(A, B, Cm, (int)M, N, K);
        else gemm_f32_kernel<false, 128><<<grid, 256, 0, s>>>(A, B, Cm, (int)M, N, K);
    }
    return (int)hipGetLastError();
}

// The layer's two GEMMs (R = h W2 and g_h = gR W2^T) are plain fp32 GEMMs and
// go to rocBLAS, which runs these shapes faster than gemm_f32_kernel (65536 x
// 64 x 4352: 478 vs 525 us; 65536 x 4352 x 64: 361 vs 659 us on one MI355X).
// One handle per device, bound to the caller's stream on every call.
static rocblas_handle blas_handle() {
    static std::mutex mu;
    static rocblas_handle handles[64] = {};
    int dev = 0;
    if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 64) return nullptr;
    std::lock_guard<std::mutex> lock(mu);
    if (!handles[dev] && rocblas_create_handle(&handles[dev]) != rocblas_status_success)
        handles[dev] = nullptr;
    return handles[dev];
}

// Row-major C[M x N] = A[M x K] B[K x N] (tb: B given as [N x K], C = A B^T),
// as the column-major product C^T = B^T A^T.
static int blas_gemm(const float* A, const float* B, float* Cm, int64_t M, int N, int K, bool tb,
                     hipStream_t s) {
    if (M <= 0 || N <= 0 || K <= 0) return BM_OK;
    if (M > INT32_MAX) return BM_ERR_ARG;
    rocblas_handle h = blas_handle();
    if (!h || rocblas_set_stream(h, s) != rocblas_status_success) return BM_ERR_BLAS;
    const float one = 1.0f, zero = 0.0f;
    const rocblas_status st =
        tb ? rocblas_sgemm(h, rocblas_operation_transpose, rocblas_operation_none, N, (int)M, K,
                           &one, B, K, A, K, &zero, Cm, N)
           : rocblas_sgemm(h, rocblas_operation_none, rocblas_operation_none, N, (int)M, K, &one,
                           B, N, A, K, &zero, Cm, N);
    return st == rocblas_status_success ? BM_OK : BM_ERR_BLAS;
}

// Rows of a chunk's GEMMs: a graph of more than one chunk runs every chunk's
// GEMMs at the full chunk height (the workspace holds a chunk's rows; rows
// past the chunk's last edge hold the previous chunk's finite values and their
// results are never read), so that rocBLAS picks the same kernel for the last,
// shorter chunk (65536 x 64 x 4352 at 323 us; 57844 rows picked a 992 us one).
static int64_t gemm_rows(int64_t n_edges, int64_t eb, int64_t chunk) {
    return n_edges > chunk ? chunk : eb;
}

}  // namespace bmhip

using namespace bmhip;

extern "C" int batteries_gemm_f32(const float* A, const float* B, float* C, int64_t M, int N, int K,
                                  int trans_b, hipStream_t stream) {
    if (M < 0 || N < 0 || K < 0 || M > INT32_MAX) return BM_ERR_ARG;
    return gemm_launch(A, B, C, M, N, K, trans_b != 0, stream);
}

extern "C" size_t batteries_mace_workspace_bytes(int64_t N_edges, int C, int backward,
                                                 int external_weights) {
    if (N_edges < 0 || C <= 0) return 0;
    return mace_ws(nullptr, N_edges, C, backward != 0, external_weights != 0).bytes;
}

// Rows of a caller buffer for the per-edge weights of all edges: whole chunks
// (every chunk's GEMM writes a full chunk of rows; rows past N_edges are padding).
extern "C" int64_t batteries_mace_edge_weight_rows(int64_t N_edges, int C) {
    if (N_edges <= 0 || C <= 0) return 0;
    const int64_t chunk = mace_chunk(N_edges, C);
    return ceil_div(N_edges, chunk) * chunk;
}

extern "C" int batteries_mace_reverse_edges(const int64_t* row_ptr, const int64_t* src,
                                            int64_t* rev, int* d_missing, int64_t N,
                                            int64_t N_edges, hipStream_t stream) {
    if (N < 0 || N_edges < 0 || !d_missing) return BM_ERR_ARG;
    mace_zero_int_kernel<<<1, 1, 0, stream>>>(d_missing);
    if (N_edges == 0) return (int)hipGetLastError();
    mace_reverse_edges_kernel<<<(unsigned)ceil_div(N_edges, 256), 256, 0, stream>>>(
        row_ptr, src, rev, d_missing, N, N_edges);
    return (int)hipGetLastError();
}

static bool mace_args_ok(const float* box, int64_t N, int64_t E, int C, float cutoff) {
    if (!box || N < 0 || E < 0 || C <= 0 || C > 256 || !(cutoff > 0.0f)) return false;
    if (ceil_div(N, 8) * 8 > INT32_MAX) return false;  // one workgroup per position
    for (int k = 0; k < 3; ++k)
        if (!(box[k] > 0.0f)) return false;
    return true;  // chunk offsets are kept within 32 bits by mace_chunk
}

static MaceBox mace_box(const float* box) {
    MaceBox b;
    for (int k = 0; k < 3; ++k) {
        b.box[k] = box[k];
        b.inv[k] = 1.0f / box[k];
    }
    return b;
}

extern "C" int batteries_mace_forward(const float* positions, const float* box,
                                      const float* node_features, const float* w1,
                                      const float* b1, const float* w2, const int64_t* src,
                                      const int64_t* dst, const int64_t* row_ptr,
                                      const int64_t* order, float* out,
                                      float* edge_weights, int64_t N, int64_t N_edges, int C,
                                      float cutoff, void* workspace, size_t workspace_bytes,
                                      hipStream_t stream) {
    if (!mace_args_ok(box, N, N_edges, C, cutoff)) return BM_ERR_ARG;
    if (N == 0) return BM_OK;
    const MaceWs w = mace_ws(workspace, N_edges, C, false, edge_weights != nullptr);
    if (!workspace || workspace_bytes < w.bytes) return BM_ERR_WORKSPACE;
    const int64_t count = N * (int64_t)C * 16;
    mace_fill_zero_kernel<<<(unsigned)ceil_div(count, 256), 256, 0, stream>>>(out, count);
    if (N_edges == 0) return (int)hipGetLastError();
    const MaceBox bx = mace_box(box);
    mace_edge_vectors_kernel<<<(unsigned)ceil_div(N_edges, 256), 256, 0, stream>>>(
        positions, bx, src, dst, w.vec, N_edges);
    const int nthr = C >= 256 ? 256 : (int)ceil_div(C, 64) * 64;
    const int64_t chunk = mace_chunk(N_edges, C);
    const int n_chunks = (int)ceil_div(N_edges, chunk);
    mace_chunk_rows_kernel<<<(unsigned)ceil_div(n_chunks, 64), 64, 0, stream>>>(
        row_ptr, N, N_edges, chunk, n_chunks, w.rows);
    for (int64_t e0 = 0; e0 < N_edges; e0 += chunk) {
        const int64_t e1 = std::min(N_edges, e0 + chunk), eb = e1 - e0;
        // this chunk's R: the workspace chunk, or rows e0.. of the caller's buffer
        float* R = edge_weights ? edge_weights + e0 * (int64_t)C * kNumPaths : w.R;
        mace_radial_kernel<<<(unsigned)ceil_div(eb, 256), 256, 0, stream>>>(w.vec, w1, b1, w.h, e0,
                                                                             e1, cutoff);
        int rc = blas_gemm(w.h, w2, R, gemm_rows(N_edges, eb, chunk), C * kNumPaths, kHidden, false,
                           stream);
        if (rc != BM_OK) return rc;
        dim3 grid(order ? (unsigned)(ceil_div(N, 8) * 8) : mace_row_blocks(chunk),
                  (unsigned)ceil_div(C, nthr));
        mace_tp_scatter_kernel<<<grid, nthr, 0, stream>>>(w.vec, node_features, src, row_ptr, R,
                                                          w.rows + 2 * (e0 / chunk), order, N,
                                                          e0, e1, out, C);
    }
    return (int)hipGetLastError();
}

extern "C" int batteries_mace_backward(const float* positions, const float* box,
                                       const float* node_features, const float* w1,
                                       const float* b1, const float* w2, const int64_t* src,
                                       const int64_t* dst, const int64_t* row_ptr,
                                       const int64_t* order, const int64_t* rev,
                                       const float* grad_out,
                                       const float* edge_weights, float* grad_pos, int64_t N,
                                       int64_t N_edges, int C, float cutoff, void* workspace,
                                       size_t workspace_bytes, hipStream_t stream) {
    if (!mace_args_ok(box, N, N_edges, C, cutoff)) return BM_ERR_ARG;
    if (N == 0) return BM_OK;
    const MaceWs w = mace_ws(workspace, N_edges, C, true, edge_weights != nullptr);
    if (!workspace || workspace_bytes < w.bytes) return BM_ERR_WORKSPACE;
    if (N_edges == 0) {
        mace_fill_zero_kernel<<<(unsigned)ceil_div(N * 3, 256), 256, 0, stream>>>(grad_pos, N * 3);
        return (int)hipGetLastError();
    }
    const MaceBox bx = mace_box(box);
    mace_edge_vectors_kernel<<<(unsigned)ceil_div(N_edges, 256), 256, 0, stream>>>(
        positions, bx, src, dst, w.vec, N_edges);
    const int nthr = (int)ceil_div(C, 64) * 64;
    const int64_t chunk = mace_chunk(N_edges, C);
    const int n_chunks = (int)ceil_div(N_edges, chunk);
    mace_chunk_rows_kernel<<<(unsigned)ceil_div(n_chunks, 64), 64, 0, stream>>>(
        row_ptr, N, N_edges, chunk, n_chunks, w.rows);
    for (int64_t e0 = 0; e0 < N_edges; e0 += chunk) {
        const int64_t e1 = std::min(N_edges, e0 + chunk), eb = e1 - e0;
        // R: the forward's saved weights (rows e0..), or recomputed into the workspace
        const float* R = edge_weights ? edge_weights + e0 * (int64_t)C * kNumPaths : w.R;
        int rc = BM_OK;
        if (!edge_weights) {
            mace_radial_kernel<<<(unsigned)ceil_div(eb, 256), 256, 0, stream>>>(w.vec, w1, b1, w.h,
                                                                                 e0, e1, cutoff);
            rc = blas_gemm(w.h, w2, w.R, gemm_rows(N_edges, eb, chunk), C * kNumPaths, kHidden,
                           false, stream);
            if (rc != BM_OK) return rc;
        }
        mace_tp_backward_kernel<<<order ? (unsigned)(ceil_div(N, 8) * 8) : mace_row_blocks(chunk),
                                  nthr, 0, stream>>>(w.vec, node_features, src, row_ptr, R,
                                                     grad_out, w.rows + 2 * (e0 / chunk), order,
                                                     N, e0, e1, w.gR, w.gY, C);
        rc = blas_gemm(w.gR, w2, w.gh, gemm_rows(N_edges, eb, chunk), kHidden, C * kNumPaths, true, stream);
        if (rc != BM_OK) return rc;
        mace_radial_backward_kernel<<<(unsigned)ceil_div(eb, 256), 256, 0, stream>>>(
            w.vec, w1, b1, w.gh, w.gY, e0, e1, cutoff, w.gv);
    }
    mace_forces_kernel<<<(unsigned)ceil_div(N, 256), 256, 0, stream>>>(w.gv, row_ptr, rev, grad_pos,
                                                                        N);
    return (int)hipGetLastError();
}
