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
// (557 kflop per edge at C = 128).  One kernel per pass runs it on MFMA and
// consumes each tile of per-edge weights R straight from the accumulators in
// the channel-wise CG product on the VALU (611 products with a coefficient,
// 256 bilinear products and 156 path weightings per edge and channel), so R
// (26 GB at configs[4]) never reaches memory.  The backward runs the same
// tiles with the MLP's transpose GEMM on MFMA fed by the path gradients, and
// ends in per-edge position gradients; forces are gathered per atom through
// the reverse-edge map of the symmetric edge list.  Every sum runs in a fixed
// order (deterministic, no atomics).
#include "common.h"
#include "batmobile_hip.h"

namespace bmhip {

constexpr int kNBasis = 8;
constexpr int kHidden = 64;

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

__device__ __forceinline__ float sigmoidf(float z) { return 1.0f / (1.0f + expf(-z)); }

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

// The backward's two contractions of c x[a] Y[b] g[o], by (l1, l_out) blocks:
// each product x[a] g[o] is formed once (256 per edge and channel) and summed
// into the block's per-path U_p[b] = sum c x[a] g[o] (one path per l2 within the
// block, so U is indexed by b); then
//   gy[b] += R_p U_p[b]                      (the gradient of the pair's Y)
//   path_grad(p, sum_b Y[b] U_p[b])         (gR_p = g . T_p(x, Y), the weight gradient)
// so both come from the one set of U (1179 operations per edge and channel against
// 2046 with T_p formed for gR_p separately).
template <typename F>
__device__ __forceinline__ void mace_grad_y(const float* xs, const float* g, const float* Y,
                                            const float* rr, float* gy, F&& path_grad) {
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
                    float gr = Y[l2 * l2] * U[l2 * l2];
#pragma unroll
                    for (int i = 1; i < 2 * l2 + 1; ++i) gr = fmaf(Y[l2 * l2 + i], U[l2 * l2 + i], gr);
                    path_grad(std::integral_constant<int, p>{}, gr);
                }
            });
        });
    });
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

// ---------------------------------------------------------------------------
// Fused layer kernels.
//
// Edges are taken in "positions": the destinations in the given order (a
// spatial order keeps shared source rows in cache), each destination's edges
// consecutive and ascending.  A prepass writes per position the unit vector and
// length, the source and destination, and the radial MLP's hidden layer h
// [E][64] (the backward also s[E][64], below).
//
// A workgroup owns one quad of 4 channels c0..c0+3 and keeps that quad's slice
// of W2 in LDS as sW[g][4 ch + j][k] = W2[k][(4g + j) C + c0 + ch] (paths in 9
// groups of 4, the last two slots zero; rows of 68 floats).  Each of its 4
// waves walks its own range of positions (ranges end at destination
// boundaries) in tiles of 16 edges.  Per tile, v_mfma_f32_16x16x4f32 gives
//   D[4 ch + j][e] = sum_k W2[k][(4g + j) C + c0 + ch] h[e][k]  = R[e, c0 + ch, 4g + j]
// (A = the W2 rows from LDS, B = h of the tile, K = 64 in 16 steps, 9 groups:
// 144 MFMAs), and by the accumulator layout lane l = 16 ch + e holds the 34
// weights of its own (edge e, channel c0 + ch) pair.  The lane then forms the
// message of that pair, sum_p R_p T_p(x[src, c], Y(u)), on the VALU.
// R never leaves the registers.
//
// Each destination's messages are summed in ascending edge order by one lane
// after another along the tile (lane e adds lane e - 1's running sum when both
// belong to the same destination), the running sum of a destination that
// continues into the next tile carried in LDS.  The sum is therefore the same
// sequence of additions whatever the tiling, the order of the destinations or
// the launch shape; each output row is written once, with no atomics.
// ---------------------------------------------------------------------------
constexpr int kMaceFwdWaves = 8;                     // waves (position ranges) per workgroup
constexpr int kMaceBwdWaves = 4;
constexpr int kPG = 9;                               // groups of 4 paths (36 slots)
constexpr int kW2Row = kHidden + 4;                  // LDS row of sW, in floats
constexpr int kW2Floats = kPG * 16 * kW2Row;         // 39,168 bytes per channel quad
constexpr int kMaceMaxWorkers = 8192;                // position ranges (wstart entries - 1)

// sW for the channel quad c0..c0+3 (zeros past path 33 and past channel C - 1)
__device__ __forceinline__ void mace_fill_w2(const float* __restrict__ w2, int C, int c0,
                                             float* sW) {
    for (int i = threadIdx.x; i < kHidden * 36 * 4; i += blockDim.x) {
        const int ch = i & 3, p = (i >> 2) % 36, k = i / 144;
        const int c = c0 + ch;
        float v = 0.0f;
        if (p < kNumPaths && c < C) v = w2[(int64_t)k * kNumPaths * C + p * C + c];
        sW[((p >> 2) * 16 + 4 * ch + (p & 3)) * kW2Row + k] = v;
    }
}

// The 34 weights of the lane's pair: sA = sW + (lane % 16) row + 4 (lane / 16),
// hb[j] = h[e][16 j + 4 (lane / 16) .. + 3] (k-step s of block j is
// k = 16 j + 4 (lane / 16) + s for both operands).
__device__ __forceinline__ void mace_tile_weights(const float* sA, const float4* hb, float* rr) {
    // the W2 operands are the same for every tile: read them from LDS per tile (an
    // opaque base keeps the compiler from hoisting all 36 reads, 144 registers, out
    // of the tile loop)
    int base = 0;
    asm volatile("" : "+v"(base));
    sA += base;
    v4f acc[kPG];
#pragma unroll
    for (int g = 0; g < kPG; ++g) acc[g] = v4f{0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int j = 0; j < 4; ++j) {
#pragma unroll
        for (int g = 0; g < kPG; ++g) {
            const float4 a = *reinterpret_cast<const float4*>(sA + g * 16 * kW2Row + 16 * j);
            acc[g] = mfma4(a, hb[j], acc[g]);
        }
    }
#pragma unroll
    for (int p = 0; p < kNumPaths; ++p) rr[p] = acc[p >> 2][p & 3];
}

// Lane reads within the 16-lane row.  Call them where every lane runs (a lane that
// reads a lane skipped by a branch, e.g. the right side of a short-circuit ||,
// gets no value).
__device__ __forceinline__ int dpp_prev_i(int v) {  // lane e - 1
    return __builtin_amdgcn_update_dpp(0, v, 0x111, 0xF, 0xF, false);
}
__device__ __forceinline__ int dpp_next_i(int v) {  // lane e + 1 of the 16-lane row
    return __builtin_amdgcn_update_dpp(0, v, 0x101, 0xF, 0xF, false);
}

// One tile's per-position operands (pos clamped into the range by the caller).
struct MaceTileIn {
    float4 hb[4];
    float4 u;  // unit vector, length
    int s, d;
};

__device__ __forceinline__ void mace_load_tile(const float4* __restrict__ u4,
                                               const int* __restrict__ srcp,
                                               const int* __restrict__ dstp,
                                               const float* __restrict__ h, int64_t pos, int kk,
                                               MaceTileIn& t) {
    const float4* hr = reinterpret_cast<const float4*>(h + pos * kHidden + 4 * kk);
#pragma unroll
    for (int j = 0; j < 4; ++j) t.hb[j] = hr[4 * j];
    t.u = u4[pos];
    t.s = srcp[pos];
    t.d = dstp[pos];
}

// Sum of the tile's messages over each destination, in ascending edge order.
// The 16 x 16 messages of a row (channel) go through LDS so that lane (row, o)
// holds component o of all 16 edges; it adds them one after another into acc,
// restarting at each destination's first edge (the tile's destination pattern
// is the same on every row, so it is one scalar bit mask), and stores acc when a
// destination closes.  acc carries a destination that continues into the next
// tile.  sT: [row (272 floats)][edge (16)][component, in quads rotated by
// edge / 4] (conflict-free 16-byte writes and 4-byte reads).
constexpr int kTRow = 272;
// messages to LDS: lane (row kk, edge e16) writes its 16 components
__device__ __forceinline__ void mace_stage_tile(const float* v, int e16, int kk, float* sT) {
#pragma unroll
    for (int i = 0; i < 4; ++i)
        *reinterpret_cast<float4*>(sT + kk * kTRow + e16 * 16 + 4 * ((i + (e16 >> 2)) & 3)) =
            make_float4(v[4 * i], v[4 * i + 1], v[4 * i + 2], v[4 * i + 3]);
}
__device__ __forceinline__ void mace_scatter_tile(int d, bool valid, int e16, int kk, bool cok,
                                                  int64_t c, int C, const float* sT, float& acc,
                                                  int& carry_d, float* __restrict__ out) {
    const int dp = dpp_prev_i(d), dn = dpp_next_i(d);
    const uint64_t head = __ballot((e16 == 0) | (dp != d));
    const uint64_t ends = __ballot(valid & (e16 < 15) & (dn != d));
    const int d0 = __builtin_amdgcn_readfirstlane(d);  // lane 0 of a tile is always valid
    // component o = e16 of row kk for all 16 edges
    float col[16];
#pragma unroll
    for (int e = 0; e < 16; ++e)
        col[e] = sT[kk * kTRow + e * 16 + 4 * (((e16 >> 2) + (e >> 2)) & 3) + (e16 & 3)];
    float* orow = out + c * 16 + e16;  // + destination * C * 16
    if (carry_d >= 0 && d0 != carry_d && cok) orow[(int64_t)carry_d * C * 16] = acc;
    acc = (d0 == carry_d) ? acc + col[0] : col[0];
#pragma unroll
    for (int e = 0; e < 16; ++e) {
        if (e > 0) acc = ((head >> e) & 1) ? col[e] : acc + col[e];
        if ((ends >> e) & 1) {
            const int de = __builtin_amdgcn_readlane(d, e);
            if (cok) orow[(int64_t)de * C * 16] = acc;
        }
    }
    carry_d = __builtin_amdgcn_readlane(d, 15);  // -1: the tile's last lane is past the range
}

// Workgroup -> (channel quad, position range): consecutive workgroup ids go to
// consecutive XCDs, so (bid % 8, bid / 8) puts all quads of a position range on one
// XCD, whose L2 then serves the range's h rows to every quad.
struct MaceWg {
    int quad, wave_range;
};
template <int WAVES>
__device__ __forceinline__ MaceWg mace_wg(int n_quads, int ranges_per_xcd) {
    const int bid = blockIdx.x, xcd = bid & 7, k = bid >> 3;
    MaceWg w;
    w.quad = k % n_quads;
    w.wave_range = ((xcd * ranges_per_xcd + k / n_quads) * WAVES) + (threadIdx.x >> 6);
    return w;
}

// out[d, c, :] = sum_{e -> d} sum_p R[e, c, p] T_p(x[src_e, c], Y(u_e)) for every
// destination with an edge (out of the others is zeroed by the caller).
__global__ __launch_bounds__(64 * kMaceFwdWaves) __attribute__((amdgpu_waves_per_eu(4))) void
mace_fused_forward_kernel(const float4* __restrict__ u4, const int* __restrict__ srcp,
                          const int* __restrict__ dstp, const float* __restrict__ h,
                          const float* __restrict__ w2, const float* __restrict__ x,
                          const int64_t* __restrict__ wstart, float* __restrict__ out, int C,
                          int n_quads, int ranges_per_xcd) {
    __shared__ __attribute__((aligned(16))) float sW[kW2Floats];
    __shared__ __attribute__((aligned(16))) float sTAll[kMaceFwdWaves * 4 * kTRow];
    const MaceWg wg = mace_wg<kMaceFwdWaves>(n_quads, ranges_per_xcd);
    const int lane = threadIdx.x & 63, e16 = lane & 15, kk = lane >> 4;
    const int c0 = wg.quad * 4;
    mace_fill_w2(w2, C, c0, sW);
    __syncthreads();
    float* sT = sTAll + (threadIdx.x >> 6) * 4 * kTRow;
    const int64_t p0 = wstart[wg.wave_range], p1 = wstart[wg.wave_range + 1];
    const int c = c0 + kk;
    const bool cok = c < C;
    const int cc = cok ? c : C - 1;
    const float* sA = sW + (lane & 15) * kW2Row + 4 * kk;
    int carry_d = -1;
    float acc = 0.0f;
    MaceTileIn cur;
    if (p0 < p1) mace_load_tile(u4, srcp, dstp, h, min(p0 + e16, p1 - 1), kk, cur);
    for (int64_t t0 = p0; t0 < p1; t0 += 16) {
        const bool valid = t0 + e16 < p1;
        // source row of the pair (issued first: the MFMAs below hide its latency)
        float xs[16];
        load_row16(x + ((int64_t)cur.s * C + cc) * 16, xs);
        if (!valid) {
#pragma unroll
            for (int j = 0; j < 4; ++j) cur.hb[j] = make_float4(0.f, 0.f, 0.f, 0.f);
        }
        float rr[kNumPaths];
        mace_tile_weights(sA, cur.hb, rr);
        float Y[16];
        sh_forward<3>(cur.u.x, cur.u.y, cur.u.z, Y);
        float m[16];
#pragma unroll
        for (int o = 0; o < 16; ++o) m[o] = 0.0f;
        mace_message(Y, xs, rr, m);
        mace_stage_tile(m, e16, kk, sT);
        const int dcur = valid ? cur.d : -1;
        // the next tile's operands (the other waves of the SIMD cover their latency)
        const int64_t t1 = t0 + 16;
        mace_load_tile(u4, srcp, dstp, h, t1 < p1 ? min(t1 + e16, p1 - 1) : p1 - 1, kk, cur);
        mace_scatter_tile(dcur, valid, e16, kk, cok, c, C, sT, acc, carry_d, out);
    }
    if (carry_d >= 0 && cok) out[((int64_t)carry_d * C + c) * 16 + e16] = acc;
}

// Backward: per pair, gR_p = sum_o g[d, c, o] T_p[o] feeds the MLP's transpose GEMM
//   D[k][e] += sum_{ch} W2[k][p C + c0 + ch] gR[e, c0 + ch, p]   (K = the quad's 4
// channels, one MFMA per path and 16-row block of k: A = W2 from LDS, B = the lane's
// own gR_p), and gY[b] = sum c x[a] R_p g[o] is summed over the quad's channels.
// The quad's share of the edge's position gradient,
//   g_v = g_r u + (g_u - u (u . g_u)) / r,  g_r = sum_k D[k][e] s[e][k],
//   g_u = SH backward of gY at u,
// with s[e][k] = silu'(z_k) sum_b W1[b][k] dB_b/dr, goes to gv_part[quad][position].
__global__ __launch_bounds__(64 * kMaceBwdWaves) __attribute__((amdgpu_waves_per_eu(3))) void mace_fused_backward_kernel(
    const float4* __restrict__ u4, const int* __restrict__ srcp, const int* __restrict__ dstp,
    const float* __restrict__ h, const float* __restrict__ sg, const float* __restrict__ w2,
    const float* __restrict__ x, const float* __restrict__ gout,
    const int64_t* __restrict__ wstart, float* __restrict__ gv_part, int64_t n_pos, int C,
    int n_quads, int ranges_per_xcd) {
    __shared__ __attribute__((aligned(16))) float sW[kW2Floats];
    const MaceWg wg = mace_wg<kMaceBwdWaves>(n_quads, ranges_per_xcd);
    const int lane = threadIdx.x & 63, e16 = lane & 15, kk = lane >> 4;
    const int c0 = wg.quad * 4;
    mace_fill_w2(w2, C, c0, sW);
    __syncthreads();
    const int64_t p0 = wstart[wg.wave_range], p1 = wstart[wg.wave_range + 1];
    const int c = c0 + kk;
    const bool cok = c < C;
    const int cc = cok ? c : C - 1;
    const float* sA = sW + (lane & 15) * kW2Row + 4 * kk;
    float* gvq = gv_part + (int64_t)wg.quad * n_pos * 3;
    MaceTileIn cur;
    if (p0 < p1) mace_load_tile(u4, srcp, dstp, h, min(p0 + e16, p1 - 1), kk, cur);
    for (int64_t t0 = p0; t0 < p1; t0 += 16) {
        const int64_t pos = t0 + e16;
        const bool valid = pos < p1;
        const int64_t pc = valid ? pos : p1 - 1;
        float xs[16], g[16];
        load_row16(x + ((int64_t)cur.s * C + cc) * 16, xs);
        load_row16(gout + ((int64_t)cur.d * C + cc) * 16, g);
        if (!valid) {
#pragma unroll
            for (int j = 0; j < 4; ++j) cur.hb[j] = make_float4(0.f, 0.f, 0.f, 0.f);
        }
        float rr[kNumPaths];
        mace_tile_weights(sA, cur.hb, rr);
        if (!(valid && cok)) {
#pragma unroll
            for (int o = 0; o < 16; ++o) g[o] = 0.0f;
        }
        float Y[16];
        sh_forward<3>(cur.u.x, cur.u.y, cur.u.z, Y);
        // gY of the pair, and gR_p = g . T_p per path straight into the transpose GEMM
        v4f gh[4];
#pragma unroll
        for (int j = 0; j < 4; ++j) gh[j] = v4f{0.f, 0.f, 0.f, 0.f};
        float gy[16];
        // (W2 read per tile through an opaque base, as in mace_tile_weights)
        int wbase = 0;
        asm volatile("" : "+v"(wbase));
        const float* sWt = sW + wbase;
        mace_grad_y(xs, g, Y, rr, gy, [&](auto pp, float gr) {
            constexpr int p = decltype(pp)::value;
            const float* a = sWt + ((p >> 2) * 16 + 4 * kk + (p & 3)) * kW2Row + e16;
#pragma unroll
            for (int j = 0; j < 4; ++j) gh[j] = mfma1(a[16 * j], gr, gh[j]);
        });
        // the next tile's operands and this tile's s, in flight during the reductions
        MaceTileIn nxt;
        const int64_t t1 = t0 + 16;
        mace_load_tile(u4, srcp, dstp, h, t1 < p1 ? min(t1 + e16, p1 - 1) : p1 - 1, kk, nxt);
        const float4* sr = reinterpret_cast<const float4*>(sg + pc * kHidden + 4 * kk);
        float4 sv[4];
#pragma unroll
        for (int j = 0; j < 4; ++j) sv[j] = sr[4 * j];
        // summed over the quad's channels (rows of the wave)
#pragma unroll
        for (int b = 0; b < 16; ++b) {
            gy[b] += __shfl_xor(gy[b], 16, 64);
            gy[b] += __shfl_xor(gy[b], 32, 64);
        }
        float gux, guy, guz;
        sh_backward<3>(cur.u.x, cur.u.y, cur.u.z, Y, gy, gux, guy, guz);
        // g_r: D[k][e] of the lane's k = 16 j + 4 (lane / 16) + r against s[e][k]
        float gr = 0.0f;
#pragma unroll
        for (int j = 0; j < 4; ++j) {
            gr = fmaf(gh[j][0], sv[j].x, gr);
            gr = fmaf(gh[j][1], sv[j].y, gr);
            gr = fmaf(gh[j][2], sv[j].z, gr);
            gr = fmaf(gh[j][3], sv[j].w, gr);
        }
        gr += __shfl_xor(gr, 16, 64);
        gr += __shfl_xor(gr, 32, 64);
        if (valid && kk == 0) {
            const float ux = cur.u.x, uy = cur.u.y, uz = cur.u.z, ir = 1.0f / cur.u.w;
            const float dot = ux * gux + uy * guy + uz * guz;
            float* o = gvq + pos * 3;
            o[0] = gr * ux + (gux - ux * dot) * ir;
            o[1] = gr * uy + (guy - uy * dot) * ir;
            o[2] = gr * uz + (guz - uz * dot) * ir;
        }
        cur = nxt;
    }
}

// ---------------------------------------------------------------------------
// Positions: deg[i] = degree of order[i] (then an exclusive scan gives pos0[i]),
// perm[pos0[i] + j] = row_ptr[order[i]] + j.  Writes past n_edges are dropped
// (order must be a permutation of the rows for the layer to be correct; a
// malformed one cannot make these kernels read or write out of bounds).
// ---------------------------------------------------------------------------
__global__ void mace_order_degrees_kernel(const int64_t* __restrict__ row_ptr,
                                          const int64_t* __restrict__ order, int64_t n,
                                          int64_t* __restrict__ deg) {
    const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (i >= n) return;
    int64_t d = order ? order[i] : i;
    d = d < 0 ? 0 : (d >= n ? n - 1 : d);
    deg[i] = row_ptr[d + 1] - row_ptr[d];
}

__global__ void mace_positions_kernel(const int64_t* __restrict__ row_ptr,
                                      const int64_t* __restrict__ order,
                                      const int64_t* __restrict__ pos0, int64_t n,
                                      int64_t n_edges, int64_t* __restrict__ perm) {
    const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (i >= n) return;
    int64_t d = order ? order[i] : i;
    d = d < 0 ? 0 : (d >= n ? n - 1 : d);
    const int64_t e0 = row_ptr[d], k = row_ptr[d + 1] - e0, p = pos0[i];
    for (int64_t j = 0; j < k && p + j < n_edges; ++j) perm[p + j] = e0 + j;
}

// wstart[w] = the first position of the first destination that starts at or after
// w * n_edges / n_workers (positions of whole destinations per worker), wstart[n_workers]
// = n_edges.
__global__ void mace_worker_starts_kernel(const int64_t* __restrict__ pos0, int64_t n,
                                          int64_t n_edges, int n_workers,
                                          int64_t* __restrict__ wstart) {
    const int w = blockIdx.x * blockDim.x + threadIdx.x;
    if (w > n_workers) return;
    if (w == n_workers) {
        wstart[w] = n_edges;
        return;
    }
    const int64_t target = n_edges * w / n_workers;
    int64_t lo = 0, hi = n;  // smallest i in [0, n] with pos0[i] >= target (pos0[n] = total)
    while (lo < hi) {
        const int64_t mid = (lo + hi) >> 1;
        if (pos0[mid] < target) lo = mid + 1;
        else hi = mid;
    }
    wstart[w] = min(pos0[lo], n_edges);
}

// Per position p (edge e = perm[p]): unit vector and length, source, destination,
// h = silu(B(r) W1 + b1); with sg, also s[k] = silu'(z_k) sum_b W1[b][k] dB_b/dr.
// Sixteen lanes per position: lane q evaluates Bessel function q % 8 (one sincos)
// and shares it with the position's other lanes, then forms hidden units
// 4q .. 4q + 3, so every store instruction writes whole 256-byte rows.
constexpr int kPrepPositions = 16;  // positions per 256-thread workgroup
__global__ __launch_bounds__(256) void mace_prep_kernel(
    const float* __restrict__ pos, MaceBox bx, const int64_t* __restrict__ src,
    const int64_t* __restrict__ dst, const int64_t* __restrict__ perm,
    const float* __restrict__ w1, const float* __restrict__ b1, float rc, int64_t n_edges,
    float4* __restrict__ u4, int* __restrict__ srcp, int* __restrict__ dstp,
    float* __restrict__ h, float* __restrict__ sg) {
    __shared__ float sW[kNBasis * kHidden + kHidden];
    for (int i = threadIdx.x; i < kNBasis * kHidden + kHidden; i += blockDim.x)
        sW[i] = i < kNBasis * kHidden ? w1[i] : b1[i - kNBasis * kHidden];
    __syncthreads();
    const int q = threadIdx.x & 15;
    int64_t p = (int64_t)blockIdx.x * kPrepPositions + (threadIdx.x >> 4);
    const bool valid = p < n_edges;
    p = valid ? p : n_edges - 1;  // every lane takes part in the shuffles below
    int64_t e = perm[p];
    e = e < 0 ? 0 : (e >= n_edges ? n_edges - 1 : e);
    const int64_t s = src[e], d = dst[e];
    float v[3];
    edge_vector(pos, s, d, bx.box, bx.inv, v);
    const float r = normalize3(v[0], v[1], v[2]);
    if (valid && q == 0) {
        u4[p] = make_float4(v[0], v[1], v[2], r);
        srcp[p] = (int)s;
        dstp[p] = (int)d;
    }
    // Bessel function k = q % 8 of this position, with the envelope
    const float dd = r / rc;
    float f = 0.f, df = 0.f;
    if (dd < 1.0f) {
        const float d5 = dd * dd * dd * dd * dd, d6 = d5 * dd;
        f = 1.0f - 28.0f * d6 + 48.0f * d6 * dd - 21.0f * d6 * dd * dd;
        const float om = 1.0f - dd;
        df = -168.0f * d5 * om * om / rc;
    }
    const float norm = sqrtf(2.0f / rc), ir = 1.0f / r;
    const float w = (float)((q & 7) + 1) * 3.14159265358979323846f / rc;
    float sn, cs;
    sincosf(w * r, &sn, &cs);
    const float gk = norm * sn * ir;
    const float bk = gk * f;
    const float dbk = sg ? (norm * (w * cs * ir - sn * ir * ir)) * f + gk * df : 0.0f;
    const int base = (threadIdx.x & 63) & ~15;
    float B[kNBasis], dB[kNBasis];
#pragma unroll
    for (int k = 0; k < kNBasis; ++k) B[k] = __shfl(bk, base + k, 64);
    if (sg) {
#pragma unroll
        for (int k = 0; k < kNBasis; ++k) dB[k] = __shfl(dbk, base + k, 64);
    }
    float z[4], sd[4];
#pragma unroll
    for (int t = 0; t < 4; ++t) {
        const int j = 4 * q + t;
        float acc = sW[kNBasis * kHidden + j];
#pragma unroll
        for (int k = 0; k < kNBasis; ++k) acc = fmaf(B[k], sW[k * kHidden + j], acc);
        const float sgm = sigmoidf(acc);
        z[t] = acc * sgm;
        if (sg) {
            float qq = 0.0f;
#pragma unroll
            for (int k = 0; k < kNBasis; ++k) qq = fmaf(sW[k * kHidden + j], dB[k], qq);
            sd[t] = sgm * (1.0f + acc * (1.0f - sgm)) * qq;
        }
    }
    if (valid) {
        reinterpret_cast<float4*>(h + p * kHidden)[q] = make_float4(z[0], z[1], z[2], z[3]);
        if (sg) reinterpret_cast<float4*>(sg + p * kHidden)[q] = make_float4(sd[0], sd[1], sd[2], sd[3]);
    }
}

// out rows of destinations without edges (the fused kernel writes the others)
__global__ void mace_zero_empty_rows_kernel(const int64_t* __restrict__ row_ptr, int64_t n,
                                            int C, float4* __restrict__ out) {
    const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    const int64_t per = (int64_t)C * 4;
    if (i >= n * per) return;
    const int64_t d = i / per;
    if (row_ptr[d + 1] == row_ptr[d]) out[i] = make_float4(0.f, 0.f, 0.f, 0.f);
}

// g_v[perm[p]] = sum over the channel quads, in order, of gv_part[quad][p]
__global__ void mace_gv_reduce_kernel(const float* __restrict__ gv_part,
                                      const int64_t* __restrict__ perm, int64_t n_edges,
                                      int n_quads, float* __restrict__ gv) {
    const int64_t p = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (p >= n_edges) return;
    float a = 0.f, b = 0.f, c = 0.f;
    for (int q = 0; q < n_quads; ++q) {
        const float* s = gv_part + ((int64_t)q * n_edges + p) * 3;
        a += s[0];
        b += s[1];
        c += s[2];
    }
    int64_t e = perm[p];
    e = e < 0 ? 0 : (e >= n_edges ? n_edges - 1 : e);
    gv[e * 3 + 0] = a;
    gv[e * 3 + 1] = b;
    gv[e * 3 + 2] = c;
}

__global__ void mace_fill_zero_kernel(float* __restrict__ p, int64_t count) {
    const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (i < count) p[i] = 0.0f;
}

__global__ void mace_zero_int_kernel(int* __restrict__ p) { *p = 0; }

// Workspace of one pass (per-position arrays; the backward adds s, the quads'
// gradient shares and the per-edge gradient).
struct MaceWs {
    int64_t *deg, *pos0, *perm, *wstart;
    float4* u4;
    int *srcp, *dstp;
    float *h, *sg, *gv_part, *gv;
    size_t bytes;
};

static size_t a256(size_t x) { return (x + 255) & ~size_t(255); }

static int mace_quads(int C) { return (int)ceil_div(C, 4); }

static MaceWs mace_ws(void* base, int64_t N, int64_t E, int C, bool backward) {
    char* p = static_cast<char*>(base);
    size_t o = 0;
    MaceWs w{};
    auto take = [&](size_t bytes) {
        void* r = p ? static_cast<void*>(p + o) : nullptr;
        o = a256(o + bytes);
        return r;
    };
    const size_t e = (size_t)std::max<int64_t>(E, 1);
    w.deg = static_cast<int64_t*>(take(sizeof(int64_t) * (size_t)std::max<int64_t>(N, 1)));
    w.pos0 = static_cast<int64_t*>(take(sizeof(int64_t) * (size_t)(N + 1)));
    w.perm = static_cast<int64_t*>(take(sizeof(int64_t) * e));
    w.wstart = static_cast<int64_t*>(take(sizeof(int64_t) * (kMaceMaxWorkers + 1)));
    w.u4 = static_cast<float4*>(take(sizeof(float4) * e));
    w.srcp = static_cast<int*>(take(sizeof(int) * e));
    w.dstp = static_cast<int*>(take(sizeof(int) * e));
    w.h = static_cast<float*>(take(sizeof(float) * kHidden * e));
    if (backward) {
        w.sg = static_cast<float*>(take(sizeof(float) * kHidden * e));
        w.gv_part = static_cast<float*>(take(sizeof(float) * 3 * e * (size_t)mace_quads(C)));
        w.gv = static_cast<float*>(take(sizeof(float) * 3 * e));
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

// Compute units of the current device.
static int mace_cu_count() {
    int dev = 0, n = 0;
    if (hipGetDevice(&dev) != hipSuccess ||
        hipDeviceGetAttribute(&n, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess || n <= 0)
        n = 256;
    return n;
}

// Launch shape of a fused kernel: every quad of a position range on one XCD, as
// many ranges per XCD as fill one round of resident workgroups (occupancy from the
// runtime for this kernel), so no second, partly idle round follows.
struct MaceShape {
    int n_quads, ranges_per_xcd, n_workers;
    unsigned grid;
};

template <typename K>
static int mace_shape(K kernel, int waves, int C, MaceShape* sh) {
    int occ = 0;
    if (hipOccupancyMaxActiveBlocksPerMultiprocessor(&occ, kernel, 64 * waves, 0) != hipSuccess ||
        occ < 1)
        occ = 1;
    const int per_xcd = std::max(1, mace_cu_count() / 8);
    sh->n_quads = mace_quads(C);
    sh->ranges_per_xcd = std::max(1, per_xcd * occ / sh->n_quads);
    sh->n_workers = 8 * sh->ranges_per_xcd * waves;
    if (sh->n_workers > kMaceMaxWorkers) return BM_ERR_ARG;
    sh->grid = (unsigned)(8 * sh->ranges_per_xcd * sh->n_quads);
    return BM_OK;
}

// Positions (destinations in `order`, each destination's edges ascending), the
// workers' ranges, and the per-position operands.
static int mace_prepare(const float* positions, const MaceBox& bx, const float* w1,
                        const float* b1, const int64_t* src, const int64_t* dst,
                        const int64_t* row_ptr, const int64_t* order, int64_t N, int64_t E,
                        float cutoff, const MaceShape& sh, const MaceWs& w, bool backward,
                        hipStream_t stream) {
    const unsigned nb = (unsigned)ceil_div(N, 256);
    mace_order_degrees_kernel<<<nb, 256, 0, stream>>>(row_ptr, order, N, w.deg);
    int rc = batteries_exclusive_scan_i64(w.deg, w.pos0, N, stream);
    if (rc != BM_OK) return rc;
    mace_positions_kernel<<<nb, 256, 0, stream>>>(row_ptr, order, w.pos0, N, E, w.perm);
    mace_worker_starts_kernel<<<(unsigned)ceil_div(sh.n_workers + 1, 256), 256, 0, stream>>>(
        w.pos0, N, E, sh.n_workers, w.wstart);
    mace_prep_kernel<<<(unsigned)ceil_div(E, kPrepPositions), 256, 0, stream>>>(
        positions, bx, src, dst, w.perm, w1, b1, cutoff, E, w.u4, w.srcp, w.dstp, w.h,
        backward ? w.sg : nullptr);
    return (int)hipGetLastError();
}

}  // namespace bmhip

using namespace bmhip;

extern "C" int batteries_gemm_f32(const float* A, const float* B, float* C, int64_t M, int N, int K,
                                  int trans_b, hipStream_t stream) {
    if (M < 0 || N < 0 || K < 0 || M > INT32_MAX) return BM_ERR_ARG;
    return gemm_launch(A, B, C, M, N, K, trans_b != 0, stream);
}

extern "C" size_t batteries_mace_workspace_bytes(int64_t N, int64_t N_edges, int C, int backward) {
    if (N < 0 || N_edges < 0 || C <= 0) return 0;
    return mace_ws(nullptr, N, N_edges, C, backward != 0).bytes;
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
    if (N > INT32_MAX || E > INT32_MAX) return false;  // int32 indices per position
    for (int k = 0; k < 3; ++k)
        if (!(box[k] > 0.0f)) return false;
    return true;
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
                                      const int64_t* order, float* out, int64_t N,
                                      int64_t N_edges, int C, float cutoff, void* workspace,
                                      size_t workspace_bytes, hipStream_t stream) {
    if (!mace_args_ok(box, N, N_edges, C, cutoff)) return BM_ERR_ARG;
    if (N == 0) return BM_OK;
    if ((reinterpret_cast<uintptr_t>(node_features) | reinterpret_cast<uintptr_t>(out)) & 15)
        return BM_ERR_ARG;
    const MaceWs w = mace_ws(workspace, N, N_edges, C, false);
    if (!workspace || workspace_bytes < w.bytes) return BM_ERR_WORKSPACE;
    const int64_t n4 = N * (int64_t)C * 4;
    mace_zero_empty_rows_kernel<<<(unsigned)ceil_div(n4, 256), 256, 0, stream>>>(
        row_ptr, N, C, reinterpret_cast<float4*>(out));
    if (N_edges == 0) return (int)hipGetLastError();
    MaceShape sh;
    int rc = mace_shape(mace_fused_forward_kernel, kMaceFwdWaves, C, &sh);
    if (rc != BM_OK) return rc;
    rc = mace_prepare(positions, mace_box(box), w1, b1, src, dst, row_ptr, order, N, N_edges,
                      cutoff, sh, w, false, stream);
    if (rc != BM_OK) return rc;
    mace_fused_forward_kernel<<<sh.grid, 64 * kMaceFwdWaves, 0, stream>>>(w.u4, w.srcp, w.dstp, w.h, w2,
                                                            node_features, w.wstart, out, C,
                                                            sh.n_quads, sh.ranges_per_xcd);
    return (int)hipGetLastError();
}

extern "C" int batteries_mace_backward(const float* positions, const float* box,
                                       const float* node_features, const float* w1,
                                       const float* b1, const float* w2, const int64_t* src,
                                       const int64_t* dst, const int64_t* row_ptr,
                                       const int64_t* order, const int64_t* rev,
                                       const float* grad_out, float* grad_pos, int64_t N,
                                       int64_t N_edges, int C, float cutoff, void* workspace,
                                       size_t workspace_bytes, hipStream_t stream) {
    if (!mace_args_ok(box, N, N_edges, C, cutoff)) return BM_ERR_ARG;
    if (N == 0) return BM_OK;
    if ((reinterpret_cast<uintptr_t>(node_features) | reinterpret_cast<uintptr_t>(grad_out)) & 15)
        return BM_ERR_ARG;
    const MaceWs w = mace_ws(workspace, N, N_edges, C, true);
    if (!workspace || workspace_bytes < w.bytes) return BM_ERR_WORKSPACE;
    if (N_edges == 0) {
        mace_fill_zero_kernel<<<(unsigned)ceil_div(N * 3, 256), 256, 0, stream>>>(grad_pos, N * 3);
        return (int)hipGetLastError();
    }
    MaceShape sh;
    int rc = mace_shape(mace_fused_backward_kernel, kMaceBwdWaves, C, &sh);
    if (rc != BM_OK) return rc;
    rc = mace_prepare(positions, mace_box(box), w1, b1, src, dst, row_ptr, order, N, N_edges,
                      cutoff, sh, w, true, stream);
    if (rc != BM_OK) return rc;
    mace_fused_backward_kernel<<<sh.grid, 64 * kMaceBwdWaves, 0, stream>>>(
        w.u4, w.srcp, w.dstp, w.h, w.sg, w2, node_features, grad_out, w.wstart, w.gv_part,
        N_edges, C, sh.n_quads, sh.ranges_per_xcd);
    mace_gv_reduce_kernel<<<(unsigned)ceil_div(N_edges, 256), 256, 0, stream>>>(
        w.gv_part, w.perm, N_edges, sh.n_quads, w.gv);
    mace_forces_kernel<<<(unsigned)ceil_div(N, 256), 256, 0, stream>>>(w.gv, row_ptr, rev, grad_pos,
                                                                        N);
    return (int)hipGetLastError();
}
