// 34-path L<=3 Clebsch-Gordan tensor products: simple and channel-weighted,
// forward and backward.
//
// Replaces reference src/tensor_product/tensor_product.cu:29-214 and
// src/tensor_product/tensor_product_backward.cu:32-1026.  The weight gradient
// is the exact adjoint of the forward (tensor_product_backward.cu:7-16), not
// the hand-written CG lines of :159-872.
#include "common.h"
#include "batmobile_hip.h"

#include <mutex>

namespace bmhip {

constexpr int kTpBlock = 256;
constexpr int kRowStride = 17;  // odd LDS stride for 16-float rows

// ---------------------------------------------------------------------------
// simple product: one thread per row, rows staged through LDS.  A block's rows
// are contiguous, so each thread issues its four 16-byte loads per input before
// any LDS write (item t + 256 k of the block: row item / 4, quad item % 4), and
// writes its results back as 16-byte stores of the same items.
// ---------------------------------------------------------------------------
__device__ __forceinline__ void load_rows16(const float* __restrict__ g, int64_t base, int rows,
                                            float4 (&v)[4]) {
    const float4* g4 = reinterpret_cast<const float4*>(g + base * 16);
    const int nq = rows * 4;
#pragma unroll
    for (int k = 0; k < 4; ++k) v[k] = g4[min((int)threadIdx.x + kTpBlock * k, nq - 1)];
}
__device__ __forceinline__ void put_rows16(float* s, int rows, const float4 (&v)[4]) {
    const int nq = rows * 4;
#pragma unroll
    for (int k = 0; k < 4; ++k) {
        const int i = threadIdx.x + kTpBlock * k;
        if (i < nq) {
            float* d = s + (i >> 2) * kRowStride + (i & 3) * 4;
            d[0] = v[k].x;
            d[1] = v[k].y;
            d[2] = v[k].z;
            d[3] = v[k].w;
        }
    }
}
__device__ __forceinline__ void store_rows16(const float* s, float* __restrict__ g, int64_t base,
                                             int rows) {
    float4* g4 = reinterpret_cast<float4*>(g + base * 16);
    const int nq = rows * 4;
#pragma unroll
    for (int k = 0; k < 4; ++k) {
        const int i = threadIdx.x + kTpBlock * k;
        if (i < nq) {
            const float* d = s + (i >> 2) * kRowStride + (i & 3) * 4;
            g4[i] = make_float4(d[0], d[1], d[2], d[3]);
        }
    }
}

// out = M(y) x with M[o][a] = sum_b c y[b] built row by row (611 + 256 VALU
// operations per row, against 2 x 611 for the term-by-term form)
__device__ __forceinline__ void tp_simple_rows(const float* x, const float* y, float* out) {
    static_for<16>([&](auto oo) {
        constexpr int O = decltype(oo)::value;
        float m[16];
        edge_operator_row<O>(y, m);
        float acc = m[0] * x[0];
#pragma unroll
        for (int a = 1; a < 16; ++a) acc = fmaf(m[a], x[a], acc);
        out[O] = acc;
    });
}

// Adjoint, row o of the operators at a time:
//   gx[a] = sum_o M[o][a] g[o],  M[o][a] = sum_b c y[b]
//   gy[b] = sum_o N[o][b] g[o],  N[o][b] = sum_a c x[a]
// (2 x (611 + 256) VALU operations per row, with 32 accumulators live)
__device__ __forceinline__ void tp_simple_backward_rows(const float* x, const float* y,
                                                        const float* g, float* gx, float* gy) {
#pragma unroll
    for (int k = 0; k < 16; ++k) {
        gx[k] = 0.0f;
        gy[k] = 0.0f;
    }
    static_for<16>([&](auto oo) {
        constexpr int O = decltype(oo)::value;
        float m[16], nb[16];
        edge_operator_row<O>(y, m);
#pragma unroll
        for (int b = 0; b < 16; ++b) nb[b] = 0.0f;
        static_for<kNumEntries>([&](auto kk) {
            constexpr CGEntry e = kCG[decltype(kk)::value];
            if constexpr (e.o == O) nb[e.b] = fmaf(e.c, x[e.a], nb[e.b]);
        });
#pragma unroll
        for (int k = 0; k < 16; ++k) {
            gx[k] = fmaf(m[k], g[O], gx[k]);
            gy[k] = fmaf(nb[k], g[O], gy[k]);
        }
    });
}

__global__ __launch_bounds__(kTpBlock) void tp_simple_kernel(const float* __restrict__ x,
                                                             const float* __restrict__ y,
                                                             float* __restrict__ out, int64_t n) {
    // one staging buffer, used in turn for x, y and the output (half the LDS of
    // separate buffers, so registers, not LDS, bound the waves per SIMD)
    __shared__ float sb[kTpBlock * kRowStride];
    const int64_t base = (int64_t)blockIdx.x * kTpBlock;
    const int rows = (int)min<int64_t>(kTpBlock, n - base);
    float4 vx[4], vy[4];
    load_rows16(x, base, rows, vx);
    load_rows16(y, base, rows, vy);
    const int t = threadIdx.x;
    float a[16], b[16], o[16];
    put_rows16(sb, rows, vx);
    __syncthreads();
#pragma unroll
    for (int k = 0; k < 16; ++k) a[k] = sb[t * kRowStride + k];
    __syncthreads();
    put_rows16(sb, rows, vy);
    __syncthreads();
#pragma unroll
    for (int k = 0; k < 16; ++k) b[k] = sb[t * kRowStride + k];
    if (t < rows) {
        tp_simple_rows(a, b, o);
#pragma unroll
        for (int k = 0; k < 16; ++k) sb[t * kRowStride + k] = o[k];  // own row: read above
    }
    __syncthreads();
    store_rows16(sb, out, base, rows);
}

// Small inputs (at most kTpDirectRows rows: one round of at most 256 workgroups): each
// lane its own rows straight from global memory, the next row's loads issued before
// this row's products, no LDS and no barriers.  With a single round there is no other
// workgroup to cover the LDS kernel's barriers: 3.7 us against 4.35 us at configs[0]
// (20,000 rows).  From about 10^5 rows up the coalesced LDS-staged kernel above is
// faster (31.7 us against 34.4 us at 10^6: lanes reading 64-byte rows 64 bytes apart
// use the memory pipeline less well).
constexpr int64_t kTpDirectRows = 65536;
__global__ __launch_bounds__(kTpBlock) void tp_simple_direct_kernel(const float* __restrict__ x,
                                                                    const float* __restrict__ y,
                                                                    float* __restrict__ out,
                                                                    int64_t n) {
    const int64_t stride = (int64_t)gridDim.x * kTpBlock;
    int64_t r = (int64_t)blockIdx.x * kTpBlock + threadIdx.x;
    if (r >= n) return;
    float4 ux[4], uy[4];
    auto ld = [&](int64_t row) {
        const float4* x4 = reinterpret_cast<const float4*>(x + row * 16);
        const float4* y4 = reinterpret_cast<const float4*>(y + row * 16);
#pragma unroll
        for (int k = 0; k < 4; ++k) {
            ux[k] = x4[k];
            uy[k] = y4[k];
        }
    };
    ld(r);
    for (; r < n; r += stride) {
        float a[16], b[16], o[16];
#pragma unroll
        for (int k = 0; k < 4; ++k) {
            a[4 * k] = ux[k].x;
            a[4 * k + 1] = ux[k].y;
            a[4 * k + 2] = ux[k].z;
            a[4 * k + 3] = ux[k].w;
            b[4 * k] = uy[k].x;
            b[4 * k + 1] = uy[k].y;
            b[4 * k + 2] = uy[k].z;
            b[4 * k + 3] = uy[k].w;
        }
        ld(r + stride < n ? r + stride : r);  // the last row re-reads itself (in bounds)
        tp_simple_rows(a, b, o);
        float4* o4 = reinterpret_cast<float4*>(out + r * 16);
#pragma unroll
        for (int k = 0; k < 4; ++k)
            o4[k] = make_float4(o[4 * k], o[4 * k + 1], o[4 * k + 2], o[4 * k + 3]);
    }
}

__global__ __launch_bounds__(kTpBlock) void tp_simple_backward_kernel(
    const float* __restrict__ x, const float* __restrict__ y, const float* __restrict__ g,
    float* __restrict__ gx, float* __restrict__ gy, int64_t n) {
    __shared__ float sx[kTpBlock * kRowStride];
    __shared__ float sy[kTpBlock * kRowStride];
    __shared__ float sg[kTpBlock * kRowStride];
    const int64_t base = (int64_t)blockIdx.x * kTpBlock;
    const int rows = (int)min<int64_t>(kTpBlock, n - base);
    float4 vx[4], vy[4], vg[4];
    load_rows16(x, base, rows, vx);
    load_rows16(y, base, rows, vy);
    load_rows16(g, base, rows, vg);
    put_rows16(sx, rows, vx);
    put_rows16(sy, rows, vy);
    put_rows16(sg, rows, vg);
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
        tp_simple_backward_rows(a, b, c, ga, gb);
#pragma unroll
        for (int k = 0; k < 16; ++k) {
            sx[t * kRowStride + k] = ga[k];
            sy[t * kRowStride + k] = gb[k];
        }
    }
    __syncthreads();
    store_rows16(sx, gx, base, rows);
    store_rows16(sy, gy, base, rows);
}

// ---------------------------------------------------------------------------
// Weighted product on MFMA.
//
//   T[n,ci,q]   = sum_{(a,b) in slot q} c * x[n,ci,a] * y[n,b]      156 slots q = (path, m_out)
//   out[n,co,o] = sum_{q: out(q) = o} sum_ci W[p(q),ci,co] T[n,ci,q]
//   h[n,ci,q]   = sum_co W[p(q),ci,co] g[n,co,out(q)]
//   gx[n,ci,a]  = sum_{q,b} c * y[n,b] * h[n,ci,q]
//   gy[n,b]     = sum_{ci,q,a} c * x[n,ci,a] * h[n,ci,q]
//   gW[p,ci,co] = sum_n sum_{q in p} T[n,ci,q] * g[n,co,out(q)]
//
// The three channel contractions (out, h, gW) are GEMMs per slot and run on
// v_mfma_f32_16x16x4f32 over 16-row tiles; the CG contractions (T, gx, gy) run
// on the VALU with compile-time coefficients.  Each kernel splits the slots
// into groups taken by different workgroups, so that a group's
// outputs are disjoint from the others':
//   forward:  output components o in [4G, 4G + 4)      (4 groups)
//   backward: paths with l1 in {0,1}, {2}, {3}          (3 groups; disjoint gx columns)
// K-dimension trick: a float4 read by lane group g = lane / 16 supplies k-steps
// s = 0..3, and A and B agree on which channel (or row) each (g, s) stands for.
// ---------------------------------------------------------------------------
constexpr int kTile = 16;  // rows per MFMA tile

constexpr bool fwd_path_in_group(int p, int G) {
    for (int m = 0; m < 2 * kPathL[p][2] + 1; ++m)
        if (fwd_in_group(kPathSlot[p] + m, G)) return true;
    return false;
}
constexpr int fwd_group_paths(int G) {
    int c = 0;
    for (int p = 0; p < kNumPaths; ++p) c += fwd_path_in_group(p, G) ? 1 : 0;
    return c;
}
constexpr int fwd_path_local(int p, int G) {
    int c = 0;
    for (int i = 0; i < p; ++i) c += fwd_path_in_group(i, G) ? 1 : 0;
    return c;
}
constexpr int fwd_path_at(int k, int G) {  // the k-th path of group G
    for (int p = 0; p < kNumPaths; ++p)
        if (fwd_path_in_group(p, G) && fwd_path_local(p, G) == k) return p;
    return -1;
}
constexpr int fwd_max_group() {
    int m = 0;
    for (int G = 0; G < kFwdGroups; ++G) m = fwd_group_size(G) > m ? fwd_group_size(G) : m;
    return m;
}
constexpr int kFwdMaxSlots = fwd_max_group();

constexpr int kBwdGroups = 3;
constexpr int kBwdL1First[kBwdGroups] = {0, 2, 3};
constexpr int kBwdL1Last[kBwdGroups] = {1, 2, 3};
constexpr bool bwd_path_in_group(int p, int G) {
    return kPathL[p][0] >= kBwdL1First[G] && kPathL[p][0] <= kBwdL1Last[G];
}
constexpr int bwd_a0(int G) { return kBwdL1First[G] * kBwdL1First[G]; }
constexpr int bwd_na(int G) { return (kBwdL1Last[G] + 1) * (kBwdL1Last[G] + 1) - bwd_a0(G); }
constexpr int bwd_group_size(int G) {
    int c = 0;
    for (int p = 0; p < kNumPaths; ++p) c += bwd_path_in_group(p, G) ? 2 * kPathL[p][2] + 1 : 0;
    return c;
}
constexpr int bwd_group_paths(int G) {
    int c = 0;
    for (int p = 0; p < kNumPaths; ++p) c += bwd_path_in_group(p, G) ? 1 : 0;
    return c;
}
// position of path p among the paths of group G, and of slot q among its slots
constexpr int bwd_path_local(int p, int G) {
    int c = 0;
    for (int i = 0; i < p; ++i) c += bwd_path_in_group(i, G) ? 1 : 0;
    return c;
}
constexpr int bwd_path_at(int k, int G) {  // the k-th path of group G
    for (int p = 0; p < kNumPaths; ++p)
        if (bwd_path_in_group(p, G) && bwd_path_local(p, G) == k) return p;
    return -1;
}
constexpr int bwd_slot_local(int q, int G) {
    int c = 0;
    for (int i = 0; i < q; ++i) c += bwd_path_in_group(kSlotPath[i], G) ? 1 : 0;
    return c;
}
constexpr int bwd_max_group() {
    int m = 0;
    for (int G = 0; G < kBwdGroups; ++G) m = bwd_group_size(G) > m ? bwd_group_size(G) : m;
    return m;
}
constexpr int kBwdMaxSlots = bwd_max_group();

// Out-of-range operands.  Every load reads a clamped, valid address and is
// issued unconditionally (a branch around a load costs a full wait right after
// it).  Where an out-of-range value could reach a stored result it is zeroed
// with mask0, an exact byte select (v_perm_b32) that the compiler does not turn
// back into a branch; elsewhere the tail is harmless by construction (it meets
// a zero operand, or lands in a discarded output row or column).
__device__ __forceinline__ float mask0(float v, bool ok) {
    return __uint_as_float(
        __builtin_amdgcn_perm(__float_as_uint(v), 0u, ok ? 0x07060504u : 0x0c0c0c0cu));
}

// 16 floats at p + off (off a multiple of 4 floats, a valid address)
__device__ __forceinline__ void load16(const float* __restrict__ p, int64_t off, float* v) {
    const float4* q = reinterpret_cast<const float4*>(p + off);
#pragma unroll
    for (int k = 0; k < 4; ++k) {
        const float4 t = q[k];
        v[4 * k + 0] = t.x;
        v[4 * k + 1] = t.y;
        v[4 * k + 2] = t.z;
        v[4 * k + 3] = t.w;
    }
}
// the same, zeroed when !ok
__device__ __forceinline__ void load16_mask(const float* __restrict__ p, int64_t off, bool ok,
                                            float* v) {
    load16(p, off, v);
#pragma unroll
    for (int k = 0; k < 16; ++k) v[k] = mask0(v[k], ok);
}

// ---- forward ---------------------------------------------------------------
// Workgroup: 16 rows x 64 output channels x one output group G, in H halves of
// 4 waves (H = 2 when C_in > 16): wave w of a half owns output channels
// co0 .. co0+15, and half h takes the 16-channel input chunks h, h + H, ...
// into its own LDS buffer.  Per chunk: thread (row, ci) builds the group's T
// values into LDS, then each wave runs
//   D[co][row] += W[p][ci][co] (A, global/L2) x T[row][ci][q] (B, LDS)
// for every slot q of the group, one accumulator per output component.  The
// halves' accumulators are added in LDS in a fixed order.  Two halves put two
// waves on each SIMD: one hides the other's load latency, and the pair issues
// VALU work at about twice the rate of a lone wave.
// LDS layout sT[slot][g][row][s] with ci = 4g + s: the B read of lane
// (row = lane % 16, g) is one float4, and a wave's T writes are contiguous.
template <int G>
__device__ __forceinline__ void fwd_group(const float* __restrict__ x, const float* __restrict__ w,
                                          float* __restrict__ out, int64_t n, int cin, int cout,
                                          float* sTall, const float* __restrict__ y, int tile) {
    constexpr int NS = fwd_group_size(G);
    const int tid = threadIdx.x & 255, lane = tid & 63, wv = tid >> 6;
    const int half = threadIdx.x >> 8, nhalf = blockDim.x >> 8;
    float* sT = sTall + half * (kFwdMaxSlots * 256);
    const int g4 = lane >> 4, i16 = lane & 15;
    const int64_t row0 = (int64_t)tile * kTile;
    const int co0 = (blockIdx.y * 4 + wv) * 16;
    const bool live = co0 < cout;
    const int trow = tid & 15, tcl = tid >> 4;
    // y of the T thread's row, straight from global memory (issued with the
    // first chunk's x and W loads; rows past n only reach discarded outputs)
    float yb[16];
    load16(y, min<int64_t>(row0 + trow, n - 1) * 16, yb);
    v4f acc[4];
#pragma unroll
    for (int j = 0; j < 4; ++j) acc[j] = v4f{0.f, 0.f, 0.f, 0.f};

    constexpr int NP = fwd_group_paths(G);
    const int co = co0 + i16;
    const int wpath_bytes = cin * cout * 4;
    const __amdgpu_buffer_rsrc_t wr = buffer_rsrc(w, (uint32_t)(kNumPaths * wpath_bytes));
    // every half runs the same number of chunks (a chunk past cin builds T = 0)
    const int nchunk = (cin + 16 * nhalf - 1) / (16 * nhalf);
    for (int ch = 0; ch < nchunk; ++ch) {
        const int c0 = (ch * nhalf + half) * 16;
        // A operands W[p][c0 + 4 g4 + s][co] of the group's paths through a
        // register ring of kWRing paths: the first ones are issued before the T
        // computation (their latency hides behind it), and each path's MFMAs
        // issue the load of the path kWRing ahead.
        // (ci >= cin meets T = 0; co >= cout lands in a discarded output row).
        // Buffer loads: lane offset in a VGPR, path offset p * cin * cout in an SGPR.
        int wo[4];
#pragma unroll
        for (int s = 0; s < 4; ++s) wo[s] = (min(c0 + 4 * g4 + s, cin - 1) * cout + min(co, cout - 1)) * 4;
        auto load_w = [&](int p) {
            const int so = p * wpath_bytes;
            return make_float4(buffer_ld(wr, wo[0], so), buffer_ld(wr, wo[1], so),
                               buffer_ld(wr, wo[2], so), buffer_ld(wr, wo[3], so));
        };
        constexpr int kWRing = 4;
        float4 wring[kWRing];
        static_for<(NP < kWRing ? NP : kWRing)>([&](auto kk) {
            constexpr int k = decltype(kk)::value;
            constexpr int pk = fwd_path_at(k, G);
            wring[k] = load_w(pk);
        });
        float t[NS];
        {
            const int ci = c0 + tcl;
            // y through an empty asm each chunk: the products c * y[b] are formed
            // here instead of being hoisted out of the chunk loop (and kept live)
            float yk[16];
#pragma unroll
            for (int b = 0; b < 16; ++b) yk[b] = yb[b];
            asm volatile("" : "+v"(yk[0]), "+v"(yk[1]), "+v"(yk[2]), "+v"(yk[3]), "+v"(yk[4]),
                              "+v"(yk[5]), "+v"(yk[6]), "+v"(yk[7]), "+v"(yk[8]), "+v"(yk[9]),
                              "+v"(yk[10]), "+v"(yk[11]), "+v"(yk[12]), "+v"(yk[13]),
                              "+v"(yk[14]), "+v"(yk[15]));
            float xa[16];
            // T must be 0 for ci >= cin (it meets nonzero W); rows >= n are discarded
            load16_mask(x, ((min<int64_t>(row0 + trow, n - 1)) * cin + min(ci, cin - 1)) * 16,
                        ci < cin, xa);
#pragma unroll
            for (int q = 0; q < NS; ++q) t[q] = 0.0f;
            static_for<kNumEntries>([&](auto kk) {
                constexpr CGEntry e = kCG[decltype(kk)::value];
                if constexpr (fwd_in_group(e.q, G)) {
                    constexpr int sl = fwd_local(e.q, G);
                    t[sl] = fmaf(e.c * yk[e.b], xa[e.a], t[sl]);
                }
            });
        }
        __syncthreads();  // the previous chunk's B reads are done
#pragma unroll
        for (int q = 0; q < NS; ++q) sT[q * 256 + (tcl >> 2) * 64 + trow * 4 + (tcl & 3)] = t[q];
        __syncthreads();
        if (live) {
            static_for<kNumPaths>([&](auto pp) {
                constexpr int p = decltype(pp)::value;
                if constexpr (fwd_path_in_group(p, G)) {
                    constexpr int k = fwd_path_local(p, G);
                    const float4 a4 = wring[k % kWRing];
                    if constexpr (k + kWRing < NP) {
                        constexpr int pn = fwd_path_at(k + kWRing, G);
                        wring[k % kWRing] = load_w(pn);
                    }
                    constexpr int lo = kPathL[p][2];
                    static_for<2 * lo + 1>([&](auto mm) {
                        constexpr int q = kPathSlot[p] + decltype(mm)::value;
                        if constexpr (fwd_in_group(q, G)) {
                            constexpr int sl = fwd_local(q, G);
                            constexpr int oj = kSlotOut[q] & 3;
                            const float4 b4 = *reinterpret_cast<const float4*>(
                                sT + sl * 256 + g4 * 64 + i16 * 4);
                            acc[oj] = mfma4(a4, b4, acc[oj]);
                        }
                    });
                }
            });
        }
    }
    if (nhalf == 2) {  // uniform: half 1 hands its sums to half 0
        __syncthreads();  // the last chunk's B reads are done
        float* sAcc = sTall;  // [wave][j][r][lane]
        if (half == 1) {
#pragma unroll
            for (int j = 0; j < 4; ++j)
#pragma unroll
                for (int r = 0; r < 4; ++r) sAcc[((wv * 4 + j) * 4 + r) * 64 + lane] = acc[j][r];
        }
        __syncthreads();
        if (half == 1) return;
#pragma unroll
        for (int j = 0; j < 4; ++j)
#pragma unroll
            for (int r = 0; r < 4; ++r) acc[j][r] += sAcc[((wv * 4 + j) * 4 + r) * 64 + lane];
    }
    // D[4 g4 + r][i16]: output channel co0 + 4 g4 + r of row row0 + i16
    const int64_t row = row0 + i16;
    if (live && row < n) {
#pragma unroll
        for (int r = 0; r < 4; ++r) {
            const int co = co0 + 4 * g4 + r;
            if (co < cout)
                *reinterpret_cast<float4*>(out + (row * cout + co) * 16 + 4 * G) =
                    make_float4(acc[0][r], acc[1][r], acc[2][r], acc[3][r]);
        }
    }
}

// Workgroup ids are dealt so that the four groups of a row tile run on one XCD
// (the hardware gives workgroup i to XCD i mod 8): each group writes one
// 16-byte piece of every 64-byte output row (co, o = 0..15) of the tile, and the
// four pieces then meet in that XCD's L2 instead of reaching memory as partial
// lines from four L2s (12.2 -> 10.7 us at configs[1]).
__global__ __launch_bounds__(2 * kTpBlock) void tp_weighted_fwd_mfma_kernel(
    const float* __restrict__ x, const float* __restrict__ y, const float* __restrict__ w,
    float* __restrict__ out, int64_t n, int cin, int cout, int ntile) {
    __shared__ __attribute__((aligned(16))) float sT[2 * kFwdMaxSlots * 256];
    const int id = blockIdx.x, xcd = id & 7, k = id >> 3;
    const int tile = (k >> 2) * 8 + xcd;
    if (tile >= ntile) return;  // uniform: the grid is rounded up to 8 tiles
    switch (k & 3) {
        case 0: fwd_group<0>(x, w, out, n, cin, cout, sT, y, tile); break;
        case 1: fwd_group<1>(x, w, out, n, cin, cout, sT, y, tile); break;
        case 2: fwd_group<2>(x, w, out, n, cin, cout, sT, y, tile); break;
        default: fwd_group<3>(x, w, out, n, cin, cout, sT, y, tile); break;
    }
}

// ---- backward: grad_x and grad_y ---------------------------------------------
// Workgroup: 16 rows; its waves take (l1 group G, input-channel tile) units
// u = wave, wave + nwave, ... with G = u % 3, tile = u / 3.  The grad_output
// tile of the 16 rows is staged once in LDS as sG[o][co/4][row][co%4] (plane
// stride PS): lane (row, g) reads g[row][cb + 4g .. +3][o] as one float4.
// Per path p of the group:
//   D[ci][row] = h_p[row][ci][m_out] = sum_co W[p][ci][co] (A) g[row][co][o] (B)
// lands in lane (row = lane % 16, ci = 4 g + r), which then applies the CG
// entries of p to its own 4 channels: the group's gx columns, and a grad_y
// partial in gyp.  The partials are summed over lanes and waves in a fixed order.
template <int G, int KCO>
__device__ __forceinline__ void bwd_xy_unit(const float* __restrict__ x, float* yb,
                                            const __amdgpu_buffer_rsrc_t wr, float* __restrict__ gx,
                                            int64_t n, int cin, int cout, int ct, const float* sG,
                                            float* gyp, int64_t row0) {
    constexpr int PS = KCO * 16 + 4;
    constexpr int A0 = bwd_a0(G), NA = bwd_na(G);
    const int lane = threadIdx.x & 63;
    const int g4 = lane >> 4, i16 = lane & 15;
    const int64_t row = row0 + i16;
    const bool row_ok = row < n;
    const int64_t row_c = row_ok ? row : n - 1;  // clamped row for unconditional loads
    const int wpath_bytes = cin * cout * 4;
    const int ci0 = ct * 16;
    float xa[4][NA], gxa[4][NA];
#pragma unroll
    for (int r = 0; r < 4; ++r) {
        const int ci = ci0 + 4 * g4 + r;
        const float* xr = x + (row_c * cin + min(ci, cin - 1)) * 16 + A0;
#pragma unroll
        for (int a = 0; a < NA; ++a) {
            xa[r][a] = mask0(xr[a], ci < cin);  // meets h rows of channels >= cin
            gxa[r][a] = 0.0f;
        }
    }
    // A operands W[p][ciA][cb + 4 g4 + s] of one path, all KCO/16 channel chunks,
    // through buffer loads (lane offset in a VGPR, path offset p * cin * cout in
    // an SGPR).  Clamped addresses: channels >= cin give h rows that meet x = 0 or
    // are discarded, co >= cout meets the zero-padded g tile.  The next path's
    // operands are loaded while this path's MFMAs and CG contraction run.
    const int ciA = ci0 + i16;
    const int wrow = min(ciA, cin - 1) * cout;
    constexpr int NCB = KCO / 16;
    // With cout % 4 == 0 a lane's 4 channels cb*16 + 4 g4 + (0..3) are either all
    // below cout or all at or above it (then clamped to the last 4, which meet zero
    // g rows): one 16-byte load per chunk instead of four.
    const bool w_vec = (cout & 3) == 0;  // uniform
    auto load_w = [&](int p, float4* dst) {
        const int so = p * wpath_bytes;
        if (w_vec) {
#pragma unroll
            for (int cb = 0; cb < NCB; ++cb)
                dst[cb] = buffer_ld4(wr, (wrow + min(cb * 16 + 4 * g4, cout - 4)) * 4, so);
        } else {
#pragma unroll
            for (int cb = 0; cb < NCB; ++cb) {
                float a[4];
#pragma unroll
                for (int s = 0; s < 4; ++s)
                    a[s] = buffer_ld(wr, (wrow + min(cb * 16 + 4 * g4 + s, cout - 1)) * 4, so);
                dst[cb] = make_float4(a[0], a[1], a[2], a[3]);
            }
        }
    };
    // One path per iteration of a loop that is not unrolled: each path is a basic
    // block of its own, so instruction selection cannot hoist every path's MFMAs
    // ahead of the CG contractions (which would keep all of the group's h
    // accumulators live at once).
    constexpr int NPG = bwd_group_paths(G);
    constexpr bool PF = KCO <= 64;  // next-path prefetch (registers allow it up to 64 channels)
    // two operand buffers used in turn (path kc reads wbuf[kc & 1] and fills the
    // other one), so no per-path register copies
    float4 wbuf[2][NCB];
    constexpr int p0 = bwd_path_at(0, G);
    load_w(p0, wbuf[0]);
#pragma clang loop unroll(disable)
    for (int k = 0; k < NPG; ++k) {
        // y through an empty asm each iteration, in place: the products c * y[b]
        // are then formed per path instead of being hoisted out of the loop (some
        // 200 loop-invariant values that would not fit in registers)
        float* yk = yb;
        asm volatile("" : "+v"(yk[0]), "+v"(yk[1]), "+v"(yk[2]), "+v"(yk[3]), "+v"(yk[4]),
                          "+v"(yk[5]), "+v"(yk[6]), "+v"(yk[7]), "+v"(yk[8]), "+v"(yk[9]),
                          "+v"(yk[10]), "+v"(yk[11]), "+v"(yk[12]), "+v"(yk[13]),
                          "+v"(yk[14]), "+v"(yk[15]));
        static_for<NPG>([&](auto kk) {
            constexpr int kc = decltype(kk)::value;
            if (k == kc) {
                constexpr int p = bwd_path_at(kc, G);
                float4* wcur = wbuf[PF ? (kc & 1) : 0];
                if constexpr (!PF && kc > 0) load_w(p, wcur);
                if constexpr (PF && kc + 1 < NPG) {
                    constexpr int pn = bwd_path_at(kc + 1, G);
                    load_w(pn, wbuf[(kc + 1) & 1]);
                }
                constexpr int lo = kPathL[p][2];
                constexpr int NM = 2 * lo + 1;
                v4f h[NM];
                // B operands of output component m (all chunks) are read from LDS
                // while the MFMAs of component m - 1 run.  Chunks past cout meet
                // the zero-padded g tile (no per-chunk branches).
                float4 bq[2][NCB];
                auto read_b = [&](int m, float4* dst) {
#pragma unroll
                    for (int cb = 0; cb < NCB; ++cb)
                        dst[cb] = *reinterpret_cast<const float4*>(
                            sG + (lo * lo + m) * PS + (cb * 4 + g4) * 64 + i16 * 4);
                };
                read_b(0, bq[0]);
                static_for<NM>([&](auto mm) {
                    constexpr int m = decltype(mm)::value;
                    if constexpr (m + 1 < NM) read_b(m + 1, bq[(m + 1) & 1]);
                    // chunk 0 starts from a zero accumulator operand (no register zeroing)
                    h[m] = mfma4(wcur[0], bq[m & 1][0], v4f{0.f, 0.f, 0.f, 0.f});
#pragma unroll
                    for (int cb = 1; cb < NCB; ++cb) h[m] = mfma4(wcur[cb], bq[m & 1][cb], h[m]);
                    __builtin_amdgcn_sched_barrier(0);  // one component's reads ahead, no more
                });
                static_for<kPathEntry[p + 1] - kPathEntry[p]>([&](auto ee) {
                    constexpr CGEntry e = kCG[kPathEntry[p] + decltype(ee)::value];
                    constexpr int m = e.o - lo * lo;
                    constexpr int ai = e.a - A0;
                    const float cy = e.c * yk[e.b];
                    float sacc = 0.0f;
#pragma unroll
                    for (int r = 0; r < 4; ++r) {
                        gxa[r][ai] = fmaf(cy, h[m][r], gxa[r][ai]);
                        sacc = fmaf(xa[r][ai], h[m][r], sacc);
                    }
                    gyp[e.b] = fmaf(e.c, sacc, gyp[e.b]);
                });
            }
        });
    }
    if (gx && row_ok) {
#pragma unroll
        for (int r = 0; r < 4; ++r) {
            const int ci = ci0 + 4 * g4 + r;
            if (ci < cin)
#pragma unroll
                for (int a = 0; a < NA; ++a) gx[(row * cin + ci) * 16 + A0 + a] = gxa[r][a];
        }
    }
}

// Up to RT row tiles per workgroup.  One tile: up to 8 waves share the
// 3 * (C_in / 16) (path group, channel tile) units of one 16-row tile.  Two
// tiles (RT = 2, C_in / 16 even): 8 waves, 4 per row tile, each wave on one
// tile; the unit order of the second tile is mirrored so that waves w and w + 4
// (one SIMD when waves are placed round-robin) carry the same number of units
// between them.  At C_in = 32 that is 6 units per tile and 3 per SIMD, where
// one tile leaves SIMDs with 2, 2, 1, 1.  Workgroups below npair take two
// tiles, the rest one (rows from 32 npair on): single-tile workgroups fill the
// last, partial round of the grid in about 2/3 of the time of a pair.
template <int KCO, int RT>
__global__ __launch_bounds__(512) void tp_weighted_bwd_xy_mfma_kernel(
    const float* __restrict__ x, const float* __restrict__ y, const float* __restrict__ w,
    const float* __restrict__ g, float* __restrict__ gx, float* __restrict__ gy, int64_t n,
    int cin, int cout, int64_t npair) {
    constexpr int PS = KCO * 16 + 4;
    constexpr int TS = kTile * PS;  // floats of one row tile's g planes
    __shared__ __attribute__((aligned(16))) float sG[RT * TS];
    const int tid = threadIdx.x, lane = tid & 63, wv = tid >> 6;
    const int nwave = blockDim.x >> 6;
    const int g4 = lane >> 4, i16 = lane & 15;
    const bool pair = RT == 2 && (int64_t)blockIdx.x < npair;  // uniform
    const int rtn = pair ? 2 : 1;                               // row tiles of this workgroup
    const int64_t row0 = pair ? (int64_t)blockIdx.x * (2 * kTile)
                              : npair * (2 * kTile) + ((int64_t)blockIdx.x - npair) * kTile;
    const int cout16 = KCO;  // every MFMA chunk of the tile is staged
    // stage g[row0 .. row0 + 16 rtn - 1][co][o] (zeros past n and past cout).
    // Eight float4 loads per thread are in flight before their LDS writes: the
    // loads are unconditional (clamped addresses, masked values), since a
    // conditional load is a branch with a full wait behind it.
    {
        const int total = rtn * kTile * cout16 * 4;
        constexpr int kStage = 8;
        for (int i0 = tid; i0 < total; i0 += kStage * (int)blockDim.x) {
            float4 v[kStage];
#pragma unroll
            for (int k = 0; k < kStage; ++k) {
                const int i = min(i0 + k * (int)blockDim.x, total - 1);
                const int rr = i / (cout16 * 4), rem = i - rr * cout16 * 4;
                const int co = rem >> 2, j = rem & 3;
                const bool ok = row0 + rr < n && co < cout;
                const float4 t = *reinterpret_cast<const float4*>(
                    g + (min<int64_t>(row0 + rr, n - 1) * cout + min(co, cout - 1)) * 16 + 4 * j);
                v[k] = make_float4(mask0(t.x, ok), mask0(t.y, ok), mask0(t.z, ok), mask0(t.w, ok));
            }
#pragma unroll
            for (int k = 0; k < kStage; ++k) {
                const int i = i0 + k * (int)blockDim.x;
                if (i < total) {
                    const int rr = i / (cout16 * 4), rem = i - rr * cout16 * 4;
                    const int co = rem >> 2, j = rem & 3;
                    float* d = sG + (rr / kTile) * TS + (co >> 2) * 64 + (rr % kTile) * 4 + (co & 3);
                    d[(4 * j + 0) * PS] = v[k].x;
                    d[(4 * j + 1) * PS] = v[k].y;
                    d[(4 * j + 2) * PS] = v[k].z;
                    d[(4 * j + 3) * PS] = v[k].w;
                }
            }
        }
    }
    __syncthreads();
    float gyp[16];
#pragma unroll
    for (int k = 0; k < 16; ++k) gyp[k] = 0.0f;
    const int wpath_bytes = cin * cout * 4;
    const __amdgpu_buffer_rsrc_t wr = buffer_rsrc(w, (uint32_t)(kNumPaths * wpath_bytes));
    const int units = kBwdGroups * ((cin + 15) / 16);  // per row tile
    const int wpt = nwave / rtn;                        // waves per row tile
    const int rt = wv / wpt;
    const int lw = (rt & 1) ? wpt - 1 - (wv - rt * wpt) : wv - rt * wpt;
    const int64_t rbase = row0 + rt * kTile;
    const float* sGt = sG + rt * TS;
    float yb[16];
    load16(y, min<int64_t>(rbase + i16, n - 1) * 16, yb);  // rows >= n reach discarded outputs
    for (int u = lw; u < units; u += wpt) {
        const int ct = u / kBwdGroups;
        switch (u % kBwdGroups) {
            case 0: bwd_xy_unit<0, KCO>(x, yb, wr, gx, n, cin, cout, ct, sGt, gyp, rbase); break;
            case 1: bwd_xy_unit<1, KCO>(x, yb, wr, gx, n, cin, cout, ct, sGt, gyp, rbase); break;
            default: bwd_xy_unit<2, KCO>(x, yb, wr, gx, n, cin, cout, ct, sGt, gyp, rbase); break;
        }
    }
    if (!gy) return;   // uniform over the workgroup
    __syncthreads();   // sG is reused for the reduction
    float* sRed = sG;  // [wave][g][row][16]; waves of tile t are t * wpt .. t * wpt + wpt - 1
#pragma unroll
    for (int k = 0; k < 16; ++k) sRed[((wv * 4 + g4) * 16 + i16) * 16 + k] = gyp[k];
    __syncthreads();
    for (int i = tid; i < rtn * kTile * 16; i += blockDim.x) {
        const int t = i / (kTile * 16), rr = (i >> 4) % kTile, k = i & 15;
        float sum = 0.0f;
        for (int v = t * wpt; v < t * wpt + wpt; ++v)
#pragma unroll
            for (int gg = 0; gg < 4; ++gg) sum += sRed[((v * 4 + gg) * 16 + rr) * 16 + k];
        const int64_t row = row0 + t * kTile + rr;
        if (row < n) gy[row * 16 + k] = sum;
    }
}

// ---- backward: grad_W partials over row segments ----------------------------
// Workgroup: one row segment x 16 input channels x one l1 group x 64 output
// channels (wave w: co0 .. co0+15).  Per 16-row chunk: thread t builds T for
// (row 4 (t % 4) + t / 64, ci (t / 4) % 16) into sT[slot][g][ci][r] (row = 4 r + g),
// lane (co, g) holds g[row 4 r + g][co][0..15] in registers, and
//   D[ci][co] += T[row][ci][q] (A, LDS float4 over r) x g[row][co][out(q)] (B)
// with k = (m_out, r) for every path of the group; one accumulator per path.
template <int G>
__device__ __forceinline__ void bwd_w_group(const float* __restrict__ x, const float* __restrict__ y,
                                            const float* __restrict__ g, float* __restrict__ part,
                                            int64_t n, int cin, int cout, int64_t rows_per_seg,
                                            float* sT, float* sY) {
    constexpr int NS = bwd_group_size(G);
    constexpr int NP = bwd_group_paths(G);
    const int tid = threadIdx.x, lane = tid & 63, wv = tid >> 6;
    const int g4 = lane >> 4, i16 = lane & 15;
    const int64_t seg = blockIdx.x;
    const int ci0 = blockIdx.y * 16;
    const int co0 = ((blockIdx.z / kBwdGroups) * 4 + wv) * 16;
    const bool live = co0 < cout;
    const int64_t r0 = seg * rows_per_seg;
    const int64_t r1 = min<int64_t>(n, r0 + rows_per_seg);
    // T thread mapping
    const int t_r = tid & 3, t_ci = ci0 + ((tid >> 2) & 15), t_g = tid >> 6;
    const int t_row = 4 * t_r + t_g;
    v4f acc[NP];
#pragma unroll
    for (int j = 0; j < NP; ++j) acc[j] = v4f{0.f, 0.f, 0.f, 0.f};

    for (int64_t rc = r0; rc < r1; rc += kTile) {
        __syncthreads();  // the previous chunk's reads of sT and sY are done
        {
            const int rr = tid >> 4, k = tid & 15;
            sY[tid] = y[min<int64_t>(rc + rr, n - 1) * 16 + k];
        }
        // B operands of this chunk, issued before the T computation hides their latency
        float gv[4][16];
        {
            const int co = co0 + i16;
#pragma unroll
            for (int r = 0; r < 4; ++r) {
                // rows past the segment meet T = 0 (below); co >= cout is a discarded column
                const int64_t rw = rc + 4 * r + g4;
                load16(g, (min<int64_t>(rw, n - 1) * cout + min(co, cout - 1)) * 16, gv[r]);
            }
        }
        __syncthreads();
        {
            float xa[16], yb[16], t[NS];
            // rows past the segment must not count: their T is zero (x masked: 16 selects
            // per thread, against 64 for masking the thread's g values); channels >= cin
            // are discarded rows
            load16_mask(x, (min<int64_t>(rc + t_row, n - 1) * cin + min(t_ci, cin - 1)) * 16,
                        rc + t_row < r1, xa);
#pragma unroll
            for (int k = 0; k < 16; ++k) yb[k] = sY[t_row * 16 + k];
#pragma unroll
            for (int q = 0; q < NS; ++q) t[q] = 0.0f;
            static_for<kNumEntries>([&](auto kk) {
                constexpr CGEntry e = kCG[decltype(kk)::value];
                if constexpr (bwd_path_in_group(e.p, G)) {
                    constexpr int sl = bwd_slot_local(e.q, G);
                    t[sl] = fmaf(e.c * yb[e.b], xa[e.a], t[sl]);
                }
            });
#pragma unroll
            for (int q = 0; q < NS; ++q) sT[q * 256 + tid] = t[q];
        }
        __syncthreads();
        // Unconditional, also in waves whose channels are all past cout (their
        // results are not stored): under a branch, the compiler sinks the g loads
        // above into it, right in front of their first use.
        static_for<kNumPaths>([&](auto pp) {
            constexpr int p = decltype(pp)::value;
            if constexpr (bwd_path_in_group(p, G)) {
                constexpr int lo = kPathL[p][2];
                constexpr int pl = bwd_path_local(p, G);
                static_for<2 * lo + 1>([&](auto mm) {
                    constexpr int m = decltype(mm)::value;
                    constexpr int sl = bwd_slot_local(kPathSlot[p] + m, G);
                    const float4 a4 =
                        *reinterpret_cast<const float4*>(sT + sl * 256 + g4 * 64 + i16 * 4);
                    const float4 b4 = make_float4(gv[0][lo * lo + m], gv[1][lo * lo + m],
                                                  gv[2][lo * lo + m], gv[3][lo * lo + m]);
                    acc[pl] = mfma4(a4, b4, acc[pl]);
                });
            }
        });
    }
    // D[4 g4 + r][i16]: input channel ci0 + 4 g4 + r, output channel co0 + i16
    if (live) {
        const int co = co0 + i16;
        static_for<kNumPaths>([&](auto pp) {
            constexpr int p = decltype(pp)::value;
            if constexpr (bwd_path_in_group(p, G)) {
                constexpr int pl = bwd_path_local(p, G);
#pragma unroll
                for (int r = 0; r < 4; ++r) {
                    const int ci = ci0 + 4 * g4 + r;
                    if (ci < cin && co < cout)
                        part[((seg * kNumPaths + p) * cin + ci) * cout + co] = acc[pl][r];
                }
            }
        });
    }
}

__global__ __launch_bounds__(kTpBlock) void tp_weighted_bwd_w_mfma_kernel(
    const float* __restrict__ x, const float* __restrict__ y, const float* __restrict__ g,
    float* __restrict__ part, int64_t n, int cin, int cout, int64_t rows_per_seg) {
    __shared__ __attribute__((aligned(16))) float sT[kBwdMaxSlots * 256];
    __shared__ float sY[kTile * 16];
    switch (blockIdx.z % kBwdGroups) {
        case 0: bwd_w_group<0>(x, y, g, part, n, cin, cout, rows_per_seg, sT, sY); break;
        case 1: bwd_w_group<1>(x, y, g, part, n, cin, cout, rows_per_seg, sT, sY); break;
        default: bwd_w_group<2>(x, y, g, part, n, cin, cout, rows_per_seg, sT, sY); break;
    }
}

// grad_x and grad_y for C_out above the LDS tile of the MFMA kernel (128):
// h[n,ci,q] = sum_co W[path(q),ci,co] g[n,co,out(q)], gx = CG^T(h, y),
// gy = sum_ci CG^T(h, x).  One thread per (row, ci); the per-ci gy partials are
// reduced in a fixed order.
// STAGE_G: the rows' g is staged in LDS (kBRows rows per workgroup) beside every
// (row, ci) partial of gy.  Otherwise (C_out or C_in too large for that) one row
// per workgroup reads g from memory, where the row's C_out x 64 bytes stay in
// cache for the workgroup's threads; thread t sums the partials of its channels
// t, t + 256, ... in registers, and the 256 sums meet in LDS (16 KB whatever
// C_in is), so neither C_in nor C_out is bounded.
constexpr int kBRows = 2;
template <bool STAGE_G>
__global__ __launch_bounds__(kTpBlock) void tp_weighted_backward_xy_kernel(
    const float* __restrict__ x, const float* __restrict__ y, const float* __restrict__ w,
    const float* __restrict__ g, float* __restrict__ gx, float* __restrict__ gy, int64_t n, int cin,
    int cout) {
    constexpr int kRows = STAGE_G ? kBRows : 1;
    extern __shared__ float smem[];
    // gy partials: [kRows][cin][16] when STAGE_G, else [kTpBlock][16]
    const int npart = STAGE_G ? kRows * cin : kTpBlock;
    float* sgy = smem;
    float* sy = sgy + npart * 16;              // [kRows][16]
    float* sg = sy + kRows * 16;               // [kRows][cout][16] when STAGE_G
    const int64_t row0 = (int64_t)blockIdx.x * kRows;
    const int rows = (int)min<int64_t>(kRows, n - row0);
    const int tid = threadIdx.x;
    if constexpr (STAGE_G)
        for (int i = tid; i < rows * cout * 16; i += kTpBlock) sg[i] = g[row0 * cout * 16 + i];
    for (int i = tid; i < rows * 16; i += kTpBlock) sy[i] = y[row0 * 16 + i];
    __syncthreads();
    float gyacc[16];
#pragma unroll
    for (int k = 0; k < 16; ++k) gyacc[k] = 0.0f;
    for (int it = tid; it < rows * cin; it += kTpBlock) {
        const int r = it / cin, ci = it - r * cin;
        float h[kNumSlots];
#pragma unroll
        for (int q = 0; q < kNumSlots; ++q) h[q] = 0.0f;
        const float* wci = w + (int64_t)ci * cout;
        const float* gr = STAGE_G ? sg + r * cout * 16 : g + (row0 + r) * cout * 16;
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
        if constexpr (STAGE_G) {
#pragma unroll
            for (int k = 0; k < 16; ++k) sgy[(r * cin + ci) * 16 + k] = gb[k];
        } else {
#pragma unroll
            for (int k = 0; k < 16; ++k) gyacc[k] += gb[k];
        }
    }
    if constexpr (!STAGE_G) {
#pragma unroll
        for (int k = 0; k < 16; ++k) sgy[tid * 16 + k] = gyacc[k];
    }
    __syncthreads();
    if (!gy) return;
    if constexpr (STAGE_G) {
        for (int i = tid; i < rows * 16; i += kTpBlock) {
            const int r = i >> 4, k = i & 15;
            float s = 0.0f;
            for (int ci = 0; ci < cin; ++ci) s += sgy[(r * cin + ci) * 16 + k];
            gy[(row0 + r) * 16 + k] = s;
        }
    } else {
        // 16 groups of 16 partials per component, then the 16 group sums, in order
        const int k = tid & 15, grp = tid >> 4;
        float s = 0.0f;
#pragma unroll
        for (int j = 0; j < 16; ++j) s += sgy[(grp * 16 + j) * 16 + k];
        __syncthreads();
        sgy[grp * 16 + k] = s;
        __syncthreads();
        if (tid < 16) {
            float t = 0.0f;
#pragma unroll
            for (int j = 0; j < 16; ++j) t += sgy[j * 16 + tid];
            gy[row0 * 16 + tid] = t;
        }
    }
}

// gW[i] = sum_s part[s, i] in ascending s (deterministic).  Eight segments'
// loads are issued before their adds, which keep the ascending order.
__global__ __launch_bounds__(kTpBlock) void reduce_segments_kernel(const float* __restrict__ part,
                                                                   float* __restrict__ out,
                                                                   int64_t count, int nseg) {
    const int64_t i = (int64_t)blockIdx.x * kTpBlock + threadIdx.x;
    if (i >= count) return;
    float s = 0.0f;
    int k = 0;
    for (; k + 8 <= nseg; k += 8) {
        float v[8];
#pragma unroll
        for (int j = 0; j < 8; ++j) v[j] = part[(int64_t)(k + j) * count + i];
#pragma unroll
        for (int j = 0; j < 8; ++j) s += v[j];
    }
    for (; k < nseg; ++k) s += part[(int64_t)k * count + i];
    out[i] = s;
}

__global__ void fill_zero_kernel(float* __restrict__ p, int64_t count) {
    const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (i < count) p[i] = 0.0f;
}

// Two-tile workgroups of the grad_x / grad_y kernel (one per CU at a time):
// whole rounds of them (kBwdXyRound, MI355X's 256 CUs), and single-tile
// workgroups for the rest of the tiles when those fill at most half a round of
// pairs (each takes about 2/3 of a pair's time, so one round of singles ends
// before half a round of pairs would); otherwise pairs throughout.  A function
// of the tile count only, so results do not depend on the device.
constexpr int64_t kBwdXyRound = 256;
static int64_t bwd_xy_pairs(int64_t tiles) {
    const int64_t full = tiles / (2 * kBwdXyRound) * kBwdXyRound;
    const int64_t rest = tiles - 2 * full;  // tiles past the whole rounds of pairs
    if (rest <= kBwdXyRound) return full;   // one round of single-tile workgroups
    return ceil_div(tiles, 2);
}

// Row segments of the grad_W reduction: a fixed function of (N, C_in, C_out),
// not of the device, so results are the same on every GPU.  The grid
// (segments x input-channel tiles x output-channel blocks x 3 groups) is sized
// to about kGwTargetWorkgroups, one full round of the kernel's workgroups on
// MI355X (256 CUs x 2 resident workgroups), so no second, mostly idle round
// follows; segments hold whole 16-row chunks and none is empty.
constexpr int64_t kGwTargetWorkgroups = 512;
constexpr int64_t kGwMaxSegments = 256;
static int64_t gw_combos(int cin, int cout) {
    return ceil_div(cin, 16) * ceil_div(cout, 64) * kBwdGroups;
}
static int64_t gw_rows_per_seg(int64_t n, int cin, int cout) {
    const int64_t chunks = std::max<int64_t>(1, ceil_div(n, kTile));
    const int64_t want = std::min<int64_t>(
        kGwMaxSegments, std::max<int64_t>(1, kGwTargetWorkgroups / gw_combos(cin, cout)));
    return ceil_div(chunks, std::min(want, chunks)) * kTile;
}
static int64_t gw_segments(int64_t n, int cin, int cout) {
    return ceil_div(std::max<int64_t>(1, ceil_div(n, kTile)) * kTile, gw_rows_per_seg(n, cin, cout));
}

}  // namespace bmhip

using namespace bmhip;

extern "C" int batteries_get_num_paths_l3(void) { return kNumPaths; }

extern "C" void batteries_get_path_info_l3(int* path_info) {
    for (int p = 0; p < kNumPaths; ++p)
        for (int k = 0; k < 3; ++k) path_info[p * 3 + k] = kPathL[p][k];
}

static bool aligned16(const void* p) { return (reinterpret_cast<uintptr_t>(p) & 15) == 0; }

extern "C" int batteries_tensor_product_simple_l3(const float* input1, const float* input2,
                                                  float* output, int64_t N, hipStream_t stream) {
    if (N < 0) return BM_ERR_ARG;
    if (N == 0) return BM_OK;
    if (!aligned16(input1) || !aligned16(input2) || !aligned16(output)) return BM_ERR_ARG;
    if (N <= kTpDirectRows)
        tp_simple_direct_kernel<<<(unsigned)ceil_div(N, kTpBlock), kTpBlock, 0, stream>>>(
            input1, input2, output, N);
    else
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
    if (!aligned16(input1) || !aligned16(input2) || !aligned16(grad_output) ||
        !aligned16(grad_input1) || !aligned16(grad_input2))
        return BM_ERR_ARG;
    tp_simple_backward_kernel<<<(unsigned)ceil_div(N, kTpBlock), kTpBlock, 0, stream>>>(
        input1, input2, grad_output, grad_input1, grad_input2, N);
    return (int)hipGetLastError();
}

// Rows per launch of the weighted forward: keeps grid.x * blockDim.x (at most
// 512 work-items per 16-row tile and group) below 2^32 - 1, the dispatch limit;
// larger N runs as consecutive launches over row ranges.
constexpr int64_t kFwdMaxRowsPerLaunch = int64_t(1) << 24;

extern "C" int batteries_tensor_product_l3(const float* input1, const float* input2,
                                           const float* weights, float* output, int64_t N,
                                           int C_in, int C_out, hipStream_t stream) {
    if (N < 0 || C_in <= 0 || C_out <= 0) return BM_ERR_ARG;
    if (N == 0) return BM_OK;
    if (ceil_div(C_out, 64) > 65535) return BM_ERR_ARG;
    if ((int64_t)kNumPaths * C_in * C_out * 4 > INT32_MAX) return BM_ERR_ARG;  // W via 32-bit offsets
    if ((reinterpret_cast<uintptr_t>(input1) | reinterpret_cast<uintptr_t>(output)) & 15)
        return BM_ERR_ARG;
    const int halves = C_in > 16 ? 2 : 1;  // input-channel chunks split over two wave halves
    for (int64_t r0 = 0; r0 < N; r0 += kFwdMaxRowsPerLaunch) {
        const int64_t rows = std::min(kFwdMaxRowsPerLaunch, N - r0);
        const int64_t ntile = ceil_div(rows, kTile);
        // (row tile, group) pairs: tiles rounded up to 8, four groups each
        dim3 grid((unsigned)(ceil_div(ntile, 8) * 8 * kFwdGroups), (unsigned)ceil_div(C_out, 64), 1);
        tp_weighted_fwd_mfma_kernel<<<grid, halves * kTpBlock, 0, stream>>>(
            input1 + r0 * C_in * 16, input2 + r0 * 16, weights, output + r0 * C_out * 16, rows,
            C_in, C_out, (int)ntile);
        const hipError_t e = hipGetLastError();
        if (e != hipSuccess) return (int)e;
    }
    return BM_OK;
}

// Workspace of the weighted backward: grad_W partials of the row segments
// [S][34][C_in][C_out] (grad_input1 / grad_input2 alone need none).
extern "C" size_t batteries_tensor_product_backward_workspace_bytes(int64_t N, int C_in,
                                                                    int C_out) {
    if (N <= 0 || C_in <= 0 || C_out <= 0) return 0;
    return (size_t)gw_segments(N, C_in, C_out) * kNumPaths * (size_t)C_in * (size_t)C_out *
           sizeof(float);
}

// The weighted backward on a given workspace (gw_part: the grad_W partials, at least
// batteries_tensor_product_backward_workspace_bytes when grad_weights is computed).
static int tp_backward_run(const float* input1, const float* input2, const float* weights,
                           const float* grad_output, float* grad_input1, float* grad_input2,
                           float* grad_weights, int64_t N, int C_in, int C_out, float* gw_part,
                           hipStream_t stream) {
    if (grad_input1 || grad_input2) {
        if (C_out <= 128 && (int64_t)kNumPaths * C_in * C_out * 4 <= INT32_MAX) {
            // one wave per (path group, 16-channel tile), at most 8 per workgroup;
            // two row tiles on 8 waves when that spreads the units evenly over the SIMDs
            const int nct = (int)ceil_div(C_in, 16);
            const int units = kBwdGroups * nct;
            const int64_t tiles = ceil_div(N, kTile);
            if (C_out <= 64 && nct % 2 == 0 && tiles >= 2) {
                const int64_t npair = bwd_xy_pairs(tiles);
                const int64_t nsingle = tiles - 2 * npair;  // may be -1: a last half-empty pair
                tp_weighted_bwd_xy_mfma_kernel<64, 2>
                    <<<(unsigned)(npair + std::max<int64_t>(nsingle, 0)), 512, 0, stream>>>(
                        input1, input2, weights, grad_output, grad_input1, grad_input2, N, C_in,
                        C_out, npair);
            } else {
                const int nwave = std::min(units, 8);
                const unsigned grid = (unsigned)tiles;
                if (C_out <= 64)
                    tp_weighted_bwd_xy_mfma_kernel<64, 1><<<grid, 64 * nwave, 0, stream>>>(
                        input1, input2, weights, grad_output, grad_input1, grad_input2, N, C_in,
                        C_out, 0);
                else
                    tp_weighted_bwd_xy_mfma_kernel<128, 1><<<grid, 64 * nwave, 0, stream>>>(
                        input1, input2, weights, grad_output, grad_input1, grad_input2, N, C_in,
                        C_out, 0);
            }
            hipError_t e = hipGetLastError();
            if (e != hipSuccess) return (int)e;
        } else {
            // g staged in LDS while two rows of it fit in 64 KB beside the gy partials;
            // above that one row per workgroup with g read from memory (no bound on C_out)
            const size_t staged = sizeof(float) * ((size_t)kBRows * C_out * 16 +
                                                   (size_t)kBRows * C_in * 16 + kBRows * 16);
            const size_t unstaged = sizeof(float) * ((size_t)kTpBlock * 16 + 16);
            if (staged <= 64 * 1024) {
                tp_weighted_backward_xy_kernel<true>
                    <<<(unsigned)ceil_div(N, kBRows), kTpBlock, staged, stream>>>(
                        input1, input2, weights, grad_output, grad_input1, grad_input2, N, C_in,
                        C_out);
            } else {
                if (N > UINT32_MAX) return BM_ERR_ARG;  // one row per workgroup
                tp_weighted_backward_xy_kernel<false><<<(unsigned)N, kTpBlock, unstaged, stream>>>(
                    input1, input2, weights, grad_output, grad_input1, grad_input2, N, C_in, C_out);
            }
            hipError_t e = hipGetLastError();
            if (e != hipSuccess) return (int)e;
        }
    }
    if (grad_weights) {
        const int64_t segs = gw_segments(N, C_in, C_out);
        const int64_t rps = gw_rows_per_seg(N, C_in, C_out);
        if (ceil_div(C_in, 16) > 65535 || ceil_div(C_out, 64) * kBwdGroups > 65535) return BM_ERR_ARG;
        dim3 grid((unsigned)segs, (unsigned)ceil_div(C_in, 16),
                  (unsigned)(ceil_div(C_out, 64) * kBwdGroups));
        tp_weighted_bwd_w_mfma_kernel<<<grid, kTpBlock, 0, stream>>>(input1, input2, grad_output,
                                                                     gw_part, N, C_in, C_out, rps);
        hipError_t e = hipGetLastError();
        if (e != hipSuccess) return (int)e;
        const int64_t count = (int64_t)kNumPaths * C_in * C_out;
        reduce_segments_kernel<<<(unsigned)ceil_div(count, kTpBlock), kTpBlock, 0, stream>>>(
            gw_part, grad_weights, count, (int)segs);
        e = hipGetLastError();
        if (e != hipSuccess) return (int)e;
    }
    return BM_OK;
}

// Argument checks shared by both entry points; N = 0 fills grad_weights with zeros.
// Returns 1 when the call is complete (nothing more to launch).
static int tp_backward_check(const float* input1, const float* grad_output, float* grad_weights,
                             int64_t N, int C_in, int C_out, hipStream_t stream) {
    if (N < 0 || C_in <= 0 || C_out <= 0) return BM_ERR_ARG;
    if (N == 0) {
        if (grad_weights) {
            const int64_t count = (int64_t)kNumPaths * C_in * C_out;
            fill_zero_kernel<<<(unsigned)ceil_div(count, kTpBlock), kTpBlock, 0, stream>>>(
                grad_weights, count);
            const hipError_t e = hipGetLastError();
            return e != hipSuccess ? (int)e : 1;
        }
        return 1;
    }
    if (ceil_div(N, kTile) > INT32_MAX) return BM_ERR_ARG;
    if ((reinterpret_cast<uintptr_t>(input1) | reinterpret_cast<uintptr_t>(grad_output)) & 15)
        return BM_ERR_ARG;
    return BM_OK;
}

extern "C" int batteries_tensor_product_backward_l3(
    const float* input1, const float* input2, const float* weights, const float* grad_output,
    float* grad_input1, float* grad_input2, float* grad_weights, int64_t N, int C_in, int C_out,
    void* workspace, size_t workspace_bytes, hipStream_t stream) {
    const int rc = tp_backward_check(input1, grad_output, grad_weights, N, C_in, C_out, stream);
    if (rc != BM_OK) return rc == 1 ? BM_OK : rc;
    const size_t need = batteries_tensor_product_backward_workspace_bytes(N, C_in, C_out);
    if (grad_weights && (!workspace || workspace_bytes < need)) return BM_ERR_WORKSPACE;
    return tp_backward_run(input1, input2, weights, grad_output, grad_input1, grad_input2,
                           grad_weights, N, C_in, C_out, static_cast<float*>(workspace), stream);
}

// ---------------------------------------------------------------------------
// The same backward without any allocation: the grad_W partials live in
// `scratch`, a file-scope device array of BATMOBILE_HIP_NOALLOC_SCRATCH_BYTES that
// each GPU holds (its own copy) from the library's load until the process ends.
// In host code `scratch` names a host-side stand-in, not device memory: the
// device address comes from hipGetSymbolAddress, resolved once per device (with
// that device current) on the first call there and kept in scratch_dev[].  Every
// call on one GPU shares that GPU's array; each call writes every partial it
// reads, so nothing needs clearing, and calls that overlap on one GPU race.
// ---------------------------------------------------------------------------
static __device__ __align__(256) float scratch[BATMOBILE_HIP_NOALLOC_SCRATCH_BYTES / sizeof(float)];

namespace {
constexpr int kMaxDevices = 64;
std::mutex scratch_mu;
void* scratch_dev[kMaxDevices];

int scratch_address(float** out) {
    int dev = -1;
    hipError_t e = hipGetDevice(&dev);
    if (e != hipSuccess) return (int)e;
    if (dev < 0 || dev >= kMaxDevices) return BM_ERR_ARG;
    std::lock_guard<std::mutex> lock(scratch_mu);
    if (!scratch_dev[dev]) {
        void* p = nullptr;
        e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
        if (e != hipSuccess) return (int)e;
        if (!p) return (int)hipErrorInvalidSymbol;
        scratch_dev[dev] = p;
    }
    *out = static_cast<float*>(scratch_dev[dev]);
    return BM_OK;
}
}  // namespace

extern "C" int batteries_tensor_product_backward_l3_noalloc(
    const float* input1, const float* input2, const float* weights, const float* grad_output,
    float* grad_input1, float* grad_input2, float* grad_weights, int64_t N, int C_in, int C_out,
    hipStream_t stream) {
    // size limit first: a rejected call touches no device state
    if (N > 0 && C_in > 0 && C_out > 0 && grad_weights &&
        batteries_tensor_product_backward_workspace_bytes(N, C_in, C_out) >
            (size_t)BATMOBILE_HIP_NOALLOC_SCRATCH_BYTES)
        return BATMOBILE_HIP_ERR_SCRATCH;
    const int rc = tp_backward_check(input1, grad_output, grad_weights, N, C_in, C_out, stream);
    if (rc != BM_OK) return rc == 1 ? BM_OK : rc;
    float* part = nullptr;
    if (grad_weights) {
        const int e = scratch_address(&part);
        if (e != BM_OK) return e;
    }
    return tp_backward_run(input1, input2, weights, grad_output, grad_input1, grad_input2,
                           grad_weights, N, C_in, C_out, part, stream);
}
