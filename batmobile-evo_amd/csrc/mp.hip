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
#include "mp_schedule.h"

namespace bmhip {

constexpr int kMpBlock = 256;
constexpr int kBatch = 64;        // edges per LDS batch
constexpr int kMStride = 260;     // floats per edge operator in LDS (256 + pad)
constexpr int kChanGroup = 64;    // channels per workgroup (4 waves x 16)
constexpr int kPrefetch = 16;     // source-row gathers in flight per lane
constexpr int kMaxRowsPerBlock = 64;    // destinations per workgroup (row_ptr slice in LDS)

// Operator rows sit in LDS with their four 16-byte column quads permuted by
// quad_swizzle(o): the phase-2 read of one edge (lane (o, g) reads quad g of
// row o) then covers all 32 banks in every group of 8 lanes.
__host__ __device__ constexpr int quad_swizzle(int o) { return (o >> 1) & 3; }

// Rows of M built by each wave in phase 1, chosen so that the four waves
// carry nearly equal numbers of CG terms (168, 169, 168, 170 terms + writes;
// rows in order of o would give 150, 189, 174, 162).
constexpr int kRowsOfWave[4][4] = {{0, 1, 3, 5}, {2, 4, 6, 11}, {7, 9, 10, 14}, {8, 12, 13, 15}};

// Phase 1: lane j of wave w builds rows kRowsOfWave[w] of M for edge j of the batch.
template <int W>
__device__ __forceinline__ void build_rows(const float* Y, float* sMj) {
    static_for<4>([&](auto rr) {
        constexpr int o = kRowsOfWave[W][decltype(rr)::value];
        constexpr int sw = quad_swizzle(o);
        float m[16];
        edge_operator_row<o>(Y, m);
        float4* dst = reinterpret_cast<float4*>(sMj + o * 16);
        dst[0 ^ sw] = make_float4(m[0], m[1], m[2], m[3]);
        dst[1 ^ sw] = make_float4(m[4], m[5], m[6], m[7]);
        dst[2 ^ sw] = make_float4(m[8], m[9], m[10], m[11]);
        dst[3 ^ sw] = make_float4(m[12], m[13], m[14], m[15]);
    });
}

// The scatter kernel's phase 1: wave 0 also computes the next batch's Y (into LDS, for
// all four waves), so it builds fewer rows.  Rows per wave (-1: none) chosen so that the
// waves' VALU work comes out nearly equal: Y (about 45 instructions) + 126 CG terms,
// 164, 162 and 159 terms, against 45 + 152-154 terms in every wave when each computes Y.
constexpr int kRowsOfWaveSh[4][5] = {
    {7, 9, 13, -1, -1}, {5, 8, 10, 14, -1}, {1, 2, 3, 4, -1}, {0, 6, 11, 12, 15}};

template <int W>
__device__ __forceinline__ void build_rows_sh(const float* Y, float* sMj) {
    static_for<5>([&](auto rr) {
        constexpr int o = kRowsOfWaveSh[W][decltype(rr)::value];
        if constexpr (o >= 0) {
            constexpr int sw = quad_swizzle(o);
            float m[16];
            edge_operator_row<o>(Y, m);
            float4* dst = reinterpret_cast<float4*>(sMj + o * 16);
            dst[0 ^ sw] = make_float4(m[0], m[1], m[2], m[3]);
            dst[1 ^ sw] = make_float4(m[4], m[5], m[6], m[7]);
            dst[2 ^ sw] = make_float4(m[8], m[9], m[10], m[11]);
            dst[3 ^ sw] = make_float4(m[12], m[13], m[14], m[15]);
        }
    });
}

// One edge of a batch as seen by the lane that owns it in phase 1.
struct EdgeRec {
    float x, y, z;
    int src;  // source row (node counts are < 2^31)
};

__device__ __forceinline__ EdgeRec load_edge(const float* __restrict__ vec,
                                             const int64_t* __restrict__ perm,
                                             const int64_t* __restrict__ src_idx, int64_t k,
                                             int64_t e1) {
    EdgeRec r{0.f, 0.f, 0.f, 0};
    if (k < e1) {
        const int64_t e = perm ? perm[k] : k;
        r.x = vec[e * 3 + 0];
        r.y = vec[e * 3 + 1];
        r.z = vec[e * 3 + 2];
        r.src = (int)src_idx[e];
    }
    return r;
}

// Y (L = 3) of one edge record, normalised first when NORM.
template <bool NORM>
__device__ __forceinline__ void edge_sh(EdgeRec r, float* Y) {
    float x = r.x, y = r.y, z = r.z;
    if constexpr (NORM) {
        // v / max(|v|, 1e-10) with one reciprocal square root (about 1 ulp)
        const float inv = __builtin_amdgcn_rsqf(fmaxf(x * x + y * y + z * z, 1e-20f));
        x *= inv;
        y *= inv;
        z *= inv;
    }
    sh_forward_l3(x, y, z, Y);
}

// Wave w's four operator rows of one edge, from its Y, into sMj.
__device__ __forceinline__ void edge_rows(const float* Y, float* sMj, int w) {
    switch (w) {
        case 0: build_rows<0>(Y, sMj); break;
        case 1: build_rows<1>(Y, sMj); break;
        case 2: build_rows<2>(Y, sMj); break;
        default: build_rows<3>(Y, sMj); break;
    }
}

// Phase 1 of a batch: lane j < nb of wave w builds rows 4w..4w+3 of the
// operator of its edge into sM (no global memory access: the edge was loaded
// into registers during the previous batch).
template <bool NORM>
__device__ __forceinline__ void phase1_build(EdgeRec r, int nb, float* sM) {
    const int lane = threadIdx.x & 63;
    const int w = threadIdx.x >> 6;
    if (lane < nb) {
        float Y[16];
        edge_sh<NORM>(r, Y);
        edge_rows(Y, sM + lane * kMStride, w);
    }
}

// Gather of one lane's float4 of source row `src` at byte offset `voff` inside
// the row.  BUF: raw buffer load with the row offset in a scalar register (X
// below 4 GiB); otherwise a 64-bit global load.

template <bool BUF>
__device__ __forceinline__ float4 gather(const float* __restrict__ X, __amdgpu_buffer_rsrc_t rsrc,
                                         int voff, int src, uint32_t row_bytes) {
    if constexpr (BUF) {
        typedef int v4i __attribute__((ext_vector_type(4)));
        const v4i r = __builtin_amdgcn_raw_buffer_load_b128(rsrc, voff, (int)((uint32_t)src * row_bytes), 0);
        return make_float4(__int_as_float(r.x), __int_as_float(r.y), __int_as_float(r.z),
                           __int_as_float(r.w));
    } else {
        return *reinterpret_cast<const float4*>(reinterpret_cast<const char*>(X) +
                                                (int64_t)src * row_bytes + voff);
    }
}

// Is k the first edge of one of the rows described by sRow[0..n] (k < sRow[n])?
__device__ __forceinline__ bool row_starts_at(const int64_t* sRow, int n, int64_t k) {
    int lo = 0, hi = n;  // first index with sRow[idx] >= k
    while (lo < hi) {
        const int mid = (lo + hi) >> 1;
        if (sRow[mid] < k) lo = mid + 1;
        else hi = mid;
    }
    return lo < n && sRow[lo] == k;
}

// Is k1 the end (exclusive) of one of the rows described by sRow[0..n]?
__device__ __forceinline__ bool row_ends_at(const int64_t* sRow, int n, int64_t k1) {
    int lo = 0, hi = n + 1;  // first index with sRow[idx] >= k1
    while (lo < hi) {
        const int mid = (lo + hi) >> 1;
        if (sRow[mid] < k1) lo = mid + 1;
        else hi = mid;
    }
    return lo <= n && sRow[lo] == k1;
}

// SCATTER: out[d, c, :] = sum over the CSR row of d, for the items_per_block
// (scheduled) rows of this workgroup.  MESSAGES: out[e, c, :] per edge, for the
// items_per_block (a multiple of kBatch) edges of this workgroup.
//
// Phase 2 walks the batch edge by edge with wave-uniform control only:
//   - the operator fragment of edge j+1 is read from LDS while edge j's four
//     MFMAs run;
//   - source rows come through a register ring of kPrefetch float4 per lane:
//     slot u holds the edge at distance u (mod kPrefetch) from the batch start,
//     and loads for the next batch's first edges are issued in this batch, so
//     kPrefetch gathers stay in flight across batch boundaries;
//   - row ends inside the batch are a 64-bit mask (ballot in phase 1): the
//     per-edge test is one scalar bit test; flushing is the rare path.
template <bool SCATTER, bool NORM, bool BUF>
__global__ __launch_bounds__(kMpBlock) void mp_simple_mfma_kernel(
    const float* __restrict__ vec, const float* __restrict__ X, const int64_t* __restrict__ src_idx,
    const int64_t* __restrict__ perm, const int64_t* __restrict__ row_ptr,
    const int64_t* __restrict__ row_dst, float* __restrict__ out, int64_t n_items,
    int64_t n_edges, int C, int items_per_block, int n_logical, uint32_t x_bytes) {
    static_assert(kBatch % kPrefetch == 0, "batch must be a multiple of the prefetch depth");
    static_assert(kBatch == 64, "one edge per lane in phase 1");
    __shared__ __attribute__((aligned(16))) float sM[kBatch * kMStride];
    __shared__ int64_t sRow[kMaxRowsPerBlock + 1];
    __shared__ int64_t sDst[kMaxRowsPerBlock];

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
    const uint32_t row_bytes = (uint32_t)C * 64u;
    // lanes past the last channel read a valid channel; their output column is never stored
    const int voff = (c < C ? c : C - 1) * 64 + g * 16;
    const __amdgpu_buffer_rsrc_t xr = __builtin_amdgcn_make_buffer_rsrc(
        const_cast<float*>(X), (short)0, BUF ? (int)x_bytes : 0, kBufferDword3);

    int64_t e0, e1, d0 = 0, d1 = 0;
    int nrows = 0;
    if constexpr (SCATTER) {
        d0 = (int64_t)logical * items_per_block;
        d1 = min<int64_t>(n_items, d0 + items_per_block);
        nrows = (int)(d1 - d0);
        for (int i = threadIdx.x; i <= nrows; i += kMpBlock) {
            sRow[i] = row_ptr[d0 + i];
            if (i < nrows) sDst[i] = row_dst ? row_dst[d0 + i] : d0 + i;
        }
        __syncthreads();
        e0 = sRow[0];
        e1 = sRow[nrows];
    } else {
        e0 = (int64_t)logical * items_per_block;
        e1 = min<int64_t>(n_edges, e0 + items_per_block);
    }

    const v4f zero4 = {0.f, 0.f, 0.f, 0.f};
    v4f acc = zero4;
    int d_cur = 0;  // current row, relative to d0

    auto store_v = [&](int64_t orow, const v4f& v) {
        if (c < C && orow >= 0)
            *reinterpret_cast<float4*>(out + (orow * C + c) * 16 + 4 * g) =
                make_float4(v[0], v[1], v[2], v[3]);
    };
    // zeros for the empty rows starting at d_cur
    auto skip_empty = [&]() {
        while (d_cur < nrows && sRow[d_cur + 1] == sRow[d_cur]) {
            store_v(sDst[d_cur], zero4);
            ++d_cur;
        }
    };
    if constexpr (SCATTER) {
        if (tile_live) skip_empty();
    }
    // One edge: four MFMAs into the row accumulator (started from zero on the
    // first edge of a row, so the accumulator is never written outside MFMAs),
    // then the row's store when the edge ends it.
    auto edge = [&](int j, int64_t kb, const float4& m, const float4& xv, uint64_t starts,
                    uint64_t ends) {
        if constexpr (SCATTER) {
            if ((starts >> j) & 1ull) acc = mfma4(m, xv, zero4);
            else acc = mfma4(m, xv, acc);
            if ((ends >> j) & 1ull) {
                store_v(sDst[d_cur], acc);
                ++d_cur;
                skip_empty();
            }
        } else {
            store_v(kb + j, mfma4(m, xv, zero4));
        }
    };

    EdgeRec cur = load_edge(vec, perm, src_idx, e0 + lane, e1);
    float4 ring[kPrefetch];
    bool first = true;
    for (int64_t kb = e0; kb < e1; kb += kBatch) {
        const int nb = (int)min<int64_t>(kBatch, e1 - kb);
        const int lim = (int)min<int64_t>(e1 - kb, 4 * kBatch);  // prefetch bound, batch-relative
        __syncthreads();
        phase1_build<NORM>(cur, nb, sM);
        uint64_t starts = 0, ends = 0;
        if constexpr (SCATTER) {
            starts = __ballot(lane < nb && row_starts_at(sRow, nrows, kb + lane));
            ends = __ballot(lane < nb && row_ends_at(sRow, nrows, kb + lane + 1));
        }
        __syncthreads();
        // the next batch's edges, in flight during this batch's phase 2
        const EdgeRec nxt = load_edge(vec, perm, src_idx, kb + kBatch + lane, e1);
        if (tile_live) {
            if (first) {
#pragma unroll
                for (int u = 0; u < kPrefetch; ++u)
                    if (u < nb)
                        ring[u] = gather<BUF>(X, xr, voff, __builtin_amdgcn_readlane(cur.src, u),
                                              row_bytes);
                first = false;
            }
            const float* mrow = sM + i16 * 16 + 4 * (g ^ quad_swizzle(i16));
            float4 mr[2];
            mr[0] = *reinterpret_cast<const float4*>(mrow);
            if (lim >= kBatch + kPrefetch) {
                // full batch whose prefetch targets all exist: fully unrolled, no checks
                static_for<kBatch>([&](auto jj) {
                    constexpr int j = decltype(jj)::value;
                    constexpr int u = j % kPrefetch;
                    if constexpr (j + 1 < kBatch)
                        mr[(j + 1) & 1] = *reinterpret_cast<const float4*>(mrow + (j + 1) * kMStride);
                    edge(j, kb, mr[j & 1], ring[u], starts, ends);
                    constexpr int jn = j + kPrefetch;
                    const int s = jn < kBatch ? __builtin_amdgcn_readlane(cur.src, jn)
                                              : __builtin_amdgcn_readlane(nxt.src, jn - kBatch);
                    ring[u] = gather<BUF>(X, xr, voff, s, row_bytes);
                });
            } else {
                for (int jj = 0; jj < nb; jj += kPrefetch) {
#pragma unroll
                    for (int u = 0; u < kPrefetch; ++u) {
                        const int j = jj + u;
                        if (j < nb) {
                            if (j + 1 < nb)
                                mr[(u + 1) & 1] =
                                    *reinterpret_cast<const float4*>(mrow + (j + 1) * kMStride);
                            edge(j, kb, mr[u & 1], ring[u], starts, ends);
                            const int jn = j + kPrefetch;
                            if (jn < lim) {
                                const int s = jn < nb ? __builtin_amdgcn_readlane(cur.src, jn)
                                                      : __builtin_amdgcn_readlane(nxt.src, jn - nb);
                                ring[u] = gather<BUF>(X, xr, voff, s, row_bytes);
                            }
                        }
                    }
                }
            }
        }
        cur = nxt;
    }
    if constexpr (SCATTER) {
        if (tile_live)
            while (d_cur < nrows) {
                store_v(sDst[d_cur], zero4);
                ++d_cur;
            }
    }
}

// ---------------------------------------------------------------------------
// Scatter kernel: out[d, c, :] = sum over the CSR row of d, for the
// rows_per_block (<= kScatterRows, scheduled) rows of this workgroup.
//
// Same operator/MFMA scheme as above, in batches of 64 edges so that phase 1
// (Y and four operator rows per wave) runs on every lane: on gfx950 VALU work
// does not overlap the MFMAs of its SIMD, so each phase-1 instruction costs its
// full issue time, and a 32-edge batch would leave half of the lanes idle.
//
// On gfx9 loads and stores share one counter, and with a store pending the
// compiler treats the counter as out of order and drains every outstanding
// gather at the next use; a gather issued under a data-dependent condition has
// the same effect.  Hence the edge loop has neither:
//   - every batch is kSBatch edges fully unrolled, and every edge issues the
//     gather for the edge kRing positions ahead (past the block's last edge it
//     gathers row 0 of the same tensor, a valid address whose value is never
//     used: edges past the end only touch the accumulator after the block's
//     last row has been written or staged);
//   - a row that closes is written where it closes, straight from the MFMA
//     accumulator, by a store the compiler does not see (store_row_acc): the
//     gathers' waits stay exact, because loads complete in order and a store
//     only ever adds to the count (a wait for a gather with a store in flight
//     can only last longer, never end before the gather is in);
//   - the last batch issues no gathers for a next batch.
// The per-edge control is one scalar bit test: `ends` (a 64-bit mask per batch,
// built with scalar arithmetic from the row ends) marks the edges that close a
// row; there the accumulator is written and reset to zero.
// ---------------------------------------------------------------------------
constexpr int kSBatch = 64;       // edges per batch (operators in LDS, one edge per lane in phase 1)
constexpr int kRing = 32;         // gathers in flight per lane (edges ahead)
constexpr int kLdsAhead = 3;      // operator rows read from LDS this many edges ahead

template <bool NORM, bool BUF, bool PERM, bool IDX>
__global__ __launch_bounds__(kMpBlock) void mp_scatter_kernel(
    const float* __restrict__ vec, const float* __restrict__ X, const int64_t* __restrict__ src_idx,
    const int64_t* __restrict__ perm, const int64_t* __restrict__ row_ptr,
    const int64_t* __restrict__ row_dst, float* __restrict__ out, int64_t n_rows, int C,
    int rows_per_block, int n_logical, uint32_t x_bytes) {
    static_assert(kSBatch == 64, "one edge per lane in phase 1, 64-bit row-end mask");
    static_assert(kSBatch % kRing == 0, "ring slots must line up across batches");
    static_assert(!IDX || BUF, "index-mode gathers use the buffer descriptor");
    static_assert(kScatterRows <= 16, "row ends gathered by a 16-lane OR (row0_or)");
    // 66.5 KB + row ranges: two workgroups per compute unit
    __shared__ __attribute__((aligned(16))) float sM[kSBatch * kMStride];
    __shared__ int64_t sRow[kScatterRows + 1];
    __shared__ int64_t sDst[kScatterRows];
    __shared__ int64_t sNE[kScatterRows];  // output rows of the non-empty rows, in row order
    // IDX: source rows of the gather targets, entry t for edge kb + kRing + t
    __shared__ int sTgt[kSBatch];
    // Y of a batch's edges (lane j: edge j), written by wave 0 one batch ahead; two
    // buffers by batch parity.  Lane j's four quads at j * 16, quad q at q ^ (j >> 1 & 3).
    __shared__ __attribute__((aligned(16))) float sYb[2][kSBatch * 16];

    const int per_xcd = (n_logical + 7) / 8;
    const int logical = (blockIdx.x & 7) * per_xcd + (blockIdx.x >> 3);
    if (logical >= n_logical) return;

    const int lane = threadIdx.x & 63;
    const int w = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);  // wave-uniform
    const int g = lane >> 4;
    const int i16 = lane & 15;
    const int c = blockIdx.y * kChanGroup + w * 16 + i16;
    const uint32_t row_bytes = (uint32_t)C * 64u;
    const int voff = (c < C ? c : C - 1) * 64 + g * 16;
    const __amdgpu_buffer_rsrc_t xr = __builtin_amdgcn_make_buffer_rsrc(
        const_cast<float*>(X), (short)0, BUF ? (int)x_bytes : 0, kBufferDword3);
    // IDX: rows of row_bytes as records (index = source row, no scalar offset)
    const __amdgpu_buffer_rsrc_t xs = __builtin_amdgcn_make_buffer_rsrc(
        const_cast<float*>(X), (short)(IDX ? row_bytes : 0u), IDX ? (int)(x_bytes / row_bytes) : 0,
        kBufferDword3);

    const int64_t d0 = (int64_t)logical * rows_per_block;
    const int nrows = (int)(min<int64_t>(n_rows, d0 + rows_per_block) - d0);
    for (int i = threadIdx.x; i <= nrows; i += kMpBlock) {
        sRow[i] = row_ptr[d0 + i];
        if (i < nrows) sDst[i] = row_dst ? row_dst[d0 + i] : d0 + i;
    }
    __syncthreads();
    // the edge range in scalar registers (compared at every half)
    const int64_t e0 = uniform_i64(sRow[0]), e1 = uniform_i64(sRow[nrows]);
    auto put_out = [&](int64_t orow, float4 v) {
        if (c < C && orow >= 0) *reinterpret_cast<float4*>(out + (orow * C + c) * 16 + 4 * g) = v;
    };
    // list the non-empty rows (the empty ones are written as zeros at the end): wave
    // 0, the rank of a row among them from a ballot
    if (threadIdx.x < 64) {
        const bool ne = (int)threadIdx.x < nrows && sRow[threadIdx.x + 1] > sRow[threadIdx.x];
        const uint64_t m = __ballot(ne);
        if (ne) sNE[__builtin_popcountll(m & ((1ull << threadIdx.x) - 1))] = sDst[threadIdx.x];
    }
    __syncthreads();

    // Lane r < nrows: the last edge of row r relative to e0 (-1: empty or absent
    // row).  The row ends in a batch are then a few lane-parallel instructions and a
    // 16-lane OR, not a scalar test per row.
    int rlast = -1;
    if (lane < nrows && sRow[lane + 1] > sRow[lane]) rlast = (int)(sRow[lane + 1] - 1 - e0);

    // Edge records move through a three-stage pipeline so that no wait is on a
    // load younger than the gathers in flight: the edge id of batch b+3 (one
    // load when PERM) and the record of batch b+2 are issued at the start of
    // batch b; the record of batch b+1 (its source rows feed this batch's
    // gathers) and of batch b (phase 1) were issued one and two batches earlier.
    auto edge_id = [&](int64_t kbatch) -> int64_t {
        const int64_t k = kbatch + lane;
        if (k >= e1) return -1;
        if constexpr (PERM) return perm[k];
        else return k;
    };
    auto record = [&](int64_t e) {
        EdgeRec r{0.f, 0.f, 0.f, 0};
        if (e >= 0) {
            r.x = vec[e * 3 + 0];
            r.y = vec[e * 3 + 1];
            r.z = vec[e * 3 + 2];
            r.src = (int)src_idx[e];
        }
        return r;
    };

    const v4f zero4 = {0.f, 0.f, 0.f, 0.f};
    v4f acc = zero4;

    // Non-empty rows close in row order: k_ne of them have closed.  Lane k holds
    // the byte offset of the k-th one's output row (-1: none), which a close takes
    // with two lane reads.
    int k_ne = 0;
    int64_t obyte = -1;
    if (lane < kScatterRows) {
        const int64_t orow = sNE[lane];
        if (lane < __builtin_popcountll(__ballot(lane < nrows && sRow[lane + 1] > sRow[lane])) && orow >= 0)
            obyte = orow * (int64_t)row_bytes;
    }
    const int ob_lo = (int)(uint32_t)obyte, ob_hi = (int)((uint64_t)obyte >> 32);
    const int lane_off = c * 64 + g * 16;  // byte offset of the lane's float4 in an output row
    const bool tile_full = blockIdx.y * kChanGroup + w * 16 + 16 <= C;  // wave-uniform
    // IDX: after the first batch's (the ring fill's source rows) only wave 0 uses the
    // records (Y into LDS, gather indices into sTgt), so the other waves skip them
    const bool recs = !IDX || w == 0;  // wave-uniform
    EdgeRec cur = record(edge_id(e0));
    EdgeRec nxt = recs ? record(edge_id(e0 + kSBatch)) : EdgeRec{0.f, 0.f, 0.f, 0};
    int64_t id2 = recs ? edge_id(e0 + 2 * kSBatch) : (int64_t)-1;
    // Every wave runs the edge loop, also one whose 16 channels are all past C
    // (its lanes read channel C-1 and never store): a branch around the loop
    // would make the loop-carried records look like the youngest loads on one
    // path, and the compiler would drain every gather at the loop latch.  (The
    // guard encloses the ring fill and the loop together for the same reason:
    // the loop header is reached only after the ring fill.)
    float4 ring[kRing];
    // Per-half state of phase 2, shared with the last half's walk after the loops.
    const float* mrow = sM + i16 * 16 + 4 * (g ^ quad_swizzle(i16));
    const float* mh = mrow;
    float4 mr[kLdsAhead + 1];
    const int* th = sTgt;
    const int* th2 = sTgt;  // the next half's first gather indices
    // IDX: (gather index, lane offset) pairs, the vaddr pair of an index-mode
    // load; pair j % 4 serves edge j and is refilled with the index of edge
    // j + 4 once its load is issued, so that no index is waited for right after
    // its LDS read
    typedef int v2i_t __attribute__((ext_vector_type(2)));
    v2i_t tgp[4] = {v2i_t{0, voff}, v2i_t{0, voff}, v2i_t{0, voff}, v2i_t{0, voff}};
    int gsrc = 0, lsel = 0;
    uint32_t ends_h = 0;
    int64_t kh = e0;
    // edge j of a half: four MFMAs into the row accumulator, the gather of the
    // edge kRing positions ahead (GATHER), and where j closes a row its store
    auto edge = [&](auto jj, auto gather_c) {
        constexpr int j = decltype(jj)::value;
        // IDX: one wait per pair of edges, at the even one, for both edges'
        // gather slots, gather indices and the odd edge's operator fragment
        // (all issued two or more edges earlier): the empty asm takes them as
        // operands, so the compiler places a single s_waitcnt before it, and
        // the odd edge needs none
        if constexpr (IDX && decltype(gather_c)::value && (j & 1) == 0) {
            constexpr int m1 = (j + 1) % (kLdsAhead + 1);
            asm volatile("" ::"v"(tgp[j & 3].x), "v"(tgp[(j + 1) & 3].x), "v"(ring[j].x),
                         "v"(ring[j].y), "v"(ring[j].z), "v"(ring[j].w), "v"(ring[j + 1].x),
                         "v"(ring[j + 1].y), "v"(ring[j + 1].z), "v"(ring[j + 1].w), "v"(mr[m1].x),
                         "v"(mr[m1].y), "v"(mr[m1].z), "v"(mr[m1].w));
            __builtin_amdgcn_sched_barrier(0);
        }
        mr[(j + kLdsAhead) % (kLdsAhead + 1)] =
            *reinterpret_cast<const float4*>(mh + (j + kLdsAhead) * kMStride);
        acc = mfma4(mr[j % (kLdsAhead + 1)], ring[j], acc);
        // the slot's next gather after the MFMAs that read it: hoisted above
        // them it would need a second register ring
        __builtin_amdgcn_sched_barrier(0);
        if constexpr (decltype(gather_c)::value) {
            if constexpr (IDX) {
                const v4i_t r = struct_buffer_load_b128(xs, tgp[j & 3].x, tgp[j & 3].y, 0, 0);
                ring[j] = make_float4(__int_as_float(r.x), __int_as_float(r.y), __int_as_float(r.z),
                                      __int_as_float(r.w));
                // the index of edge j + 4: past the half, the next half's (in
                // the second half a valid address whose value is not used: the
                // next batch reloads the pairs after its phase 1)
                if constexpr (j + 4 < kRing) tgp[j & 3].x = th[j + 4];
                else tgp[j & 3].x = th2[j + 4 - kRing];
            } else {
                ring[j] = gather<BUF>(X, xr, voff, __builtin_amdgcn_readlane(gsrc, lsel + j), row_bytes);
            }
        }
        // rare: laid out off the edge path, so that an edge that closes no row
        // falls through (no taken branch, 54.2 -> 53.0 us at configs[3])
        if (__builtin_expect((ends_h >> j) & 1u, 0)) {
            const int hi = __builtin_amdgcn_readlane(ob_hi, k_ne);
            const int64_t ob = (int64_t)(((uint64_t)(uint32_t)hi << 32) |
                                         (uint32_t)__builtin_amdgcn_readlane(ob_lo, k_ne));
            if (hi >= 0 && (tile_full || c < C))
                store_row_acc(reinterpret_cast<char*>(out) + ob, lane_off, acc);
            ++k_ne;
            acc = zero4;
        }
    };
    // Y in LDS: lane j's 16 values as four swizzled quads
    auto put_y = [&](float* buf, const float* Yv) {
        float4* q = reinterpret_cast<float4*>(buf + lane * 16);
        const int sw = (lane >> 1) & 3;
        static_for<4>([&](auto qq) {
            constexpr int k = decltype(qq)::value;
            q[k ^ sw] = make_float4(Yv[4 * k], Yv[4 * k + 1], Yv[4 * k + 2], Yv[4 * k + 3]);
        });
    };
    auto get_y = [&](const float* buf, float* Yv) {
        const float4* q = reinterpret_cast<const float4*>(buf + lane * 16);
        const int sw = (lane >> 1) & 3;
        static_for<4>([&](auto qq) {
            constexpr int k = decltype(qq)::value;
            const float4 v = q[k ^ sw];
            Yv[4 * k] = v.x;
            Yv[4 * k + 1] = v.y;
            Yv[4 * k + 2] = v.z;
            Yv[4 * k + 3] = v.w;
        });
    };
    int ypar = 0;
    if (e0 == e1) goto done;
    // the first batch's Y, for the first phase 1 (after the barrier at the top of the loop)
    if (w == 0) {
        float Y0[16];
        edge_sh<NORM>(cur, Y0);
        put_y(sYb[0], Y0);
    }
    static_for<kRing>([&](auto uu) {
        constexpr int u = decltype(uu)::value;
        ring[u] = gather<BUF>(X, xr, voff, __builtin_amdgcn_readlane(cur.src, u), row_bytes);
    });
    for (int64_t kb = e0;; kb += kSBatch) {
        const int nb = (int)min<int64_t>(kSBatch, e1 - kb);
        __syncthreads();
        // records of batch b+2 and the edge ids of b+3 (no load past e1)
        const EdgeRec nn = recs ? record(id2) : EdgeRec{0.f, 0.f, 0.f, 0};
        if (recs) id2 = edge_id(kb + 3 * kSBatch);
        // wave 0: Y of the next batch's edges; every wave: its rows of this batch's
        // operators from this batch's Y (written one batch ago)
        if (w == 0) {
            float Yn[16];
            edge_sh<NORM>(nxt, Yn);
            put_y(sYb[ypar ^ 1], Yn);
        }
        {
            float Y[16];
            get_y(sYb[ypar], Y);
            if (lane < nb) {
                switch (w) {
                    case 0: build_rows_sh<0>(Y, sM + lane * kMStride); break;
                    case 1: build_rows_sh<1>(Y, sM + lane * kMStride); break;
                    case 2: build_rows_sh<2>(Y, sM + lane * kMStride); break;
                    default: build_rows_sh<3>(Y, sM + lane * kMStride); break;
                }
            }
        }
        ypar ^= 1;
        if constexpr (IDX)
            if (w == 0) sTgt[(lane + kRing) & (kSBatch - 1)] = lane >= kRing ? cur.src : nxt.src;
        // edges of this batch that close a row (distinct rows end at distinct edges)
        const int rel = (int)(kb - e0);
        uint64_t ends;
        {
            const int p = rlast - rel;
            const bool in = rlast >= 0 && p >= 0 && p < kSBatch;
            const uint32_t lo = (in && p < 32) ? 1u << (p & 31) : 0u;
            const uint32_t hi = (in && p >= 32) ? 1u << (p & 31) : 0u;
            ends = ((uint64_t)row0_or(hi) << 32) | row0_or(lo);
        }
        // This batch's record loads are waited for here, at the end of phase
        // 1, where they have had its whole length to complete: pending at the
        // half loop's header, they would make the compiler drain the gathers
        // at the first edge of every half.
        __builtin_amdgcn_s_waitcnt(0x0F70);  // vmcnt(0)
        __syncthreads();
        static_for<kLdsAhead>([&](auto qq) {
            constexpr int q = decltype(qq)::value;
            mr[q] = *reinterpret_cast<const float4*>(mrow + q * kMStride);
        });
        if constexpr (IDX)
            static_for<4>([&](auto qq) {
                constexpr int q = decltype(qq)::value;
                tgp[q].x = sTgt[q + (voff >> 30)];
            });
        // Phase 2 in two halves of kRing edges, a loop that is not unrolled:
        // each ring slot is then defined once per iteration (by the gather
        // kRing edges ahead) and stays in its registers.  Half h gathers the
        // source rows of the edges kRing ahead from lanes lsel + j of gsrc:
        // this batch's records (lanes 32..63) in half 0, the next batch's
        // (lanes 0..31) in half 1.  The loop has one path: a half that is not
        // full (last batch) leaves at its top for the walk after the loops,
        // and the last full half leaves at its end (exits from inside a half
        // would make the compiler wait for most gathers at every edge).
#pragma clang loop unroll(disable)
        for (int h = 0; h < kSBatch / kRing; ++h) {
            const int jb = h * kRing;
            mh = mrow + jb * kMStride;
            // the table address of the half in one VGPR: voff >> 30 is 0, but
            // not known to be uniform, so the address is not rebuilt from a
            // scalar register at every edge
            th = sTgt + jb + (voff >> 30);
            th2 = sTgt + (h == 0 ? kRing : 0) + (voff >> 30);
            gsrc = h == 0 ? cur.src : nxt.src;
            lsel = h == 0 ? kRing : 0;
            ends_h = (uint32_t)(ends >> jb);
            kh = kb + jb;
            if (kh + kRing > e1) goto partial;
            static_for<kRing>([&](auto jj) { edge(jj, std::true_type{}); });
            if (kh + kRing >= e1) goto done;
        }
        cur = nxt;
        nxt = nn;
    }
partial:
    // the last half, not full: the groups of 8 edges that hold real edges, no
    // gathers (no edge follows); edges past e1 in the last group only touch the
    // accumulator after the last row has closed
    static_for<kRing / 8>([&](auto gg) {
        constexpr int j8 = 8 * decltype(gg)::value;
        if (kh + j8 < e1)
            static_for<8>([&](auto ii) {
                edge(std::integral_constant<int, j8 + decltype(ii)::value>{}, std::false_type{});
            });
    });
done:
    for (int r = 0; r < nrows; ++r)
        if (sRow[r + 1] == sRow[r]) put_out(sDst[r], make_float4(0.f, 0.f, 0.f, 0.f));
}

// ---------------------------------------------------------------------------
// Channel-half scatter kernel: the sums of mp_scatter_kernel for graphs whose source rows
// have no spatial order (sources spread over all atoms).  There one XCD's workgroups gather
// from nearly every row of X, and at C = 64 (20 MB at configs[3]'s size) its 4 MB L2 holds
// a fifth of them.  Here the XCDs form 4 / NCH groups, each taking 16 NCH channels of every
// 64-channel group for every destination (NCH = 2: XCDs 0-3 channels 0-31, XCDs 4-7
// channels 32-63), so an XCD's L2 sees a part of each row.
//
// A workgroup owns its destination block for 16 NCH channels.  Its edge range [e0, e1) is
// cut into P equal parts; the 4 / P waves of a part share its NCH 16-channel tiles (P = 2,
// NCH = 2: one tile per wave, 4 MFMAs per edge; P = 4: NCH tiles per wave, on one operator
// fragment).  Phase 1 builds the operators of 64 edges per batch (64 / P of each part) as
// mp_scatter_kernel does, so each edge's operator is built once per channel group.  Gathers
// run 32 / P edges ahead (a float4 per tile; tiles 1 KB apart in the row, one index pair
// and the instruction's offset field).  The launch uses P = 2, NCH = 2 (kHalfParts,
// kHalfTiles); P = 4 ran at the same speed, NCH = 1 slower (four operator builds per edge).
//
// A row cut by a part boundary is summed in pieces: the part that holds the row's first
// edge keeps its piece in the accumulator (the tail), a part that the row covers entirely
// keeps its piece too, and the part where the row ends writes its piece (the head) to the
// output row as if the row were its own.  After the last batch the covered parts' pieces
// meet in LDS, and the wave of the first piece adds them and the head (read back from the
// output row) in part order and writes the row.  The cuts depend only on e0 and e1, so the
// result is deterministic; rows that no cut crosses are summed in the same order as by
// mp_scatter_kernel.
// ---------------------------------------------------------------------------
template <bool NORM, bool PERM, int P, int NCH>
__global__ __launch_bounds__(kMpBlock) void mp_scatter_half_kernel(
    const float* __restrict__ vec, const float* __restrict__ X, const int64_t* __restrict__ src_idx,
    const int64_t* __restrict__ perm, const int64_t* __restrict__ row_ptr,
    const int64_t* __restrict__ row_dst, float* __restrict__ out, int64_t n_rows, int C,
    int rows_per_block, int n_logical, uint32_t x_bytes) {
    static_assert(P == 2 || P == 4, "two or four parts");
    static_assert(NCH == 1 || NCH == 2, "16 or 32 channels per workgroup");
    constexpr int kEsPer = kSBatch / P;    // edges of a part per batch
    constexpr int kEsRing = kEsPer / 2;    // edges ahead whose source rows are in flight
    constexpr int kWpp = 4 / P;            // waves per part
    constexpr int kEsTiles = NCH / kWpp;   // 16-channel tiles per wave
    static_assert(kEsTiles >= 1, "every wave owns a tile");
    constexpr int kGroups = 4 / NCH;       // channel groups of a 64-channel group
    constexpr int kXcdPerGroup = 8 / kGroups;
    static_assert(kEsPer <= 32, "row ends of a part's batch in a 32-bit mask");
    static_assert(kScatterRows <= 16, "row ends gathered by a 16-lane OR (row0_or)");
    // gather source rows: entry kEsPer p + t is part p's edge kEsRing + t of the batch
    // (t >= kEsRing: the next batch's edge t - kEsRing).  Aligned above the other arrays so
    // that it is laid out first, at an LDS address that the reads' 16-bit offset field
    // reaches.
    __shared__ __attribute__((aligned(64))) int sTgt[kSBatch];
    __shared__ int sPiece[P];  // per part: see the end of the kernel
    __shared__ int64_t sRow[kScatterRows + 1];
    __shared__ int64_t sDst[kScatterRows];
    __shared__ int64_t sNE[kScatterRows];  // output rows of the non-empty rows, in row order
    // operators of a batch (+ 3 slots that the read-ahead past a part's last edge may
    // touch); after the last batch, the row pieces
    __shared__ __attribute__((aligned(16))) float sM[(kSBatch + 3) * kMStride];

    // XCD x = blockIdx % 8: channel group x / kXcdPerGroup (16 NCH channels); the group's
    // blocks dealt over its XCDs
    const int xcd = blockIdx.x & 7, cgrp = xcd / kXcdPerGroup;
    const int perx = (n_logical + kXcdPerGroup - 1) / kXcdPerGroup;
    const int logical = (xcd % kXcdPerGroup) * perx + (int)(blockIdx.x >> 3);
    if (logical >= n_logical) return;

    const int lane = threadIdx.x & 63;
    const int w = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);  // wave-uniform
    const int part = w / kWpp, tb = (w % kWpp) * kEsTiles;  // the wave's part and first tile
    const int g = lane >> 4;
    const int i16 = lane & 15;
    const uint32_t row_bytes = (uint32_t)C * 64u;
    // the lane's float4 of its first tile in a row of X or of the output; tile t at + 1024 t
    const int lane_off = (blockIdx.y * kChanGroup + cgrp * 16 * NCH + tb * 16 + i16) * 64 + g * 16;
    const __amdgpu_buffer_rsrc_t xs = __builtin_amdgcn_make_buffer_rsrc(
        const_cast<float*>(X), (short)row_bytes, (int)(x_bytes / row_bytes), kBufferDword3);

    const int64_t d0 = (int64_t)logical * rows_per_block;
    const int nrows = (int)(min<int64_t>(n_rows, d0 + rows_per_block) - d0);
    for (int i = threadIdx.x; i <= nrows; i += kMpBlock) {
        sRow[i] = row_ptr[d0 + i];
        if (i < nrows) sDst[i] = row_dst ? row_dst[d0 + i] : d0 + i;
    }
    __syncthreads();
    const int64_t e0 = uniform_i64(sRow[0]), e1 = uniform_i64(sRow[nrows]);
    if (threadIdx.x < 64) {
        const bool ne = (int)threadIdx.x < nrows && sRow[threadIdx.x + 1] > sRow[threadIdx.x];
        const uint64_t m = __ballot(ne);
        if (ne) sNE[__builtin_popcountll(m & ((1ull << threadIdx.x) - 1))] = sDst[threadIdx.x];
    }
    // the parts: the waves of part p sum edges [e0 + pb, e0 + pe)
    const int len = (int)(e1 - e0);
    const int pb = (int)((int64_t)len * part / P), pe = (int)((int64_t)len * (part + 1) / P);
    const int plen = pe - pb;
    const int nbatch = ((len + P - 1) / P + kEsPer - 1) / kEsPer;
    // lane r < nrows: the last and first edge of row r relative to e0 (-1: empty or
    // absent); the non-empty rows that end before the part (the part's first close is
    // row kw0), and whether the part starts inside a row
    int rlast = -1, rfirst = 0;
    if (lane < nrows && sRow[lane + 1] > sRow[lane]) {
        rlast = (int)(sRow[lane + 1] - 1 - e0);
        rfirst = (int)(sRow[lane] - e0);
    }
    const int kw0 = __builtin_popcountll(__ballot(rlast >= 0 && rlast < pb));
    const bool head = __ballot(rlast >= pb && rfirst < pb) != 0;
    __syncthreads();

    // lane j's edge in phase 1: part j / kEsPer, edge kEsPer b + j % kEsPer of it
    const int jw = lane / kEsPer, jpos = lane % kEsPer;
    const int jpb = (int)((int64_t)len * jw / P), jpe = (int)((int64_t)len * (jw + 1) / P);
    auto edge_id = [&](int b) -> int64_t {
        const int k = jpb + b * kEsPer + jpos;
        if (k >= jpe) return -1;
        if constexpr (PERM) return perm[e0 + k];
        else return e0 + k;
    };
    auto record = [&](int64_t e) {
        EdgeRec r{0.f, 0.f, 0.f, 0};
        if (e >= 0) {
            r.x = vec[e * 3 + 0];
            r.y = vec[e * 3 + 1];
            r.z = vec[e * 3 + 2];
            r.src = (int)src_idx[e];
        }
        return r;
    };

    const v4f zero4 = {0.f, 0.f, 0.f, 0.f};
    v4f acc[kEsTiles];
    static_for<kEsTiles>([&](auto tt) { acc[decltype(tt)::value] = zero4; });
    int k_ne = kw0;
    bool head_open = head;  // the head row has not closed yet
    int64_t onext = sNE[min(kw0, kScatterRows - 1)];

    EdgeRec cur = record(edge_id(0));
    EdgeRec nxt = record(edge_id(1));
    int64_t id2 = edge_id(2);
    float4 ring[kEsRing][kEsTiles];
    const float* mrow = sM + i16 * 16 + 4 * (g ^ quad_swizzle(i16));  // the lane's fragment of slot 0
    float4 mr[kLdsAhead + 1];
    typedef int v2i_t __attribute__((ext_vector_type(2)));
    v2i_t tgp[4] = {v2i_t{0, lane_off}, v2i_t{0, lane_off}, v2i_t{0, lane_off}, v2i_t{0, lane_off}};
    const float* mh = mrow;
    const int* th = sTgt;
    const int* th2 = sTgt;  // the next half's first gather indices
    // a zero the compiler cannot see through, so that the index table's address stays in
    // a VGPR and every read takes its offset from the instruction
    int vzero;
    asm volatile("v_mov_b32 %0, 0" : "=v"(vzero));
    uint32_t ends_h = 0;

    // the tile offset in the scalar offset operand: one (index, lane offset) pair serves
    // the tiles' loads
    auto gather_t = [&](float4* dst, int idx) {
        static_for<kEsTiles>([&](auto tt) {
            constexpr int t = decltype(tt)::value;
            const v4i_t r = struct_buffer_load_b128(xs, idx, lane_off, 1024 * t, 0);
            dst[t] = make_float4(__int_as_float(r.x), __int_as_float(r.y), __int_as_float(r.z),
                                 __int_as_float(r.w));
        });
    };
    // a closing row (the head row too: its piece) goes to its output row
    auto close_row = [&]() {
        head_open = false;
        const int64_t orow = uniform_i64(onext);
        if (orow >= 0) {
            char* base = reinterpret_cast<char*>(out) + orow * (int64_t)row_bytes;
            static_for<kEsTiles>([&](auto tt) {
                constexpr int t = decltype(tt)::value;
                store_row_acc(base, lane_off + 1024 * t, acc[t]);
            });
        }
        ++k_ne;
        onext = sNE[min(k_ne, kScatterRows - 1)];
        static_for<kEsTiles>([&](auto tt) { acc[decltype(tt)::value] = zero4; });
    };
    // edge j of a half: 4 MFMAs per tile; GATHER: the gather of the edge kEsRing ahead
    // into the slot and its index read-ahead; TEST: the row-end test
    auto edge = [&](auto jj, auto gather_c, auto test_c) {
        constexpr int j = decltype(jj)::value;
        if constexpr (decltype(gather_c)::value) {
            // the slot's gathers (8 edges back), the gather index of this edge and the
            // operator fragment (3 edges back): one wait before the MFMAs
            constexpr int m0 = j % (kLdsAhead + 1);
            if constexpr (kEsTiles == 2)
                asm volatile("" ::"v"(tgp[j & 3].x), "v"(ring[j][0].x), "v"(ring[j][0].w),
                             "v"(ring[j][1].x), "v"(ring[j][1].w), "v"(mr[m0].x), "v"(mr[m0].w));
            else
                asm volatile("" ::"v"(tgp[j & 3].x), "v"(ring[j][0].x), "v"(ring[j][0].w),
                             "v"(mr[m0].x), "v"(mr[m0].w));
            __builtin_amdgcn_sched_barrier(0);
        }
        mr[(j + kLdsAhead) % (kLdsAhead + 1)] =
            *reinterpret_cast<const float4*>(mh + (j + kLdsAhead) * kMStride);
        // tile by tile: each tile's gather for the edge kEsRing ahead follows the four
        // MFMAs that read its slot, so that the loads spread over the edge
        static_for<kEsTiles>([&](auto tt) {
            constexpr int t = decltype(tt)::value;
            acc[t] = mfma4(mr[j % (kLdsAhead + 1)], ring[j][t], acc[t]);
            __builtin_amdgcn_sched_barrier(0);
            if constexpr (decltype(gather_c)::value) {
                const v4i_t r = struct_buffer_load_b128(xs, tgp[j & 3].x, lane_off, 1024 * t, 0);
                ring[j][t] = make_float4(__int_as_float(r.x), __int_as_float(r.y), __int_as_float(r.z),
                                         __int_as_float(r.w));
            }
        });
        if constexpr (decltype(gather_c)::value) {
            // the index of edge j + 4 of the half: past the half, the next half's first
            // ones (in the second half a valid entry whose value is not used: the next
            // batch reloads the pairs after its phase 1)
            if constexpr (j + 4 < kEsRing) tgp[j & 3].x = th[j + 4];
            else tgp[j & 3].x = th2[j + 4 - kEsRing];
        }
        if (decltype(test_c)::value && __builtin_expect((ends_h >> j) & 1u, 0)) close_row();
    };

    if (e0 == e1) goto done;
    // the ring: the part's first kEsRing edges
    static_for<kEsRing>([&](auto uu) {
        constexpr int u = decltype(uu)::value;
        const int s = __builtin_amdgcn_readlane(cur.src, kEsPer * part + u);
        gather_t(ring[u], s);
    });
    for (int b = 0; b < nbatch; ++b) {
        __syncthreads();
        // records of batch b+2 and the edge ids of b+3
        const EdgeRec nn = record(id2);
        id2 = edge_id(b + 3);
        float Y[16];
        edge_sh<NORM>(cur, Y);
        edge_rows(Y, sM + lane * kMStride, w);
        if (w == 0) sTgt[lane ^ kEsRing] = (lane & kEsRing) ? cur.src : nxt.src;
        // rows that end in this batch's edges of the part (distinct rows end at distinct
        // edges: a 16-lane OR)
        const int rel = pb + b * kEsPer;
        uint32_t ends;
        {
            const int p = rlast - rel;
            const bool in = rlast >= 0 && rlast < pe && p >= 0 && p < kEsPer;
            ends = row0_or(in ? 1u << (p & 31) : 0u);
        }
        const int nv = min(kEsPer, max(0, plen - b * kEsPer));  // the part's edges in this batch
        __builtin_amdgcn_s_waitcnt(0x0F70);  // vmcnt(0): this batch's records
        __syncthreads();
        mh = mrow + kEsPer * part * kMStride;
        static_for<kLdsAhead>([&](auto qq) {
            constexpr int q = decltype(qq)::value;
            mr[q] = *reinterpret_cast<const float4*>(mh + q * kMStride);
        });
        static_for<4>([&](auto qq) {
            constexpr int q = decltype(qq)::value;
            tgp[q].x = sTgt[kEsPer * part + q + vzero];
        });
        // phase 2 in two halves of kEsRing edges, a loop that is not unrolled (each ring
        // slot is then defined once per iteration).  A half that the part does not fill
        // leaves at its top for the walk after the loop.
        int kh = kEsPer;
#pragma clang loop unroll(disable)
        for (int h = 0; h < 2; ++h) {
            const int jb = h * kEsRing;
            mh = mrow + (kEsPer * part + jb) * kMStride;
            th = sTgt + kEsPer * part + jb + vzero;
            th2 = sTgt + kEsPer * part + (h == 0 ? kEsRing : 0) + vzero;
            ends_h = ends >> jb;
            if (nv < jb + kEsRing) {
                kh = jb;
                break;
            }
            static_for<kEsRing>([&](auto jj) { edge(jj, std::true_type{}, std::true_type{}); });
        }
        if (kh < kEsPer) {
            // the part's last edges: no gathers (no edge of the part follows), and no edge
            // past the part touches the accumulators.  Later batches (other parts may have
            // one more) have none.
            const int rem = nv - kh;
            static_for<kEsRing>([&](auto jj) {
                if (decltype(jj)::value < rem) edge(jj, std::false_type{}, std::true_type{});
            });
        }
        cur = nxt;
        nxt = nn;
    }
done:
    // the pieces of the rows that part boundaries cut
    __syncthreads();
    {
        float4* sP = reinterpret_cast<float4*>(sM);  // [part][tile][lane]: pieces of parts inside one row
        // the part's last edge ends a row unless its row continues into the next part
        const bool last_ends = __ballot(rlast >= 0 && rlast == pe - 1) != 0;
        const bool tail = plen > 0 && part < P - 1 && !last_ends;
        // 1: the row that the part starts in ends in it (its piece is in the output row),
        // 2: the part lies inside one row, 3: the part is empty and inside a row
        int piece = 0;
        if (head) piece = (head_open && plen > 0) ? 2 : (head_open ? 3 : 1);
        if (piece == 2)
            static_for<kEsTiles>([&](auto tt) {
                constexpr int t = decltype(tt)::value;
                sP[(part * NCH + tb + t) * 64 + lane] = make_float4(acc[t][0], acc[t][1], acc[t][2], acc[t][3]);
            });
        if (lane == 0 && tb == 0) sPiece[part] = piece;  // the part's waves agree on it
        // the heads' stores (issued unseen by the compiler) complete before the barrier
        __builtin_amdgcn_s_waitcnt(0x0F70);  // vmcnt(0)
        __syncthreads();
        // the wave that holds a cut row's first edges adds the later pieces in part order
        if (tail && !(head && head_open)) {
            const int64_t orow = uniform_i64(onext);
            v4f sum[kEsTiles];
            static_for<kEsTiles>([&](auto tt) { sum[decltype(tt)::value] = acc[decltype(tt)::value]; });
            auto add = [&](v4f* s, const float4* v) {
                static_for<kEsTiles>([&](auto tt) {
                    constexpr int t = decltype(tt)::value;
                    s[t][0] += v[t].x;
                    s[t][1] += v[t].y;
                    s[t][2] += v[t].z;
                    s[t][3] += v[t].w;
                });
            };
            for (int q = part + 1; q < P; ++q) {
                const int pc = sPiece[q];
                float4 v[kEsTiles];
                if (pc == 2) {
                    static_for<kEsTiles>([&](auto tt) {
                        v[decltype(tt)::value] = sP[(q * NCH + tb + decltype(tt)::value) * 64 + lane];
                    });
                    add(sum, v);
                } else if (pc == 1) {
                    // the head: read back from the output row past the compute unit's cache
                    // (glc), where the part's wave stored it before the barrier
                    if (orow >= 0) {
                        const __amdgpu_buffer_rsrc_t orr = __builtin_amdgcn_make_buffer_rsrc(
                            out + orow * (int64_t)C * 16, (short)0, (int)row_bytes, kBufferDword3);
                        static_for<kEsTiles>([&](auto tt) {
                            constexpr int t = decltype(tt)::value;
                            const auto r = __builtin_amdgcn_raw_buffer_load_b128(orr, lane_off + 1024 * t, 0, 1);
                            v[t] = make_float4(__int_as_float(r[0]), __int_as_float(r[1]), __int_as_float(r[2]),
                                               __int_as_float(r[3]));
                        });
                        add(sum, v);
                    }
                    break;  // the row ends in part q
                }
            }
            if (orow >= 0)
                static_for<kEsTiles>([&](auto tt) {
                    constexpr int t = decltype(tt)::value;
                    *reinterpret_cast<float4*>(out + orow * (int64_t)C * 16 + (lane_off + 1024 * t) / 4) =
                        make_float4(sum[t][0], sum[t][1], sum[t][2], sum[t][3]);
                });
        }
    }
    // empty rows: zeros, written by the waves of part 0 (their tiles)
    if (part == 0)
        for (int r = 0; r < nrows; ++r)
            if (sRow[r + 1] == sRow[r] && sDst[r] >= 0)
                static_for<kEsTiles>([&](auto tt) {
                    constexpr int t = decltype(tt)::value;
                    *reinterpret_cast<float4*>(out + sDst[r] * (int64_t)C * 16 + (lane_off + 1024 * t) / 4) =
                        make_float4(0.f, 0.f, 0.f, 0.f);
                });
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

// Ascending order inside each row: one wave per row, each entry written at its
// rank (the number of smaller entries; edge ids are distinct).  Rows of up to
// 64 * kCsrSortPerLane entries are held in registers (compared against every
// entry of the row, broadcast by readlane); longer rows, far denser than any
// cutoff gives, are sorted by one lane in place.  (A thread per row with an
// insertion sort in global memory took 250 us for the 5000 rows of the
// reference's random benchmark graph.)
constexpr int kCsrSortPerLane = 8;
__global__ __launch_bounds__(256) void csr_sort_rows_kernel(const int64_t* __restrict__ row_ptr,
                                                            int64_t* __restrict__ col_idx,
                                                            int64_t n_atoms) {
    const int64_t t = (int64_t)blockIdx.x * 4 + (threadIdx.x >> 6);
    if (t >= n_atoms) return;  // wave-uniform
    const int lane = threadIdx.x & 63;
    const int64_t s = row_ptr[t];
    const int64_t len = row_ptr[t + 1] - s;
    if (len <= 1) return;
    if (len <= 64 * kCsrSortPerLane) {
        const int n = (int)len;
        int64_t v[kCsrSortPerLane];
        int rank[kCsrSortPerLane];
#pragma unroll
        for (int k = 0; k < kCsrSortPerLane; ++k) {
            const int i = k * 64 + lane;
            v[k] = i < n ? col_idx[s + i] : INT64_MAX;
            rank[k] = 0;
        }
#pragma unroll
        for (int kk = 0; kk < kCsrSortPerLane; ++kk) {
            if (kk * 64 >= n) break;  // uniform
            const int m = min(64, n - kk * 64);
            for (int j = 0; j < m; ++j) {
                const uint32_t lo = __builtin_amdgcn_readlane((uint32_t)v[kk], j);
                const uint32_t hi = __builtin_amdgcn_readlane((uint32_t)((uint64_t)v[kk] >> 32), j);
                const int64_t w = (int64_t)(((uint64_t)hi << 32) | lo);
#pragma unroll
                for (int k = 0; k < kCsrSortPerLane; ++k) rank[k] += w < v[k] ? 1 : 0;
            }
        }
#pragma unroll
        for (int k = 0; k < kCsrSortPerLane; ++k)
            if (k * 64 + lane < n) col_idx[s + rank[k]] = v[k];
        return;
    }
    if (lane == 0) {
        for (int64_t i = s + 1; i < s + len; ++i) {
            const int64_t x = col_idx[i];
            int64_t j = i - 1;
            while (j >= s && col_idx[j] > x) {
                col_idx[j + 1] = col_idx[j];
                --j;
            }
            col_idx[j + 1] = x;
        }
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

// D[abid][l][r] = the accumulator of mfma_4x4_bcast<abid>(A[l], B[l], 0) in lane l
__global__ void selftest_mfma_4x4_bcast_kernel(const float* __restrict__ A,
                                               const float* __restrict__ B, float* __restrict__ D) {
    const int l = threadIdx.x;
    const float a = A[l], b = B[l];
    static_for<16>([&](auto kk) {
        constexpr int k = decltype(kk)::value;
        const v4f d = mfma_4x4_bcast<k>(a, b, v4f{0.f, 0.f, 0.f, 0.f});
#pragma unroll
        for (int r = 0; r < 4; ++r) D[(k * 64 + l) * 4 + r] = d[r];
    });
}

}  // namespace bmhip

using namespace bmhip;

extern "C" int batteries_selftest_mfma_4x4x1_bcast(const float* A, const float* B, float* D,
                                                   hipStream_t stream) {
    if (!A || !B || !D) return BM_ERR_ARG;
    selftest_mfma_4x4_bcast_kernel<<<1, 64, 0, stream>>>(A, B, D);
    return (int)hipGetLastError();
}

extern "C" int batteries_selftest_mfma_16x16x4(const float* A, const float* B, float* D,
                                               hipStream_t stream) {
    if (!A || !B || !D) return BM_ERR_ARG;
    selftest_mfma_kernel<<<1, 64, 0, stream>>>(A, B, D);
    return (int)hipGetLastError();
}

// Compute units of the current device (cached per device).
static int device_cu_count() {
    static int cached[64] = {0};
    int dev = 0;
    if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 64) return 256;
    if (cached[dev] == 0) {
        int n = 0;
        if (hipDeviceGetAttribute(&n, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess ||
            n <= 0)
            n = 256;
        cached[dev] = n;
    }
    return cached[dev];
}

// Workgroups per XCD resident at once: 2 per compute unit (the LDS of one
// workgroup is under 80 KB of the 160 KB), spread over the channel groups.
static int blocks_per_xcd(int C) {
    const int groups = (int)ceil_div(C, kChanGroup);
    return std::max(1, 2 * device_cu_count() / groups / 8);
}

// Workgroups of one schedule group (mp_schedule.h): the workgroups resident on an XCD
// at once, at most one wave's lanes.
int bmhip::schedule_group_size(int n_blocks, int C) {
    return std::min(std::min(n_blocks / 8, blocks_per_xcd(C)), kSchedMaxQ);
}

// Launch with an explicit split: n_logical workgroups (a multiple of 8), each
// owning `per` consecutive destinations (SCATTER) or edges (MESSAGES).
static int launch_mp(bool scatter, bool norm, const float* vec, const float* X, int64_t n_src,
                     const int64_t* src_idx, const int64_t* perm, const int64_t* row_ptr,
                     const int64_t* row_dst, float* out, int64_t n_items, int64_t n_edges, int C,
                     int64_t per, int64_t n_logical, hipStream_t s) {
    if (C <= 0) return BM_ERR_ARG;
    if ((reinterpret_cast<uintptr_t>(X) | reinterpret_cast<uintptr_t>(out)) & 15) return BM_ERR_ARG;
    if (n_logical == 0) return BM_OK;
    if (per <= 0 || per > INT32_MAX || n_logical > INT32_MAX / 8) return BM_ERR_ARG;
    if (scatter && per > kScatterRows) return BM_ERR_ARG;
    if (n_src <= 0 || n_src > INT32_MAX) return BM_ERR_ARG;
    const int groups = (int)ceil_div(C, kChanGroup);
    const int64_t per_xcd = (n_logical + 7) / 8;
    dim3 grid((unsigned)(per_xcd * 8), (unsigned)groups);
    const int64_t xb = n_src * (int64_t)C * 64;
    const bool buf = xb <= (int64_t)INT32_MAX;
    const uint32_t x_bytes = buf ? (uint32_t)xb : 0u;
    // index-mode gathers: rows fit the descriptor's stride field
    const bool idx = buf && (int64_t)C * 64 <= kMaxBufferStride;
#define BM_LAUNCH(NO, BU)                                                                    \
    mp_simple_mfma_kernel<false, NO, BU><<<grid, kMpBlock, 0, s>>>(                           \
        vec, X, src_idx, perm, row_ptr, row_dst, out, n_items, n_edges, C, (int)per,          \
        (int)n_logical, x_bytes)
#define BM_LAUNCH_SC(NO, BU, PE, IX)                                                         \
    mp_scatter_kernel<NO, BU, PE, IX><<<grid, kMpBlock, 0, s>>>(vec, X, src_idx, perm, row_ptr, \
                                                                row_dst, out, n_items, C,       \
                                                                (int)per, (int)n_logical, x_bytes)
#define BM_LAUNCH_SC3(NO, BU, PE)                                                            \
    do { if (idx) BM_LAUNCH_SC(NO, true, PE, true); else BM_LAUNCH_SC(NO, BU, PE, false); } while (0)
#define BM_LAUNCH_SC2(NO, BU) \
    do { if (perm) BM_LAUNCH_SC3(NO, BU, true); else BM_LAUNCH_SC3(NO, BU, false); } while (0)
    if (scatter) {
        if (norm) {
            if (buf) BM_LAUNCH_SC2(true, true); else BM_LAUNCH_SC2(true, false);
        } else {
            if (buf) BM_LAUNCH_SC2(false, true); else BM_LAUNCH_SC2(false, false);
        }
    } else {
        if (norm) {
            if (buf) BM_LAUNCH(true, true); else BM_LAUNCH(true, false);
        } else {
            if (buf) BM_LAUNCH(false, true); else BM_LAUNCH(false, false);
        }
    }
#undef BM_LAUNCH_SC2
#undef BM_LAUNCH_SC3
#undef BM_LAUNCH_SC
#undef BM_LAUNCH
    return (int)hipGetLastError();
}

// The channel-half scatter (mp_scatter_half_kernel) over a schedule's blocks, whose edges
// come through edge_perm: C a multiple of 64 whose rows fit an index-mode descriptor, X
// under 2 GiB.  Returns BM_ERR_ARG for other inputs (the caller then runs mp_scatter_kernel).
constexpr int kHalfParts = 2;  // edge parts of a channel-half workgroup (2 or 4)
constexpr int kHalfTiles = 2;  // 16-channel tiles of a workgroup (2: XCD halves, 1: quarters)

static int launch_mp_half(bool norm, const float* vec, const float* X, int64_t n_src,
                          const int64_t* src_idx, const int64_t* perm, const int64_t* row_ptr,
                          const int64_t* row_dst, float* out, int64_t n_items, int C, int64_t per,
                          int64_t n_logical, hipStream_t s) {
    if (C <= 0 || C % kChanGroup || (int64_t)C * 64 > kMaxBufferStride || !perm) return BM_ERR_ARG;
    if ((reinterpret_cast<uintptr_t>(X) | reinterpret_cast<uintptr_t>(out)) & 15) return BM_ERR_ARG;
    if (n_logical == 0) return BM_OK;
    if (per <= 0 || per > kScatterRows || n_logical > INT32_MAX / 8) return BM_ERR_ARG;
    if (n_src <= 0 || n_src > INT32_MAX) return BM_ERR_ARG;
    const int64_t xb = n_src * (int64_t)C * 64;
    if (xb > (int64_t)INT32_MAX) return BM_ERR_ARG;
    dim3 grid((unsigned)(ceil_div(n_logical, 2 * kHalfTiles) * 8), (unsigned)(C / kChanGroup));
#define BM_LAUNCH_H(NO, PE)                                                                     \
    mp_scatter_half_kernel<NO, PE, kHalfParts, kHalfTiles><<<grid, kMpBlock, 0, s>>>(            \
        vec, X, src_idx, perm, row_ptr, row_dst, out, n_items, C, (int)per, (int)n_logical,      \
        (uint32_t)xb)
    if (norm) BM_LAUNCH_H(true, true); else BM_LAUNCH_H(false, true);
#undef BM_LAUNCH_H
    return (int)hipGetLastError();
}

// Default split: one resident wave of workgroups, each owning a contiguous range.
static int launch_mp_simple(bool scatter, bool norm, const float* vec, const float* X,
                            int64_t n_src, const int64_t* src_idx, const int64_t* perm,
                            const int64_t* row_ptr, float* out, int64_t n_items, int64_t n_edges,
                            int C, hipStream_t s) {
    const int64_t target = (int64_t)8 * blocks_per_xcd(C);
    int64_t per;
    if (scatter) {
        per = std::min<int64_t>(kScatterRows, std::max<int64_t>(1, ceil_div(n_items, target)));
    } else {
        per = std::max<int64_t>(1, ceil_div(ceil_div(n_edges, kBatch), target)) * kBatch;
    }
    const int64_t n_logical = scatter ? ceil_div(n_items, per) : ceil_div(n_edges, per);
    return launch_mp(scatter, norm, vec, X, n_src, src_idx, perm, row_ptr, nullptr, out, n_items,
                     n_edges, C, per, n_logical, s);
}

extern "C" int batteries_fused_sh_tp_simple(const float* edge_vectors, const float* node_features,
                                            const int64_t* source_idx, float* messages,
                                            int64_t N_nodes, int64_t N_edges, int C, int normalize,
                                            hipStream_t stream) {
    if (N_edges < 0 || N_nodes < 0 || C <= 0) return BM_ERR_ARG;
    if (N_edges == 0) return BM_OK;
    return launch_mp_simple(false, normalize != 0, edge_vectors, node_features, N_nodes, source_idx,
                            nullptr, nullptr, messages, 0, N_edges, C, stream);
}

extern "C" int batteries_sh_tp_scatter_csr(const float* edge_vectors, const float* node_features,
                                           const int64_t* source_idx, const int64_t* perm,
                                           const int64_t* row_ptr, float* node_output,
                                           int64_t N_src, int64_t N_dst, int64_t N_edges, int C,
                                           int normalize, hipStream_t stream) {
    if (N_src < 0 || N_dst < 0 || N_edges < 0 || C <= 0) return BM_ERR_ARG;
    if (N_dst == 0) return BM_OK;
    if (N_src == 0 && N_edges > 0) return BM_ERR_ARG;
    return launch_mp_simple(true, normalize != 0, edge_vectors, node_features,
                            std::max<int64_t>(N_src, 1), source_idx, perm, row_ptr, node_output,
                            N_dst, N_edges, C, stream);
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
                                       node_output, N_atoms, N_atoms, N_edges, C, 0, stream);
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
                                         N_atoms, N_atoms, N_edges, C_in, 0, stream);
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
        csr_sort_rows_kernel<<<(unsigned)ceil_div(N_atoms, 4), 256, 0, stream>>>(row_ptr, col_idx,
                                                                                N_atoms);
    }
    return (int)hipGetLastError();
}

// ---------------------------------------------------------------------------
// Destination schedule (the layout and the balancing are described in mp_schedule.h):
// degrees in processing order, their running sums and the group bounds, then one
// wave per group balances the group's workgroups, then edge_perm.
// ---------------------------------------------------------------------------
namespace bmhip {

// degm[m] = in-degree of destination order[m]
__global__ void sched_degm_kernel(const int64_t* __restrict__ row_ptr,
                                  const int64_t* __restrict__ order, int64_t* __restrict__ degm,
                                  int64_t n_dst) {
    const int64_t m = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (m >= n_dst) return;
    const int64_t d = order[m];
    degm[m] = (d >= 0 && d < n_dst) ? row_ptr[d + 1] - row_ptr[d] : 0;
}

// Group boundaries gb[0 .. 8G] in spatial positions: every group's target end (one
// thread per group), then one thread clamps the ends in order.
__global__ void sched_group_targets_kernel(const int64_t* __restrict__ cum, int64_t n_dst, int P,
                                           int Q, int64_t* __restrict__ gb) {
    const int G = (P + Q - 1) / Q;
    const int gi = blockIdx.x * blockDim.x + threadIdx.x;
    if (gi >= 8 * G) return;
    gb[gi + 1] = sched_group_target(gi, P, Q, n_dst, (double)cum[n_dst],
                                    [&](int64_t m) { return cum[m]; });
}

__global__ void sched_groups_kernel(int64_t n_dst, int P, int Q, int R, int64_t* __restrict__ gb) {
    if (blockIdx.x != 0 || threadIdx.x != 0) return;
    sched_clamp_groups(P, Q, R, n_dst, [&](int gi) { return gb[gi + 1]; },
                       [&](int i, int64_t v) { gb[i] = v; });
}

// The scan, sched_group_targets_kernel and sched_groups_kernel in one workgroup, for up
// to kPrepMaxDst destinations, fewer than 2^31 edges and up to kPrepMaxGroups groups:
// degm (from sched_degm_kernel, which spreads its scattered row_ptr reads over many
// compute units) is read with coalesced loads into LDS, summed there in int32 (and
// written out as cum, as the scan would), and the group targets and the clamp read the
// sums from LDS.  The sums are exact in int32, and the targets compare the same values
// in double as sched_group_targets_kernel, so gb is the same as the three kernels'.
constexpr int kPrepThreads = 1024;
constexpr int kPrepPer = 16;
constexpr int kPrepMaxDst = kPrepThreads * kPrepPer;
constexpr int kPrepMaxGroups = 2048;
__global__ __launch_bounds__(kPrepThreads) void sched_prep_kernel(
    const int64_t* __restrict__ degm, int64_t n_dst, int P, int Q, int R, int64_t* __restrict__ cum,
    int64_t* __restrict__ gb) {
    constexpr int kWaves = kPrepThreads / 64;
    __shared__ int sCum[kPrepMaxDst + 1];
    __shared__ int sPos[kPrepMaxGroups];
    __shared__ int wsum[kWaves];
    const int t = threadIdx.x, lane = t & 63, w = t >> 6;
    const int n = (int)n_dst;
    // coalesced: element j * kPrepThreads + t, all loads issued together
    {
        int64_t dv[kPrepPer];
#pragma unroll
        for (int j = 0; j < kPrepPer; ++j) {
            const int i = j * kPrepThreads + t;
            dv[j] = i < n ? degm[i] : 0;
        }
#pragma unroll
        for (int j = 0; j < kPrepPer; ++j) {
            const int i = j * kPrepThreads + t;
            if (i < n) sCum[i] = (int)dv[j];
        }
    }
    __syncthreads();
    // thread t sums its run i0 .. i0 + 15
    const int i0 = t * kPrepPer;
    int v[kPrepPer];
#pragma unroll
    for (int j = 0; j < kPrepPer; ++j) v[j] = i0 + j < n ? sCum[i0 + j] : 0;
    int s = 0;
#pragma unroll
    for (int j = 0; j < kPrepPer; ++j) s += v[j];
    int x = s;  // inclusive scan of the thread sums within the wave
#pragma unroll
    for (int off = 1; off < 64; off <<= 1) {
        const int y = __shfl_up(x, off, 64);
        if (lane >= off) x += y;
    }
    if (lane == 63) wsum[w] = x;
    __syncthreads();  // also: every thread has read its run before the sums overwrite it
    int before = 0, total = 0;
#pragma unroll
    for (int k = 0; k < kWaves; ++k) {
        const int ws = wsum[k];
        before += k < w ? ws : 0;
        total += ws;
    }
    int run = before + x - s;
#pragma unroll
    for (int j = 0; j < kPrepPer; ++j) {
        if (i0 + j < n) sCum[i0 + j] = run;
        run += v[j];
    }
    if (t == 0) sCum[n] = total;
    __syncthreads();
    // the sums to global memory for the balancing kernel (coalesced)
    for (int i = t; i <= n; i += kPrepThreads) cum[i] = sCum[i];
    const int G = (P + Q - 1) / Q;
    for (int gi = t; gi < 8 * G; gi += kPrepThreads)
        sPos[gi] = (int)sched_group_target(gi, P, Q, n_dst, (double)total,
                                           [&](int64_t m) { return (int64_t)sCum[m]; });
    __syncthreads();
    if (t == 0)
        sched_clamp_groups(P, Q, R, n_dst, [&](int gi) { return (int64_t)sPos[gi]; },
                           [&](int i, int64_t v) { gb[i] = v; });
}

// One workgroup of kSchedWaves waves per group.  TD: int when the edges number under
// 2^31 (every slot degree and workgroup load fits), else int64_t.
template <typename TD>
__global__ __launch_bounds__(64 * kSchedWaves) void sched_balance_kernel(
    const int64_t* __restrict__ degm, const int64_t* __restrict__ order,
    const int64_t* __restrict__ gb, const int64_t* __restrict__ cum, int64_t n_dst, int P, int Q,
    int R, int64_t* __restrict__ row_dst, int64_t* __restrict__ row_ptr_s) {
    __shared__ __attribute__((aligned(16))) SchedLds<TD> sL;
    const int v = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6), k = threadIdx.x & 63;
    const int gi = blockIdx.x;
    if (gi == 0 && threadIdx.x == 0) row_ptr_s[(int64_t)8 * P * R] = cum[n_dst];
    const SchedGroup s = sched_group(gi, P, Q);
    const int64_t s0 = gb[gi], s1 = gb[gi + 1];
    sched_balance_group<TD>(
        v, k, s.Qg, R, (int)(s1 - s0), cum[s0], s.b0, [&](int p) { return (TD)degm[s0 + p]; },
        [&](int p) -> int64_t {
            const int64_t o = order[s0 + p];
            return (o >= 0 && o < n_dst) ? o : -1;
        },
        row_dst, row_ptr_s, [](int64_t, int64_t) {}, sL);
}

// edge_perm over the scheduled slots: one wave per slot, a lane per edge of its row.
__global__ __launch_bounds__(256) void sched_edges_kernel(const int64_t* __restrict__ row_ptr,
                                                          const int64_t* __restrict__ col_perm,
                                                          const int64_t* __restrict__ row_dst,
                                                          const int64_t* __restrict__ row_ptr_s,
                                                          int64_t* __restrict__ edge_perm,
                                                          int64_t n_sched) {
    const int64_t q = (int64_t)blockIdx.x * 4 + (threadIdx.x >> 6);
    const int lane = threadIdx.x & 63;
    if (q >= n_sched) return;  // uniform per wave
    const int64_t d = row_dst[q];
    if (d < 0) return;
    const int64_t s0 = row_ptr[d], n = row_ptr[d + 1] - s0, o = row_ptr_s[q];
    for (int64_t i = lane; i < n; i += 64) edge_perm[o + i] = col_perm ? col_perm[s0 + i] : s0 + i;
}

}  // namespace bmhip

extern "C" int batteries_mp_schedule_shape(int64_t N_dst, int C, int* n_blocks,
                                           int* rows_per_block) {
    if (N_dst < 0 || C <= 0 || !n_blocks || !rows_per_block) return BM_ERR_ARG;
    int64_t P = blocks_per_xcd(C);
    int64_t R = std::max<int64_t>(1, ceil_div(N_dst, 8 * P));
    if (R + 1 <= kScatterRows) {
        R += 1;  // one slot of headroom: groups are cut by edges, not rows
    } else {
        R = kScatterRows;
        P = ceil_div(N_dst, 8 * (R - 1));
    }
    if (8 * P > INT32_MAX) return BM_ERR_ARG;
    *n_blocks = (int)(8 * P);
    *rows_per_block = (int)R;
    return BM_OK;
}

// degm [N_dst], cum [N_dst + 1], group bounds [8 G + 1] (G <= n_blocks / 8);
// N_dst <= n_blocks * rows_per_block.
extern "C" size_t batteries_mp_schedule_workspace_bytes(int n_blocks, int rows_per_block) {
    if (n_blocks <= 0 || rows_per_block <= 0) return 0;
    const size_t ns = (size_t)n_blocks * (size_t)rows_per_block;
    return sizeof(int64_t) * (2 * ns + (size_t)n_blocks + 2);
}

extern "C" int batteries_mp_schedule(const int64_t* row_ptr, const int64_t* col_perm,
                                     const int64_t* order, int64_t N_dst, int64_t N_edges, int C,
                                     int n_blocks, int rows_per_block, int64_t* row_ptr_s,
                                     int64_t* row_dst, int64_t* edge_perm, void* workspace,
                                     size_t workspace_bytes, hipStream_t stream) {
    if (N_dst < 0 || N_edges < 0 || C <= 0 || n_blocks <= 0 || n_blocks % 8 ||
        rows_per_block <= 0 || rows_per_block > kScatterRows)
        return BM_ERR_ARG;
    const int64_t n_sched = (int64_t)n_blocks * rows_per_block;
    if (n_sched < N_dst) return BM_ERR_ARG;
    if (!workspace || workspace_bytes < batteries_mp_schedule_workspace_bytes(n_blocks, rows_per_block))
        return BM_ERR_WORKSPACE;
    const int B = 256;
    const int P = n_blocks / 8;
    const int Q = schedule_group_size(n_blocks, C);
    const int G = (P + Q - 1) / Q;
    int64_t* degm = static_cast<int64_t*>(workspace);
    int64_t* cum = degm + N_dst;
    int64_t* gb = cum + N_dst + 1;
    int rc = BM_OK;
    if (N_dst > 0)
        sched_degm_kernel<<<(unsigned)ceil_div(N_dst, B), B, 0, stream>>>(row_ptr, order, degm, N_dst);
    if (N_dst <= kPrepMaxDst && N_edges < INT32_MAX && 8 * (int64_t)G <= kPrepMaxGroups) {
        sched_prep_kernel<<<1, kPrepThreads, 0, stream>>>(degm, N_dst, P, Q, rows_per_block, cum,
                                                          gb);
    } else {
        rc = batteries_exclusive_scan_i64(degm, cum, N_dst, stream);
        if (rc != BM_OK) return rc;
        sched_group_targets_kernel<<<(unsigned)ceil_div(8 * (int64_t)G, 64), 64, 0, stream>>>(
            cum, N_dst, P, Q, gb);
        sched_groups_kernel<<<1, 64, 0, stream>>>(N_dst, P, Q, rows_per_block, gb);
    }
    const unsigned nbal = (unsigned)(8 * G);
    if (N_edges < INT32_MAX)
        sched_balance_kernel<int><<<nbal, 64 * kSchedWaves, 0, stream>>>(
            degm, order, gb, cum, N_dst, P, Q, rows_per_block, row_dst, row_ptr_s);
    else
        sched_balance_kernel<int64_t><<<nbal, 64 * kSchedWaves, 0, stream>>>(
            degm, order, gb, cum, N_dst, P, Q, rows_per_block, row_dst, row_ptr_s);
    sched_edges_kernel<<<(unsigned)ceil_div(n_sched, 4), 256, 0, stream>>>(row_ptr, col_perm, row_dst,
                                                                          row_ptr_s, edge_perm, n_sched);
    return (int)hipGetLastError();
}

extern "C" int batteries_sh_tp_scatter_scheduled(const float* edge_vectors,
                                                 const float* node_features,
                                                 const int64_t* source_idx,
                                                 const int64_t* row_ptr_s,
                                                 const int64_t* edge_perm, const int64_t* row_dst,
                                                 int n_blocks, int rows_per_block,
                                                 float* node_output, int64_t N_src,
                                                 int64_t N_edges, int C, int normalize,
                                                 hipStream_t stream) {
    if (N_src < 0 || N_edges < 0 || C <= 0 || n_blocks <= 0 || n_blocks % 8 || rows_per_block <= 0)
        return BM_ERR_ARG;
    if (N_src == 0 && N_edges > 0) return BM_ERR_ARG;
    const int64_t n_sched = (int64_t)n_blocks * rows_per_block;
    return launch_mp(true, normalize != 0, edge_vectors, node_features, std::max<int64_t>(N_src, 1),
                     source_idx, edge_perm, row_ptr_s, row_dst, node_output, n_sched, N_edges, C,
                     rows_per_block, n_blocks, stream);
}

extern "C" int batteries_sh_tp_scatter_scheduled_chsplit(
    const float* edge_vectors, const float* node_features, const int64_t* source_idx,
    const int64_t* row_ptr_s, const int64_t* edge_perm, const int64_t* row_dst, int n_blocks,
    int rows_per_block, float* node_output, int64_t N_src, int64_t N_edges, int C, int normalize,
    hipStream_t stream) {
    if (N_src < 0 || N_edges < 0 || C <= 0 || n_blocks <= 0 || n_blocks % 8 || rows_per_block <= 0)
        return BM_ERR_ARG;
    if (N_src == 0 && N_edges > 0) return BM_ERR_ARG;
    const int64_t n_sched = (int64_t)n_blocks * rows_per_block;
    const int64_t n_src = std::max<int64_t>(N_src, 1);
    const bool fits = C % kChanGroup == 0 && (int64_t)C * 64 <= kMaxBufferStride && edge_perm &&
                      n_src * (int64_t)C * 64 <= (int64_t)INT32_MAX;
    if (!fits)  // shapes the channel-half kernel does not take: the channel-split kernel
        return launch_mp(true, normalize != 0, edge_vectors, node_features, n_src, source_idx,
                         edge_perm, row_ptr_s, row_dst, node_output, n_sched, N_edges, C,
                         rows_per_block, n_blocks, stream);
    return launch_mp_half(normalize != 0, edge_vectors, node_features, n_src, source_idx, edge_perm,
                          row_ptr_s, row_dst, node_output, n_sched, C, rows_per_block, n_blocks,
                          stream);
}

// ---------------------------------------------------------------------------
// Weighted scatter: one W [34, C_in, C_out] shared by every edge,
//   out[d, co, o] = sum_{e -> d} TP_W(X[src_e], Y(v_e))[co, o].
// Because W is shared, the sum over the edges of d moves in front of both the
// CG contraction and the channel mixing:
//   S[d, ci, a, b] = sum_{e -> d} X[src_e, ci, a] Y_e[b]              MFMA 16x16x4 over edges
//   T[d, q, ci]    = sum_{(a, b) in slot q} c S[d, ci, a, b]           CG table, VALU
//   out[d, co, o]  = sum_{q -> o} sum_ci W[p(q), ci, co] T[d, q, ci]   MFMA 4x4x1 (16 blocks)
// Work: 2 * 256 * C_in flops per edge (S), 2 * 611 * C_in + 2 * 156 * C_in * C_out per
// destination (T, mixing).
//
// One workgroup (4 waves) owns 4 destinations at consecutive positions of the
// processing order and 64 output channels, and walks C_in in 16-channel chunks.
// Per chunk:
//   S phase: wave w sums channels c0 + 4w .. c0 + 4w + 3 of all four destinations
//     (every wave does the same work), four edges per k-step:  MFMA j takes
//     A[i][g] = X[src of edge g][c0 + 4w + i / 4][4 (i % 4) + j] (one float4 gather per
//     lane) and B[g][i] = Y[edge g][i], so lane (g, i) ends with S[ch = 4w + g][a = 4r + j]
//     [b = i] in element r of acc[j]; each destination's S goes to LDS row (ch, dd).
//   contraction + mixing: lane l = 4 ch + dd reads row (ch, dd), contracts the CG blocks
//     (l1, l2) of its wave and, for each slot q of a path p, issues 16 MFMAs
//     acc[out(q)] += T[q][dd'][c0 + k] (x) W[p][c0 + k][co0 + lane'], k = 0..15, where the
//     T operand of block k (lanes 4k .. 4k + 3: channel k, destinations 0..3) is broadcast
//     to all 16 blocks (CBSZ = 4, ABID = k) and block b's B operand is W for output
//     channels co0 + 4b .. 4b + 3.  T never leaves registers.
// The waves' CG blocks carry 39 slots each (624 MFMAs per chunk); each path's W rows
// (16 x 256 contiguous bytes) are loaded one path ahead.  At the end the four waves'
// accumulators (lane l: destination r, output channel co0 + l, output component o) are
// summed in LDS in a fixed order, and wave r stores destination r: deterministic, no
// atomics.
// ---------------------------------------------------------------------------
namespace bmhip {

__device__ __forceinline__ int64_t uniform64(int64_t v) {
    const uint64_t u = (uint64_t)v;
    const uint32_t lo = __builtin_amdgcn_readfirstlane((uint32_t)u);
    const uint32_t hi = __builtin_amdgcn_readfirstlane((uint32_t)(u >> 32));
    return (int64_t)(((uint64_t)hi << 32) | lo);
}

// S of one (channel, destination) in LDS: 16 rows b of 16 a, the four 16-byte quads of
// row b at positions quad ^ ps_swz(b), rows (ch, dd) at ch * 4 + dd, kPsStride floats
// apart.  The S-phase writes (8 lanes = 8 values of b) and the contraction's reads
// (8 lanes = 8 consecutive rows) are then free of bank conflicts.
constexpr int kPsStride = 260;
__host__ __device__ constexpr int ps_swz(int b) { return (b >> 1) & 3; }

// CG blocks (l1, l2) of each wave, 39 slots each (16 + 15 + 5 + 3, 16 + 15 + 7 + 1,
// 15 + 15 + 9, 12 + 12 + 7 + 5 + 3); CG terms 130, 172, 200, 109.
constexpr int kWfBlocks[4][5][2] = {{{2, 2}, {1, 2}, {0, 2}, {0, 1}, {-1, -1}},
                                    {{3, 3}, {2, 1}, {0, 3}, {0, 0}, {-1, -1}},
                                    {{2, 3}, {3, 2}, {1, 1}, {-1, -1}, {-1, -1}},
                                    {{1, 3}, {3, 1}, {3, 0}, {2, 0}, {1, 0}}};

// The paths of wave W in processing order (blocks in kWfBlocks order, paths in path order).
constexpr int wf_num_paths(int W) {
    int n = 0;
    for (int k = 0; k < 5; ++k)
        for (int p = 0; p < kNumPaths; ++p)
            if (kWfBlocks[W][k][0] >= 0 && kPathL[p][0] == kWfBlocks[W][k][0] &&
                kPathL[p][1] == kWfBlocks[W][k][1])
                ++n;
    return n;
}
constexpr int wf_path(int W, int i) {
    for (int k = 0; k < 5; ++k)
        for (int p = 0; p < kNumPaths; ++p)
            if (kWfBlocks[W][k][0] >= 0 && kPathL[p][0] == kWfBlocks[W][k][0] &&
                kPathL[p][1] == kWfBlocks[W][k][1]) {
                if (i == 0) return p;
                --i;
            }
    return -1;
}
// does path i of wave W start a new CG block (l1, l2)?
constexpr bool wf_new_block(int W, int i) {
    if (i == 0) return true;
    const int p = wf_path(W, i), q = wf_path(W, i - 1);
    return kPathL[p][0] != kPathL[q][0] || kPathL[p][1] != kPathL[q][1];
}

// W rows of path p for the 16 channels of chunk c0: w[k] = W[p][min(c0 + k, cin - 1)][co]
// (lane offset woff = the lane's output channel, clamped, in bytes).
__device__ __forceinline__ void wf_load_w(__amdgpu_buffer_rsrc_t wr, int woff, int p, int c0,
                                          int cin, int cout, float (&w)[16]) {
#pragma unroll
    for (int k = 0; k < 16; ++k)
        w[k] = buffer_ld(wr, woff, (p * cin + min(c0 + k, cin - 1)) * cout * 4);
}

// Slots of wave W's paths before path i (its T values sit in tq[wf_slot_base(W, i) ..]).
constexpr int wf_slot_base(int W, int i) {
    int n = 0;
    for (int k = 0; k < i; ++k) n += 2 * kPathL[wf_path(W, k)][2] + 1;
    return n;
}
// Depth of the W ring of the mixing step: path i + kWfAhead - 1's rows are loaded when
// path i's products start.
constexpr int kWfAhead = 2;

// Contraction of wave W's CG blocks for the lane's (channel, destination) row: T of every
// slot of the wave's paths into tq, in path order.
template <int W>
__device__ __forceinline__ void wf_contract(const float* sSrow,
                                            float (&tq)[wf_slot_base(W, wf_num_paths(W))]) {
    constexpr int NP = wf_num_paths(W);
    float s[7][7];  // S[a in l1][b in l2] of the current block
    static_for<NP>([&](auto ii) {
        constexpr int i = decltype(ii)::value;
        constexpr int p = wf_path(W, i);
        constexpr int L1 = kPathL[p][0], L2 = kPathL[p][1], LO = kPathL[p][2];
        constexpr int a0 = L1 * L1, na = 2 * L1 + 1, b0 = L2 * L2, nb = 2 * L2 + 1;
        if constexpr (wf_new_block(W, i)) {
            // one block's S values live at a time: no reads hoisted from the next block
            __builtin_amdgcn_sched_barrier(0);
            constexpr int qa0 = a0 / 4, qa1 = (a0 + na - 1) / 4;
            static_for<nb>([&](auto bb) {
                constexpr int b = b0 + decltype(bb)::value;
                static_for<qa1 - qa0 + 1>([&](auto qq) {
                    constexpr int qa = qa0 + decltype(qq)::value;
                    const float4 v =
                        *reinterpret_cast<const float4*>(sSrow + b * 16 + (qa ^ ps_swz(b)) * 4);
                    const float vv[4] = {v.x, v.y, v.z, v.w};
                    static_for<4>([&](auto jj) {
                        constexpr int j = decltype(jj)::value;
                        constexpr int a = 4 * qa + j;
                        if constexpr (a >= a0 && a < a0 + na) s[a - a0][b - b0] = vv[j];
                    });
                });
            });
        }
        constexpr int base = wf_slot_base(W, i);
        static_for<2 * LO + 1>([&](auto m) { tq[base + decltype(m)::value] = 0.0f; });
        static_for<kPathEntry[p + 1] - kPathEntry[p]>([&](auto kk) {
            constexpr CGEntry e = kCG[kPathEntry[p] + decltype(kk)::value];
            constexpr int m = e.q - kPathSlot[p];
            tq[base + m] = fmaf(e.c, s[e.a - a0][e.b - b0], tq[base + m]);
        });
    });
}

// Mixing MFMAs of every slot of wave W's paths.  wbuf[i % kWfAhead] holds path i's W rows;
// paths 0 .. kWfAhead - 2 were loaded before the call, path i + kWfAhead - 1's rows are
// loaded when path i's products start.
template <int W>
__device__ __forceinline__ void wf_mix(__amdgpu_buffer_rsrc_t wr, int woff, int c0, int cin,
                                       int cout, const float (&tq)[wf_slot_base(W, wf_num_paths(W))],
                                       float (&wbuf)[kWfAhead][16], v4f (&acc)[16]) {
    constexpr int NP = wf_num_paths(W);
    static_for<NP>([&](auto ii) {
        constexpr int i = decltype(ii)::value;
        constexpr int p = wf_path(W, i);
        constexpr int LO = kPathL[p][2];
        if constexpr (i + kWfAhead - 1 < NP) {
            constexpr int pn = wf_path(W, i + kWfAhead - 1);
            wf_load_w(wr, woff, pn, c0, cin, cout, wbuf[(i + kWfAhead - 1) % kWfAhead]);
            // keep the loads here: sunk to their uses, each would wait on its own round trip
            __builtin_amdgcn_sched_barrier(0);
        }
        constexpr int base = wf_slot_base(W, i);
        static_for<16>([&](auto kk) {
            constexpr int k = decltype(kk)::value;
            static_for<2 * LO + 1>([&](auto mm) {
                constexpr int m = decltype(mm)::value;
                acc[LO * LO + m] =
                    mfma_4x4_bcast<k>(tq[base + m], wbuf[i % kWfAhead][k], acc[LO * LO + m]);
            });
        });
    });
}

// Step t < T of a tile: the CSR slot of its first edge (returned) and the number of
// edges left from it (cnt; lane g takes edge g when g < cnt).  Destinations 0..3 hold
// dg0..dg3 edges from slots r00..r03; steps cum1, cum2, cum3 onward belong to
// destinations 1, 2, 3.  Values by argument, not through captured references: a select
// between variables in memory becomes a load through a selected pointer.
__device__ __forceinline__ int64_t wf_step_rows(int t, int cum1, int cum2, int cum3, int64_t r00,
                                                int64_t r01, int64_t r02, int64_t r03, int dg0,
                                                int dg1, int dg2, int dg3, int& cnt) {
    const bool b1 = t >= cum1, b2 = t >= cum2, b3 = t >= cum3;
    const int64_t r = b3 ? r03 : b2 ? r02 : b1 ? r01 : r00;
    const int c = b3 ? cum3 : b2 ? cum2 : b1 ? cum1 : 0;
    const int d = b3 ? dg3 : b2 ? dg2 : b1 ? dg1 : dg0;
    cnt = d - 4 * (t - c);
    return r + 4 * (t - c);
}

// W rows of wave W's first kWfAhead - 1 paths (the ones wf_mix expects in flight)
template <int W>
__device__ __forceinline__ void wf_load_first(__amdgpu_buffer_rsrc_t wr, int woff, int c0, int cin,
                                              int cout, float (&wbuf)[kWfAhead][16]) {
    static_for<kWfAhead - 1>([&](auto ii) {
        constexpr int i = decltype(ii)::value;
        constexpr int p = wf_path(W, i);
        wf_load_w(wr, woff, p, c0, cin, cout, wbuf[i]);
    });
}

// Contraction then mixing of wave W (T of its 39 slots in registers in between)
template <int W>
__device__ __forceinline__ void wf_contract_mix(const float* sSrow, __amdgpu_buffer_rsrc_t wr,
                                                int woff, int c0, int cin, int cout,
                                                float (&wbuf)[kWfAhead][16], v4f (&acc)[16]) {
    float tq[wf_slot_base(W, wf_num_paths(W))];
    wf_contract<W>(sSrow, tq);
    __builtin_amdgcn_sched_barrier(0);
    wf_mix<W>(wr, woff, c0, cin, cout, tq, wbuf, acc);
}

// Edges of one destination staged in LDS at a time (per wave): kWfSegSteps k-steps of 4
// edges, the Y and source-row value of each edge, transposed as [edge g][component b]
// [step] (and [edge g][step]) so that one 16-byte read gives a lane four steps' values;
// rows of 12 floats put the 16 lanes of a read pass in distinct banks.
constexpr int kWfSegSteps = 12;

// BUF: source-row gathers as raw buffer loads with 32-bit offsets (X under 2 GiB); the
// staged source values are then byte offsets of the rows, otherwise row indices.
template <bool BUF>
__global__ __launch_bounds__(256, 2) void mp_weighted_fused_kernel(
    const float* __restrict__ vec, const int64_t* __restrict__ src_idx,
    const int64_t* __restrict__ perm, const float* __restrict__ X, const float* __restrict__ Wt,
    const int64_t* __restrict__ row_ptr, const int64_t* __restrict__ order, float* __restrict__ out,
    int64_t n_dst, int cin, int cout, int64_t n_tiles, int normalize, uint32_t x_bytes) {
    __shared__ __attribute__((aligned(16))) float sS[64 * kPsStride];
    __shared__ __attribute__((aligned(16))) float sYall[4][4 * 16 * kWfSegSteps];
    __shared__ __attribute__((aligned(16))) int sSrcAll[4][4 * kWfSegSteps];
    const int64_t per_xcd = (n_tiles + 7) / 8;
    const int64_t tile = (int64_t)(blockIdx.x & 7) * per_xcd + (blockIdx.x >> 3);
    if (tile >= n_tiles) return;
    const int lane = threadIdx.x & 63, g = lane >> 4, i16 = lane & 15;
    const int w = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);  // wave-uniform
    const int co0 = blockIdx.y * 64;
    const int nchunk = (cin + 15) >> 4;
    float* sY = sYall[w];
    int* sSrc = sSrcAll[w];

    // destination w of the tile (position 4 tile + w of the processing order): CSR rows
    // [r0, r0 + deg); the output is written by wave w, so every wave keeps its own
    int64_t dst = -1, r0 = 0;
    int deg = 0;
    {
        const int64_t pos = tile * 4 + w;
        int64_t a = 0, b = 0;
        if (pos < n_dst) {
            dst = order ? order[pos] : pos;
            if (dst >= 0 && dst < n_dst) {  // an order entry out of range sums no edges
                a = row_ptr[dst];
                b = row_ptr[dst + 1];
            } else {
                dst = -1;
            }
        }
        dst = uniform64(dst);
        r0 = uniform64(a);
        deg = __builtin_amdgcn_readfirstlane((int)(b - a));
    }
    // k-steps of 4 edges, padded to a multiple of 2 (the unroll of the pipeline below);
    // padding steps and lanes past the last edge have Y = 0 and source 0 (a valid row), and
    // the padding step runs no MFMAs
    const int nst = (deg + 3) >> 2;
    const int nst2 = (nst + 1) & ~1;
    const int nseg = (nst2 + kWfSegSteps - 1) / kWfSegSteps;  // 0: no edges

    const uint32_t row_bytes = (uint32_t)cin * 64u;
    // steps [s0, s0 + len) of this wave's destination into its LDS area: lane l takes edge
    // 4 s0 + l (len <= kWfSegSteps = 12, so 48 lanes); read back by the same wave only
    auto stage = [&](int s0, int len) {
        if (lane < 4 * len) {
            const int sl = lane >> 2, ge = lane & 3;
            const int k = 4 * s0 + lane;  // edge index within the destination
            float Y[16];
            int src = 0;
            if (k < deg) {
                const int64_t slot = r0 + k;
                const int64_t e = perm ? perm[slot] : slot;
                float x = vec[e * 3 + 0], y = vec[e * 3 + 1], z = vec[e * 3 + 2];
                if (normalize) normalize3(x, y, z);
                sh_forward_l3(x, y, z, Y);
                src = (int)src_idx[e];
            } else {
#pragma unroll
                for (int q = 0; q < 16; ++q) Y[q] = 0.f;
            }
#pragma unroll
            for (int q = 0; q < 16; ++q) sY[(ge * 16 + q) * kWfSegSteps + sl] = Y[q];
            sSrc[ge * kWfSegSteps + sl] = BUF ? (int)((uint32_t)src * row_bytes) : src;
        }
        // the wave's own LDS writes are complete before its reads below
        __builtin_amdgcn_s_waitcnt(0xc07f);  // lgkmcnt(0)
        __builtin_amdgcn_wave_barrier();
    };
    const __amdgpu_buffer_rsrc_t xr = __builtin_amdgcn_make_buffer_rsrc(
        const_cast<float*>(X), (short)0, BUF ? (int)x_bytes : 0, kBufferDword3);
    // lane (g, i16) gathers channels c0 + 4t + i16 / 4 (t = 0..3, clamped to the last channel),
    // components 4 (i16 % 4) .. 4 (i16 % 4) + 3 of the source row of its edge g
    auto gather4 = [&](int c0, int sv, float4 (&x)[4]) {
#pragma unroll
        for (int t = 0; t < 4; ++t) {
            const int off = min(c0 + 4 * t + (i16 >> 2), cin - 1) * 64 + (i16 & 3) * 16;
            if constexpr (BUF) {
                x[t] = buffer_ld4(xr, sv + off, 0);
            } else {
                x[t] = *reinterpret_cast<const float4*>(reinterpret_cast<const char*>(X) +
                                                        (int64_t)sv * row_bytes + off);
            }
        }
    };
    auto ld_y = [&](int col) {  // Y[edge g][b = i16] of steps col .. col + 3
        return *reinterpret_cast<const float4*>(sY + (g * 16 + i16) * kWfSegSteps + col);
    };
    auto ld_s = [&](int col) {  // source values of edge g of steps col .. col + 3
        return *reinterpret_cast<const int4*>(sSrc + g * kWfSegSteps + col);
    };

    // S rows of a destination without edges are zero for every chunk
    if (deg == 0) {
#pragma unroll
        for (int t = 0; t < 4; ++t) {
            float* row = sS + ((4 * t + g) * 4 + w) * kPsStride + i16 * 16;
#pragma unroll
            for (int r = 0; r < 4; ++r)
                *reinterpret_cast<float4*>(row + r * 4) = make_float4(0.f, 0.f, 0.f, 0.f);
        }
    }

    const __amdgpu_buffer_rsrc_t wr = buffer_rsrc(Wt, (uint32_t)((int64_t)kNumPaths * cin * cout * 4));
    const int woff = min(co0 + lane, cout - 1) * 4;
    const v4f zero4 = {0.f, 0.f, 0.f, 0.f};
    v4f macc[16];
#pragma unroll
    for (int o = 0; o < 16; ++o) macc[o] = zero4;
    float wbuf[kWfAhead][16];

    if (nseg == 1) stage(0, nst2);

    for (int c = 0; c < nchunk; ++c) {
        const int c0 = c * 16;
        if (nseg > 0) {
            // S phase: acc[t][j] accumulates S[ch = 4t + g][a = 4r + j][b = i16] (element r)
            // of destination w over its edges, four per k-step (16 MFMAs).  Steps run in
            // pairs through two pipeline stages with static register names: entering step
            // s, stage s % 2 holds its gathers (issued two steps earlier); y4/s4 hold the
            // Y and source values of the current block of four steps.
            v4f acc[4][4];
#pragma unroll
            for (int t = 0; t < 4; ++t)
#pragma unroll
                for (int j = 0; j < 4; ++j) acc[t][j] = zero4;
            for (int sg = 0; sg < nseg; ++sg) {
                const int s0 = sg * kWfSegSteps;
                const int len = min(kWfSegSteps, nst2 - s0);  // even
                const int lenr = min(kWfSegSteps, nst - s0);  // steps with edges
                if (nseg > 1) stage(s0, len);
                float4 xa[4], xb[4];
                int4 sv = ld_s(0);
                float4 yv = ld_y(0);
                gather4(c0, sv.x, xa);
                gather4(c0, len > 1 ? sv.y : 0, xb);
                // one step from stage x, whose refill is step s + 2 (source value snext); the
                // padding step of an odd step count (live false) issues its gathers but no MFMAs
                auto step = [&](float4 (&x)[4], float y, int snext, bool refill, bool live) {
                    float4 xs[4];
#pragma unroll
                    for (int t = 0; t < 4; ++t) xs[t] = x[t];
                    gather4(c0, refill ? snext : 0, x);
                    if (live)
#pragma unroll
                    for (int t = 0; t < 4; ++t) {
                        acc[t][0] = mfma1(xs[t].x, y, acc[t][0]);
                        acc[t][1] = mfma1(xs[t].y, y, acc[t][1]);
                        acc[t][2] = mfma1(xs[t].z, y, acc[t][2]);
                        acc[t][3] = mfma1(xs[t].w, y, acc[t][3]);
                    }
                };
                for (int s = 0; s < len; s += 4) {
                    // steps s .. s + 3 (the last block may hold only s, s + 1)
                    const int4 svn = s + 4 < len ? ld_s(s + 4) : make_int4(0, 0, 0, 0);
                    const float4 yn = s + 4 < len ? ld_y(s + 4) : make_float4(0.f, 0.f, 0.f, 0.f);
                    step(xa, yv.x, sv.z, s + 2 < len, true);
                    step(xb, yv.y, sv.w, s + 3 < len, s + 1 < lenr);
                    if (s + 2 < len) {
                        step(xa, yv.z, svn.x, s + 4 < len, true);
                        step(xb, yv.w, svn.y, s + 5 < len, s + 3 < lenr);
                    }
                    sv = svn;
                    yv = yn;
                }
            }
            // S of destination w to LDS rows (ch, w); channels past C_in are zero
#pragma unroll
            for (int t = 0; t < 4; ++t) {
                const bool cok = c0 + 4 * t + g < cin;
                float* row = sS + ((4 * t + g) * 4 + w) * kPsStride + i16 * 16;
#pragma unroll
                for (int r = 0; r < 4; ++r)
                    *reinterpret_cast<float4*>(row + ((r ^ ps_swz(i16)) * 4)) =
                        cok ? make_float4(acc[t][0][r], acc[t][1][r], acc[t][2][r], acc[t][3][r])
                            : make_float4(0.f, 0.f, 0.f, 0.f);
            }
        }
        // the first paths' W rows of this chunk, in flight during the barrier wait
        switch (w) {
            case 0: wf_load_first<0>(wr, woff, c0, cin, cout, wbuf); break;
            case 1: wf_load_first<1>(wr, woff, c0, cin, cout, wbuf); break;
            case 2: wf_load_first<2>(wr, woff, c0, cin, cout, wbuf); break;
            default: wf_load_first<3>(wr, woff, c0, cin, cout, wbuf); break;
        }
        __syncthreads();  // S of all four destinations is in LDS
        const float* sSrow = sS + lane * kPsStride;
        switch (w) {
            case 0: wf_contract_mix<0>(sSrow, wr, woff, c0, cin, cout, wbuf, macc); break;
            case 1: wf_contract_mix<1>(sSrow, wr, woff, c0, cin, cout, wbuf, macc); break;
            case 2: wf_contract_mix<2>(sSrow, wr, woff, c0, cin, cout, wbuf, macc); break;
            default: wf_contract_mix<3>(sSrow, wr, woff, c0, cin, cout, wbuf, macc); break;
        }
        __syncthreads();  // S is rewritten by the next chunk
    }

    // lane l of wave w holds, for output component o, macc[o][r] = partial out[dest r]
    // [co0 + l][o]; the waves' partials meet in LDS and wave r sums them in wave order
    float* sR = sS;  // [wave][r][o][lane]
#pragma unroll
    for (int o = 0; o < 16; ++o)
#pragma unroll
        for (int r = 0; r < 4; ++r) sR[((w * 4 + r) * 16 + o) * 64 + lane] = macc[o][r];
    __syncthreads();
    const int64_t d = dst;
    const int co = co0 + lane;
    if (d >= 0 && co < cout) {
        float v[16];
#pragma unroll
        for (int o = 0; o < 16; ++o) {
            float sum = sR[((0 * 4 + w) * 16 + o) * 64 + lane];
#pragma unroll
            for (int ww = 1; ww < 4; ++ww) sum += sR[((ww * 4 + w) * 16 + o) * 64 + lane];
            v[o] = sum;
        }
        float4* dstp = reinterpret_cast<float4*>(out + (d * cout + co) * 16);
#pragma unroll
        for (int q = 0; q < 4; ++q) dstp[q] = make_float4(v[4 * q], v[4 * q + 1], v[4 * q + 2], v[4 * q + 3]);
    }
}

// ---------------------------------------------------------------------------
// Processing order for the weighted scatter.  The kernel deals tile k of XCD x (4
// destinations at positions 4 (x P + k) .. + 3 of the order, P = ceil(tiles / 8)) to its
// workgroup x + 8 k, and the hardware starts workgroups in index order as slots free up.
// Two reorderings inside each XCD's range of the spatial order (the ranges, and so the
// XCDs' L2 footprints, stay as they were):
//  - within each window of 16 consecutive positions (4 tiles) the destinations are sorted
//    by decreasing edge count (ties by position), so a tile's four destinations, one per
//    wave in the edge-sum phase, have similar counts and its waves meet at the barrier
//    after that phase with less waiting;
//  - the tiles are then sorted by decreasing edge count (ties by position): at configs[3]
//    1250 tiles fill 512 slots 2.44 times, and starting the long tiles first leaves short
//    ones for the last partial round (largest-first list scheduling).
// One workgroup per XCD range, everything in LDS; a partial last tile keeps its place.
// ---------------------------------------------------------------------------
constexpr int kTileSortMax = 2048;  // tiles per XCD range sorted in LDS (more: order copied)
constexpr int kOrderWindow = 16;    // positions per degree-sorted window

__global__ __launch_bounds__(1024) void wf_tile_order_kernel(const int64_t* __restrict__ order,
                                                             const int64_t* __restrict__ row_ptr,
                                                             int64_t n_dst, int64_t per_xcd,
                                                             int64_t* __restrict__ out) {
    __shared__ uint64_t key[kTileSortMax];
    __shared__ int sdeg[4 * kTileSortMax];  // edge count of each position of the range
    __shared__ int spos[4 * kTileSortMax];  // window-sorted positions (relative to the range)
    const int64_t ntile = (n_dst + 3) / 4;
    const int64_t t0 = (int64_t)blockIdx.x * per_xcd;
    const int64_t t1 = min(ntile, t0 + per_xcd);
    if (t0 >= t1) return;
    // the last tile of all stays in place when it is partial
    const int64_t tsort = (t1 == ntile && (n_dst & 3)) ? t1 - 1 : t1;
    const int T = (int)(tsort - t0);
    const int NP = 4 * T;
    auto dst_at = [&](int64_t pos) -> int64_t { return order ? order[pos] : pos; };
    for (int q = threadIdx.x; q < NP; q += blockDim.x) {
        const int64_t d = dst_at(4 * t0 + q);
        // an order entry out of range sums no edges
        sdeg[q] = (d >= 0 && d < n_dst) ? (int)min<int64_t>(row_ptr[d + 1] - row_ptr[d], INT32_MAX)
                                        : 0;
    }
    __syncthreads();
    for (int q = threadIdx.x; q < NP; q += blockDim.x) {
        const int wb = q - q % kOrderWindow, we = min(wb + kOrderWindow, NP);
        const int dq = sdeg[q];
        int rank = 0;
        for (int r = wb; r < we; ++r) {
            const int dr = sdeg[r];
            rank += (dr > dq) || (dr == dq && r < q);
        }
        spos[wb + rank] = q;
    }
    __syncthreads();
    int Tp = 1;
    while (Tp < T) Tp <<= 1;
    for (int k = threadIdx.x; k < Tp; k += blockDim.x) {
        uint64_t v = ~0ull;
        if (k < T) {
            int64_t w = 0;
            for (int i = 0; i < 4; ++i) w += sdeg[spos[4 * k + i]];
            const uint32_t wc = (uint32_t)min<int64_t>(w, 0xfffffffell);
            v = ((uint64_t)(0xffffffffu - wc) << 32) | (uint32_t)k;
        }
        key[k] = v;
    }
    __syncthreads();
    for (int size = 2; size <= Tp; size <<= 1) {
        for (int stride = size >> 1; stride > 0; stride >>= 1) {
            for (int i = threadIdx.x; i < Tp; i += blockDim.x) {
                const int j = i ^ stride;
                if (j > i) {
                    const bool up = (i & size) == 0;
                    const uint64_t a = key[i], b = key[j];
                    if ((a > b) == up) {
                        key[i] = b;
                        key[j] = a;
                    }
                }
            }
            __syncthreads();
        }
    }
    for (int64_t q = threadIdx.x; q < 4 * (t1 - t0); q += blockDim.x) {
        const int64_t j = q >> 2;  // tile position in the range
        const int64_t pos = j < T ? 4 * t0 + spos[4 * (int)(uint32_t)key[j] + (int)(q & 3)]
                                  : 4 * t0 + q;
        const int64_t opos = 4 * t0 + q;
        if (opos < n_dst) out[opos] = pos < n_dst ? dst_at(pos) : -1;
    }
}

__global__ void wf_copy_order_kernel(const int64_t* __restrict__ order, int64_t n,
                                     int64_t* __restrict__ out) {
    const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (i < n) out[i] = order ? order[i] : i;
}

}  // namespace bmhip

extern "C" int batteries_weighted_tile_order(const int64_t* order, const int64_t* row_ptr,
                                            int64_t N_dst, int64_t* order_out, hipStream_t stream) {
    if (N_dst < 0 || !row_ptr || !order_out) return BM_ERR_ARG;
    if (N_dst == 0) return BM_OK;
    const int64_t ntile = ceil_div(N_dst, 4);
    const int64_t per_xcd = ceil_div(ntile, 8);
    if (per_xcd <= kTileSortMax)
        wf_tile_order_kernel<<<8, 1024, 0, stream>>>(order, row_ptr, N_dst, per_xcd, order_out);
    else
        wf_copy_order_kernel<<<(unsigned)ceil_div(N_dst, 256), 256, 0, stream>>>(order, N_dst,
                                                                                 order_out);
    return (int)hipGetLastError();
}

extern "C" size_t batteries_sh_tp_scatter_weighted_workspace_bytes(int64_t N_dst, int64_t N_edges,
                                                                   int C_in, int C_out) {
    (void)N_dst;
    (void)N_edges;
    (void)C_in;
    (void)C_out;
    return 0;  // the fused kernel keeps everything on chip
}

extern "C" int batteries_sh_tp_scatter_weighted(
    const float* edge_vectors, const float* node_features, const float* weights,
    const int64_t* source_idx, const int64_t* perm, const int64_t* row_ptr, const int64_t* order,
    float* node_output, int64_t N_src, int64_t N_dst, int64_t N_edges, int C_in, int C_out,
    int normalize, void* workspace, size_t workspace_bytes, hipStream_t stream) {
    (void)workspace;
    (void)workspace_bytes;
    if (N_src < 0 || N_dst < 0 || N_edges < 0 || C_in <= 0 || C_out <= 0) return BM_ERR_ARG;
    if (N_edges > 0 && N_src == 0) return BM_ERR_ARG;
    if (N_dst == 0) return BM_OK;
    if (N_src > INT32_MAX) return BM_ERR_ARG;  // int32 source rows in LDS
    if ((int64_t)kNumPaths * C_in * C_out * 4 > INT32_MAX) return BM_ERR_ARG;  // W via 32-bit offsets
    if (ceil_div(C_out, 64) > 65535) return BM_ERR_ARG;
    if ((reinterpret_cast<uintptr_t>(node_features) | reinterpret_cast<uintptr_t>(node_output)) & 15)
        return BM_ERR_ARG;
    const int64_t n_tiles = ceil_div(N_dst, 4);
    const int64_t grid = ceil_div(n_tiles, 8) * 8;
    if (grid > INT32_MAX) return BM_ERR_ARG;
    const int64_t xb = std::max<int64_t>(N_src, 1) * (int64_t)C_in * 64;
    const bool buf = xb <= (int64_t)INT32_MAX;
    dim3 g((unsigned)grid, (unsigned)ceil_div(C_out, 64), 1);
    if (buf)
        mp_weighted_fused_kernel<true><<<g, 256, 0, stream>>>(
            edge_vectors, source_idx, perm, node_features, weights, row_ptr, order, node_output,
            N_dst, C_in, C_out, n_tiles, normalize, (uint32_t)xb);
    else
        mp_weighted_fused_kernel<false><<<g, 256, 0, stream>>>(
            edge_vectors, source_idx, perm, node_features, weights, row_ptr, order, node_output,
            N_dst, C_in, C_out, n_tiles, normalize, 0u);
    return (int)hipGetLastError();
}
