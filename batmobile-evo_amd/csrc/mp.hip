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

// Phase 1 of a batch: lane j < nb of wave w builds rows 4w..4w+3 of the
// operator of its edge into sM (no global memory access: the edge was loaded
// into registers during the previous batch).
template <bool NORM>
__device__ __forceinline__ void phase1_build(EdgeRec r, int nb, float* sM) {
    const int lane = threadIdx.x & 63;
    const int w = threadIdx.x >> 6;
    if (lane < nb) {
        float x = r.x, y = r.y, z = r.z;
        if constexpr (NORM) {
            // v / max(|v|, 1e-10) with one reciprocal square root (about 1 ulp)
            const float inv = __builtin_amdgcn_rsqf(fmaxf(x * x + y * y + z * z, 1e-20f));
            x *= inv;
            y *= inv;
            z *= inv;
        }
        float Y[16];
        sh_forward<3>(x, y, z, Y);
        float* sMj = sM + lane * kMStride;
        switch (w) {
            case 0: build_rows<0>(Y, sMj); break;
            case 1: build_rows<1>(Y, sMj); break;
            case 2: build_rows<2>(Y, sMj); break;
            default: build_rows<3>(Y, sMj); break;
        }
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
// Same operator/MFMA scheme as above, arranged so that the compiler can keep
// kRing gathers in flight.  On gfx9 loads and stores share one counter, and
// with a store pending the compiler treats the counter as out of order and
// drains every outstanding gather before the next use; a gather issued under a
// data-dependent condition has the same effect.  Hence the edge loop has
// neither:
//   - every batch is kSBatch edges fully unrolled, and every edge issues the
//     gather for the edge kRing positions ahead (past the block's last edge it
//     gathers row 0 of the same tensor, a valid address whose value is never
//     used: edges past the end only touch the accumulator after the block's
//     last row has been staged);
//   - a finished row is staged in LDS (the workgroup owns at most kScatterRows
//     rows) and written to HBM only where no gather is in flight: at the start
//     of the last batch and at the end.
// The per-edge control is one scalar bit test: `ends` (a 64-bit mask per batch,
// built with scalar arithmetic from the row ends) marks the edges that close a
// row; there the accumulator is staged and reset to zero.
// ---------------------------------------------------------------------------
constexpr int kSBatch = 32;       // edges per batch (operators in LDS)
constexpr int kRing = 32;         // gathers in flight per lane (edges ahead)
constexpr int kScatterRows = 11;  // row slots per workgroup (all staged in LDS)
constexpr int kLdsAhead = 3;      // operator rows read from LDS this many edges ahead

template <bool NORM, bool BUF, bool PERM>
__global__ __launch_bounds__(kMpBlock) void mp_scatter_kernel(
    const float* __restrict__ vec, const float* __restrict__ X, const int64_t* __restrict__ src_idx,
    const int64_t* __restrict__ perm, const int64_t* __restrict__ row_ptr,
    const int64_t* __restrict__ row_dst, float* __restrict__ out, int64_t n_rows, int C,
    int rows_per_block, int n_logical, uint32_t x_bytes) {
    static_assert(kSBatch % 2 == 0 && kSBatch <= 64, "one edge per lane in phase 1");
    static_assert(kSBatch % kRing == 0, "ring slots must line up across batches");
    __shared__ __attribute__((aligned(16))) float sM[kSBatch * kMStride];
    __shared__ float4 sStage[4][kScatterRows][64];
    __shared__ int64_t sRow[kScatterRows + 1];
    __shared__ int64_t sDst[kScatterRows];

    const int per_xcd = (n_logical + 7) / 8;
    const int logical = (blockIdx.x & 7) * per_xcd + (blockIdx.x >> 3);
    if (logical >= n_logical) return;

    const int lane = threadIdx.x & 63;
    const int w = threadIdx.x >> 6;
    const int g = lane >> 4;
    const int i16 = lane & 15;
    const int c = blockIdx.y * kChanGroup + w * 16 + i16;
    const uint32_t row_bytes = (uint32_t)C * 64u;
    const int voff = (c < C ? c : C - 1) * 64 + g * 16;
    const __amdgpu_buffer_rsrc_t xr = __builtin_amdgcn_make_buffer_rsrc(
        const_cast<float*>(X), (short)0, BUF ? (int)x_bytes : 0, kBufferDword3);

    const int64_t d0 = (int64_t)logical * rows_per_block;
    const int nrows = (int)(min<int64_t>(n_rows, d0 + rows_per_block) - d0);
    for (int i = threadIdx.x; i <= nrows; i += kMpBlock) {
        sRow[i] = row_ptr[d0 + i];
        if (i < nrows) sDst[i] = row_dst ? row_dst[d0 + i] : d0 + i;
    }
    __syncthreads();
    const int64_t e0 = sRow[0], e1 = sRow[nrows];

    // Last edge of each non-empty row, relative to e0 (-1: empty or absent row).
    // Wave-uniform, kept in scalar registers.
    int row_last[kScatterRows];
    static_for<kScatterRows>([&](auto rr) {
        constexpr int r = decltype(rr)::value;
        int v = -1;
        if (r < nrows && sRow[r + 1] > sRow[r]) v = (int)(sRow[r + 1] - 1 - e0);
        row_last[r] = __builtin_amdgcn_readfirstlane(v);
    });

    // Edge records move through a three-stage pipeline so that no wait is on a
    // load younger than the gathers in flight: the edge id of batch b+3 (one
    // load when PERM) and the record of batch b+2 are issued during batch b; the
    // record of batch b+1 (its source rows feed this batch's gathers) and of
    // batch b (phase 1) were issued one and two batches earlier.
    auto edge_id = [&](int64_t kbatch) -> int64_t {
        const int64_t k = kbatch + lane;
        if (lane >= kSBatch || k >= e1) return -1;
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
    int slot = 0;  // staged rows so far (the non-empty rows, in order)

    EdgeRec cur = record(edge_id(e0));
    EdgeRec nxt = record(edge_id(e0 + kSBatch));
    int64_t id2 = edge_id(e0 + 2 * kSBatch);
    // Every wave runs the edge loop, also one whose 16 channels are all past C
    // (its lanes read channel C-1 and never store): a branch around the loop
    // would make the loop-carried records look like the youngest loads on one
    // path, and the compiler would drain every gather at the loop latch.  (The
    // guard encloses the ring fill and the loop together for the same reason:
    // the loop header is reached only after the ring fill.)
    // Write the rows that end at or before edge `upto` and are not written yet
    // (staged rows in slot order; empty rows are zeros).
    int r_out = 0, s_out = 0;
    auto store_rows = [&](int64_t upto) {
        for (; r_out < nrows && sRow[r_out + 1] <= upto; ++r_out) {
            const int64_t orow = sDst[r_out];
            float4 v = make_float4(0.f, 0.f, 0.f, 0.f);
            if (sRow[r_out + 1] > sRow[r_out]) v = sStage[w][s_out++][lane];
            if (c < C && orow >= 0)
                *reinterpret_cast<float4*>(out + (orow * C + c) * 16 + 4 * g) = v;
        }
    };
    float4 ring[kRing];
    if (e0 < e1) {
    static_for<kRing>([&](auto uu) {
        constexpr int u = decltype(uu)::value;
        ring[u] = gather<BUF>(X, xr, voff, __builtin_amdgcn_readlane(cur.src, u), row_bytes);
    });
    // The loop's back edge is taken from full batches only; the last batch
    // (full or not) leaves through the tail path, which issues no gathers and
    // walks only the groups of 8 edges that hold real edges.
    for (int64_t kb = e0;; kb += kSBatch) {
        const int nb = (int)min<int64_t>(kSBatch, e1 - kb);
        __syncthreads();
        phase1_build<NORM>(cur, nb, sM);
        // edges of this batch that close a row
        const int rel = (int)(kb - e0);
        uint64_t ends = 0;
        static_for<kScatterRows>([&](auto rr) {
            constexpr int r = decltype(rr)::value;
            const int p = row_last[r] - rel;
            if (row_last[r] >= 0 && p >= 0 && p < kSBatch) ends |= 1ull << p;
        });
        __syncthreads();
        const float* mrow = sM + i16 * 16 + 4 * (g ^ quad_swizzle(i16));
        float4 mr[kLdsAhead + 1];
        // edge j: four MFMAs into the row accumulator, the gather of the edge
        // kRing positions ahead (of the next batch only when NEXT), the row's
        // staging when j closes it
        auto edge = [&](auto jj, auto next_c) {
            constexpr int j = decltype(jj)::value;
            constexpr int jn = j + kRing;
            if constexpr (j + kLdsAhead < kSBatch)
                mr[(j + kLdsAhead) % (kLdsAhead + 1)] =
                    *reinterpret_cast<const float4*>(mrow + (j + kLdsAhead) * kMStride);
            acc = mfma4(mr[j % (kLdsAhead + 1)], ring[j % kRing], acc);
            if constexpr (jn < kSBatch)
                ring[j % kRing] = gather<BUF>(X, xr, voff, __builtin_amdgcn_readlane(cur.src, jn), row_bytes);
            else if constexpr (decltype(next_c)::value)
                ring[j % kRing] =
                    gather<BUF>(X, xr, voff, __builtin_amdgcn_readlane(nxt.src, jn - kSBatch), row_bytes);
            if ((ends >> j) & 1ull) {
                sStage[w][slot][lane] = make_float4(acc[0], acc[1], acc[2], acc[3]);
                ++slot;
                acc = zero4;
            }
        };
        if (kb + kSBatch >= e1) {
            // rows closed before this batch go to HBM now: the tail issues no
            // gathers, so these stores hold nothing up, and the output is not
            // written in one burst at the end of the kernel
            store_rows(kb);
            static_for<kLdsAhead>([&](auto qq) {
                constexpr int q = decltype(qq)::value;
                mr[q] = *reinterpret_cast<const float4*>(mrow + q * kMStride);
            });
            static_for<kSBatch / 8>([&](auto gg) {
                constexpr int g8 = decltype(gg)::value;
                if (8 * g8 < nb)
                    static_for<8>([&](auto ii) {
                        edge(std::integral_constant<int, 8 * g8 + decltype(ii)::value>{},
                             std::false_type{});
                    });
            });
            break;
        }
        const EdgeRec nn = record(id2);
        id2 = edge_id(kb + 3 * kSBatch);
        // keep these loads ahead of the gathers: sunk below them, they would be
        // the youngest loads when the next batch needs them
        __builtin_amdgcn_sched_barrier(0);
        static_for<kLdsAhead>([&](auto qq) {
            constexpr int q = decltype(qq)::value;
            mr[q] = *reinterpret_cast<const float4*>(mrow + q * kMStride);
        });
        static_for<kSBatch>([&](auto jj) { edge(jj, std::true_type{}); });
        cur = nxt;
        nxt = nn;
    }
    }
    store_rows(e1);
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
#define BM_LAUNCH(NO, BU)                                                                    \
    mp_simple_mfma_kernel<false, NO, BU><<<grid, kMpBlock, 0, s>>>(                           \
        vec, X, src_idx, perm, row_ptr, row_dst, out, n_items, n_edges, C, (int)per,          \
        (int)n_logical, x_bytes)
#define BM_LAUNCH_SC(NO, BU, PE)                                                             \
    mp_scatter_kernel<NO, BU, PE><<<grid, kMpBlock, 0, s>>>(vec, X, src_idx, perm, row_ptr,   \
                                                            row_dst, out, n_items, C,         \
                                                            (int)per, (int)n_logical, x_bytes)
#define BM_LAUNCH_SC2(NO, BU) \
    do { if (perm) BM_LAUNCH_SC(NO, BU, true); else BM_LAUNCH_SC(NO, BU, false); } while (0)
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
#undef BM_LAUNCH_SC
#undef BM_LAUNCH
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
        csr_sort_rows_kernel<<<(unsigned)ceil_div(N_atoms, B), B, 0, stream>>>(row_ptr, col_idx,
                                                                               N_atoms);
    }
    return (int)hipGetLastError();
}

// ---------------------------------------------------------------------------
// Destination schedule: the fused scatter kernel runs n_blocks workgroups of
// rows_per_block (R) row slots; slot t of workgroup b is scheduled row
// q = b * R + t.  Workgroup b = x * P + k runs on XCD x (P = n_blocks / 8), and
// the workgroups of an XCD run in generations of Q resident ones.
//
//   - Each (XCD, generation) group owns a contiguous range of the spatial
//     order, cut so that every group holds edges in proportion to its number
//     of workgroups (at most Qg * R rows).
//   - Inside a group the rows are dealt in slices of Qg consecutive spatial
//     positions: slice t goes to slot t of the group's workgroups, so the rows
//     in flight on an XCD at one time stay spatially compact and their source
//     rows stay in L2.  Within a slice the heaviest row goes to the lightest
//     workgroup so far; a few rounds of pairwise swaps inside slices (the i-th
//     heaviest workgroup with the i-th lightest) then even out the totals.
//
// The kernel time is that of the busiest compute unit, so equal edge counts
// per workgroup matter: at configs[3] this brings the largest workgroup from
// 361 edges (fixed rows per workgroup) to within a few percent of the mean.
// Every destination is still summed by one wave in ascending edge order, so
// the result does not depend on the schedule.
// ---------------------------------------------------------------------------
namespace bmhip {

constexpr int kSchedMaxQ = 256;       // workgroups of one group (threads of the balancing block)
constexpr int kSchedSwapRounds = 8;

// degm[m] = in-degree of destination order[m]
__global__ void sched_degm_kernel(const int64_t* __restrict__ row_ptr,
                                  const int64_t* __restrict__ order, int64_t* __restrict__ degm,
                                  int64_t n_dst) {
    const int64_t m = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (m >= n_dst) return;
    const int64_t d = order[m];
    degm[m] = (d >= 0 && d < n_dst) ? row_ptr[d + 1] - row_ptr[d] : 0;
}

// Group boundaries gb[0 .. 8G] in spatial positions.  First every group's
// end is placed where the cumulative edge count reaches its share (one
// thread per group), then one thread clamps the ends in order so that every
// group fits its Qg * R slots and leaves room for the later groups.
__global__ void sched_group_targets_kernel(const int64_t* __restrict__ cum, int64_t n_dst, int P,
                                           int Q, int64_t* __restrict__ gb) {
    const int G = (P + Q - 1) / Q;
    const int gi = blockIdx.x * blockDim.x + threadIdx.x;
    if (gi >= 8 * G) return;
    const int x = gi / G, gen = gi - x * G;
    const int Qg = min(Q, P - gen * Q);
    const int64_t E = cum[n_dst];
    const int64_t w_end = (int64_t)x * P + (int64_t)gen * Q + Qg;
    const double target = (double)E * (double)w_end / (8.0 * (double)P);
    // first position whose cumulative edge count reaches the target, or the
    // one before it when that is closer
    int64_t lo = 0, hi = n_dst;
    while (lo < hi) {
        const int64_t mid = (lo + hi) >> 1;
        if ((double)cum[mid] < target) lo = mid + 1;
        else hi = mid;
    }
    if (lo > 0 && target - (double)cum[lo - 1] < (double)cum[lo] - target) --lo;
    gb[gi + 1] = lo;
}

__global__ void sched_groups_kernel(int64_t n_dst, int P, int Q, int R, int64_t* __restrict__ gb) {
    if (blockIdx.x != 0 || threadIdx.x != 0) return;
    const int G = (P + Q - 1) / Q;
    const int64_t total_wg = 8LL * P;
    int64_t start = 0;
    gb[0] = 0;
    for (int gi = 0; gi < 8 * G; ++gi) {
        const int gen = gi % G;
        const int Qg = min(Q, P - gen * Q);
        const int64_t w_end = (int64_t)(gi / G) * P + (int64_t)gen * Q + Qg;
        const int64_t low = max(start, n_dst - (total_wg - w_end) * (int64_t)R);
        const int64_t high = min(n_dst, start + (int64_t)Qg * R);
        const int64_t pos = max(low, min(high, gb[gi + 1]));
        gb[gi + 1] = pos;
        start = pos;
    }
}

// One block per group: deal the group's rows to its workgroups' slots.
__global__ __launch_bounds__(kSchedMaxQ) void sched_balance_kernel(
    const int64_t* __restrict__ degm, const int64_t* __restrict__ order,
    const int64_t* __restrict__ gb, int64_t n_dst, int P, int Q, int R,
    int64_t* __restrict__ row_dst, int64_t* __restrict__ slot_deg) {
    __shared__ int64_t sLoad[kSchedMaxQ];
    __shared__ int64_t sA[kScatterRows][kSchedMaxQ];   // degree in (slot, workgroup)
    __shared__ int sPos[kScatterRows][kSchedMaxQ];     // row (offset in the group) or -1
    __shared__ int sAt[kSchedMaxQ];
    __shared__ int64_t sDeg[kScatterRows * kSchedMaxQ];  // degrees of the group's rows
    const int G = (P + Q - 1) / Q;
    const int gi = blockIdx.x;
    const int x = gi / G, gen = gi - x * G;
    const int Qg = min(Q, P - gen * Q);
    const int k = threadIdx.x;
    const int64_t s0 = gb[gi], s1 = gb[gi + 1];
    const int n = (int)(s1 - s0);
    const int T = (n + Qg - 1) / Qg;  // <= R: a group holds at most Qg * R rows
    sLoad[k] = 0;
    for (int t = 0; t < kScatterRows; ++t) {
        sA[t][k] = 0;
        sPos[t][k] = -1;
    }
    for (int i = k; i < n; i += kSchedMaxQ) sDeg[i] = degm[s0 + i];
    __syncthreads();
    for (int t = 0; t < T; ++t) {
        const int o0 = t * Qg;  // slice start, offset in the group
        const int nt = min(Qg, n - o0);
        if (k < nt) {  // rank of row k in the slice, heaviest first
            const int64_t dk = sDeg[o0 + k];
            int r = 0;
            for (int j = 0; j < nt; ++j) {
                const int64_t dj = sDeg[o0 + j];
                r += (dj > dk) || (dj == dk && j < k);
            }
            sAt[r] = k;
        }
        int rw = 0;  // rank of workgroup k, lightest first
        if (k < Qg) {
            const int64_t lk = sLoad[k];
            for (int l = 0; l < Qg; ++l) {
                const int64_t ll = sLoad[l];
                rw += (ll < lk) || (ll == lk && l < k);
            }
        }
        __syncthreads();
        if (k < Qg && rw < nt) {
            const int i = sAt[rw];
            const int64_t d = sDeg[o0 + i];
            sA[t][k] = d;
            sPos[t][k] = o0 + i;
            sLoad[k] += d;
        }
        __syncthreads();
    }
    for (int rd = 0; rd < kSchedSwapRounds; ++rd) {
        int rw = 0;
        if (k < Qg) {
            const int64_t lk = sLoad[k];
            for (int l = 0; l < Qg; ++l) {
                const int64_t ll = sLoad[l];
                rw += (ll < lk) || (ll == lk && l < k);
            }
        }
        __syncthreads();
        if (k < Qg) sAt[rw] = k;
        __syncthreads();
        if (k < Qg / 2) {  // pair: k-th lightest with k-th heaviest
            const int l = sAt[k], h = sAt[Qg - 1 - k];
            const int64_t diff = sLoad[h] - sLoad[l];
            int best = -1;
            int64_t bv = diff;
            for (int t = 0; t < T; ++t) {
                const int64_t d = sA[t][h] - sA[t][l];
                if (d > 0 && d < diff) {
                    const int64_t v = diff > 2 * d ? diff - 2 * d : 2 * d - diff;
                    if (v < bv) {
                        bv = v;
                        best = t;
                    }
                }
            }
            if (best >= 0) {
                const int64_t d = sA[best][h] - sA[best][l];
                const int64_t ah = sA[best][h];
                const int ph = sPos[best][h];
                sA[best][h] = sA[best][l];
                sPos[best][h] = sPos[best][l];
                sA[best][l] = ah;
                sPos[best][l] = ph;
                sLoad[h] -= d;
                sLoad[l] += d;
            }
        }
        __syncthreads();
    }
    if (k < Qg) {
        const int64_t b = (int64_t)x * P + (int64_t)gen * Q + k;
        for (int t = 0; t < R; ++t) {
            const int p = t < T ? sPos[t][k] : -1;
            int64_t d = -1, dg = 0;
            if (p >= 0) {
                const int64_t o = order[s0 + p];
                if (o >= 0 && o < n_dst) {
                    d = o;
                    dg = sA[t][k];
                }
            }
            row_dst[b * R + t] = d;
            slot_deg[b * R + t] = dg;
        }
    }
}

__global__ void sched_edges_kernel(const int64_t* __restrict__ row_ptr,
                                   const int64_t* __restrict__ col_perm,
                                   const int64_t* __restrict__ row_dst,
                                   const int64_t* __restrict__ row_ptr_s,
                                   int64_t* __restrict__ edge_perm, int64_t n_sched) {
    const int64_t q = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (q >= n_sched) return;
    const int64_t d = row_dst[q];
    if (d < 0) return;
    const int64_t s0 = row_ptr[d], n = row_ptr[d + 1] - s0, o = row_ptr_s[q];
    for (int64_t i = 0; i < n; ++i) edge_perm[o + i] = col_perm ? col_perm[s0 + i] : s0 + i;
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

// degm [N_dst], cum [N_dst + 1], group bounds [8 G + 1] (G <= n_blocks / 8),
// slot degrees [n_blocks * rows_per_block]; N_dst <= n_blocks * rows_per_block.
extern "C" size_t batteries_mp_schedule_workspace_bytes(int n_blocks, int rows_per_block) {
    if (n_blocks <= 0 || rows_per_block <= 0) return 0;
    const size_t ns = (size_t)n_blocks * (size_t)rows_per_block;
    return sizeof(int64_t) * (3 * ns + (size_t)n_blocks + 2);
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
    const int Q = std::min(std::min(P, blocks_per_xcd(C)), kSchedMaxQ);
    const int G = (P + Q - 1) / Q;
    int64_t* degm = static_cast<int64_t*>(workspace);
    int64_t* cum = degm + N_dst;
    int64_t* gb = cum + N_dst + 1;
    int64_t* slot_deg = gb + 8 * (int64_t)G + 1;
    if (N_dst > 0)
        sched_degm_kernel<<<(unsigned)ceil_div(N_dst, B), B, 0, stream>>>(row_ptr, order, degm, N_dst);
    int rc = batteries_exclusive_scan_i64(degm, cum, N_dst, stream);
    if (rc != BM_OK) return rc;
    sched_group_targets_kernel<<<(unsigned)ceil_div(8 * (int64_t)G, 64), 64, 0, stream>>>(cum, N_dst,
                                                                                         P, Q, gb);
    sched_groups_kernel<<<1, 64, 0, stream>>>(N_dst, P, Q, rows_per_block, gb);
    sched_balance_kernel<<<(unsigned)(8 * G), kSchedMaxQ, 0, stream>>>(
        degm, order, gb, N_dst, P, Q, rows_per_block, row_dst, slot_deg);
    rc = batteries_exclusive_scan_i64(slot_deg, row_ptr_s, n_sched, stream);
    if (rc != BM_OK) return rc;
    sched_edges_kernel<<<(unsigned)ceil_div(n_sched, B), B, 0, stream>>>(row_ptr, col_perm, row_dst,
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

// ---------------------------------------------------------------------------
// Weighted scatter: one W [34, C_in, C_out] shared by every edge,
//   out[d, co, o] = sum_{e -> d} TP_W(X[src_e], Y(v_e))[co, o].
// Because W is shared, the sum over the edges of d moves in front of both the
// CG contraction and the channel mixing:
//   S[d, ci, a, b] = sum_{e -> d} X[src_e, ci, a] Y_e[b]              MFMA over edges
//   T[d, q, ci]    = sum_{(a, b) in slot q} c S[d, ci, a, b]           CG table, VALU
//   out[d, co, o]  = sum_{q -> o} sum_ci W[p(q), ci, co] T[d, q, ci]   MFMA (tp.hip)
// Work: 2 * 256 * C_in flops per edge (S), 2 * 611 * C_in + 2 * 156 * C_in * C_out per
// destination (T, mixing).  T is [chunk][block][slot][16][16]: 16-channel chunks of
// C_in (zero past C_in), destinations by their position in the processing order
// (padded to a multiple of 16) in blocks of 16 positions, slots in fwd_slot_pos
// order, so that the mixing kernel's operand loads and the path-sum kernel's stores
// are contiguous 1 KB / 256 B blocks (whole 128-byte lines: a load that uses half of
// each line it touches runs at half the rate) and slot offsets are compile-time
// constants.
// ---------------------------------------------------------------------------
namespace bmhip {

// Blocks [0, edge_blocks): Y and the source row of CSR slot k (edge perm[k] when
// perm is given), so that the path-sum kernel reads both without indirection.
// Blocks past them: wt[chunk][p][co][16] = W[p][16 chunk + i][co], zero past cin (the
// mixing kernel's B operand: 16 output channels x 16 input channels = 1 KB contiguous).
__global__ __launch_bounds__(256) void mp_edge_prep_kernel(
    const float* __restrict__ vec, const int64_t* __restrict__ src_idx,
    const int64_t* __restrict__ perm, int64_t n_edges, int normalize, float* __restrict__ yc,
    int* __restrict__ srcc, int64_t edge_blocks, const float* __restrict__ w,
    float* __restrict__ wt, int cin, int cout, int cp) {
    if ((int64_t)blockIdx.x >= edge_blocks) {
        const int64_t i = ((int64_t)blockIdx.x - edge_blocks) * 256 + threadIdx.x;
        if (i >= (int64_t)kNumPaths * cout * cp) return;
        const int cl = (int)(i & 15);
        const int64_t r = i >> 4;  // (chunk * 34 + p) * cout + co
        const int co = (int)(r % cout);
        const int64_t cpp = r / cout;
        const int p = (int)(cpp % kNumPaths);
        const int ci = (int)(cpp / kNumPaths) * 16 + cl;
        wt[i] = ci < cin ? w[((int64_t)p * cin + ci) * cout + co] : 0.0f;
        return;
    }
    const int64_t k = (int64_t)blockIdx.x * 256 + threadIdx.x;
    if (k >= n_edges) return;
    const int64_t e = perm ? perm[k] : k;
    float x = vec[e * 3 + 0], y = vec[e * 3 + 1], z = vec[e * 3 + 2];
    if (normalize) normalize3(x, y, z);
    float Y[16];
    sh_forward<3>(x, y, z, Y);
    float4* o = reinterpret_cast<float4*>(yc + k * 16);
    o[0] = make_float4(Y[0], Y[1], Y[2], Y[3]);
    o[1] = make_float4(Y[4], Y[5], Y[6], Y[7]);
    o[2] = make_float4(Y[8], Y[9], Y[10], Y[11]);
    o[3] = make_float4(Y[12], Y[13], Y[14], Y[15]);
    srcc[k] = (int)src_idx[e];
}

// S of one (destination, channel) in LDS: 16 rows b of 16 a, the four 16-byte
// quads of row b at positions quad ^ ps_swz(b), rows of successive channels
// kPsStride floats apart.  The MFMA-layout writes (8 lanes = 8 values of b) and
// the contraction's reads (8 lanes = 8 channels) are then free of bank conflicts.
constexpr int kPsStride = 260;
// T is [chunk][16-position block][slot][16 positions][16 channels]: one slot of a
// block is 1 KB, so slot offsets are compile-time constants.
constexpr int kTSlotBytes = 16 * 16 * 4;
constexpr int kTBlockBytes = kNumSlots * kTSlotBytes;
__host__ __device__ constexpr int ps_swz(int b) { return (b >> 1) & 3; }

// CG blocks (l1, l2) contracted by each wave: 166, 149, 149, 147 CG terms.
constexpr int kPsBlocks[4][5][2] = {{{1, 0}, {3, 1}, {3, 3}, {-1, -1}, {-1, -1}},
                                    {{0, 2}, {1, 3}, {2, 3}, {3, 0}, {-1, -1}},
                                    {{0, 0}, {0, 1}, {0, 3}, {1, 2}, {3, 2}},
                                    {{1, 1}, {2, 0}, {2, 1}, {2, 2}, {-1, -1}}};

// The slots of the paths (L1, L2, *) for this lane's (destination, channel):
// reads S[a in l1][b in l2], contracts with the CG terms, stores slot q at byte
// toff + pos(q) * 1 KB of the chunk's T (the slot offset is a compile-time
// constant in a scalar register).
template <int L1, int L2>
__device__ __forceinline__ void ps_block(const float* sSrow, __amdgpu_buffer_rsrc_t tr, int toff,
                                         bool store, bool chan_ok) {
    constexpr int a0 = L1 * L1, na = 2 * L1 + 1, b0 = L2 * L2, nb = 2 * L2 + 1;
    constexpr int qa0 = a0 / 4, qa1 = (a0 + na - 1) / 4;
    float s[nb][na];
    static_for<nb>([&](auto bb) {
        constexpr int b = b0 + decltype(bb)::value;
        static_for<qa1 - qa0 + 1>([&](auto qq) {
            constexpr int qa = qa0 + decltype(qq)::value;
            const float4 v =
                *reinterpret_cast<const float4*>(sSrow + b * 16 + (qa ^ ps_swz(b)) * 4);
            const float vv[4] = {v.x, v.y, v.z, v.w};
            static_for<4>([&](auto ii) {
                constexpr int i = decltype(ii)::value;
                constexpr int a = 4 * qa + i;
                if constexpr (a >= a0 && a < a0 + na) s[b - b0][a - a0] = vv[i];
            });
        });
    });
    static_for<kNumPaths>([&](auto pp) {
        constexpr int p = decltype(pp)::value;
        if constexpr (kPathL[p][0] == L1 && kPathL[p][1] == L2) {
            constexpr int no = 2 * kPathL[p][2] + 1;
            float t[no];
            static_for<no>([&](auto m) { t[decltype(m)::value] = 0.0f; });
            static_for<kPathEntry[p + 1] - kPathEntry[p]>([&](auto kk) {
                constexpr CGEntry e = kCG[kPathEntry[p] + decltype(kk)::value];
                constexpr int m = e.q - kPathSlot[p];
                t[m] = fmaf(e.c, s[e.b - b0][e.a - a0], t[m]);
            });
            if (store) {
                static_for<no>([&](auto mm) {
                    constexpr int m = decltype(mm)::value;
                    constexpr int pos = fwd_slot_pos(kPathSlot[p] + m);  // compile time
                    __builtin_amdgcn_raw_buffer_store_b32(__float_as_int(chan_ok ? t[m] : 0.0f),
                                                          tr, toff, pos * kTSlotBytes, 0);
                });
            }
        }
    });
}

template <int W>
__device__ __forceinline__ void ps_contract(const float* sSrow, __amdgpu_buffer_rsrc_t tr,
                                            int toff, bool store, bool chan_ok) {
    static_for<5>([&](auto kk) {
        constexpr int k = decltype(kk)::value;
        if constexpr (kPsBlocks[W][k][0] >= 0)
            ps_block<kPsBlocks[W][k][0], kPsBlocks[W][k][1]>(sSrow, tr, toff, store, chan_ok);
    });
}

__device__ __forceinline__ int64_t uniform64(int64_t v) {
    const uint64_t u = (uint64_t)v;
    const uint32_t lo = __builtin_amdgcn_readfirstlane((uint32_t)u);
    const uint32_t hi = __builtin_amdgcn_readfirstlane((uint32_t)(u >> 32));
    return (int64_t)(((uint64_t)hi << 32) | lo);
}

// One workgroup per unit: 4 destinations at consecutive positions of `order`
// and `cpw` consecutive 16-channel chunks.  Per chunk:
// S phase: wave w sums the edges of destination w, four edges per k-step: lane
// (g = lane / 16, i = lane % 16) supplies
//   A[i][g] = X[src of edge g][c0 + 4t + i / 4][4 (i % 4) + j]   (MFMA (t, j), float4 over j)
//   B[g][i] = Y[edge g][b = i]
// so that MFMA (t, j) accumulates S[c0 + 4t + m / 4][a = 4 (m % 4) + j][b] in row m.
// Lane (g, i) then holds S[c0 + 4t + g][all a][b = i] and writes it to LDS.
// Contraction phase: lane (dd, ch) = (lane / 16, lane % 16) of every wave takes
// destination dd and channel c0 + ch; wave w contracts its CG blocks.
// The k-steps of a wave run through a four-stage load pipeline that continues
// across chunks: the source index and Y of step i + 3, the source-row gathers of
// steps i + 2 and i + 1, the MFMAs of step i.  The next chunk's first gathers are therefore
// in flight during this chunk's contraction.
__global__ __launch_bounds__(256, 2) void mp_path_sums_kernel(
    const float* __restrict__ yc, const int* __restrict__ srcc, const float* __restrict__ X,
    const int64_t* __restrict__ row_ptr, const int64_t* __restrict__ order, float* __restrict__ T,
    int64_t n_dst, int64_t npad, int C, int cpw, int64_t n_units) {
    __shared__ __attribute__((aligned(16))) float sS[4 * 16 * kPsStride];
    const int64_t per_xcd = (n_units + 7) / 8;
    const int64_t logical = (int64_t)(blockIdx.x & 7) * per_xcd + (blockIdx.x >> 3);
    if (logical >= n_units) return;
    const int64_t nquad = (n_dst + 3) >> 2;
    const int nchunk = (C + 15) >> 4;
    const int cgrp = (int)(logical / nquad);  // chunk-group major: an XCD works on a
    const int64_t quad = logical - cgrp * nquad;  // compact range of destinations
    const int ch0 = cgrp * cpw;                   // first chunk of this unit
    const int nch = min(cpw, nchunk - ch0);
    const int lane = threadIdx.x & 63, w = threadIdx.x >> 6, g = lane >> 4, i16 = lane & 15;

    int64_t r0 = 0, r1 = 0;
    {
        const int64_t pos = quad * 4 + w;
        if (pos < n_dst) {
            const int64_t d = order ? order[pos] : pos;
            if (d >= 0 && d < n_dst) {  // an order entry out of range sums no edges
                r0 = row_ptr[d];
                r1 = row_ptr[d + 1];
            }
        }
        r0 = uniform64(r0);
        r1 = uniform64(r1);
    }
    const int deg = (int)(r1 - r0);
    const int nst = (deg + 3) >> 2;  // k-steps per chunk
    const int64_t rowf = (int64_t)C * 16;  // floats per source row
    // CSR slot of this lane's edge in step s (past the row: its last edge, Y masked to 0)
    auto slot = [&](int s) { return r0 + min(4 * s + g, deg - 1); };
    auto gather = [&](int src, int chunk, float4(&xv)[4]) {
        const float* rowp = X + (int64_t)src * rowf;
        const int c0 = (ch0 + chunk) * 16;
#pragma unroll
        for (int t = 0; t < 4; ++t)
            xv[t] = *reinterpret_cast<const float4*>(
                rowp + min(c0 + 4 * t + (i16 >> 2), C - 1) * 16 + (i16 & 3) * 4);
    };
    // the step after (c, s), or (c, s) itself past the last step
    auto next = [&](int& c, int& s) {
        if (s + 1 < nst) {
            ++s;
        } else if (c + 1 < nch) {
            ++c;
            s = 0;
        }
    };
    // pipeline state: stage A (source index, Y of the step three ahead), stage C
    // (gathers of the step two ahead) and stage B (gathers of the next step)
    int cA = 0, sA = 0, cC = 0, sC = 0;
    int srcA = 0;
    float yA = 0.f, yB = 0.f, yC = 0.f;
    float4 xB[4], xC[4];
#pragma unroll
    for (int t = 0; t < 4; ++t) xB[t] = xC[t] = make_float4(0.f, 0.f, 0.f, 0.f);
    if (nst > 0) {
        srcA = srcc[slot(0)];
        yA = 4 * 0 + g < deg ? yc[slot(0) * 16 + i16] : 0.f;
        gather(srcA, 0, xB);
        yB = yA;
        next(cA, sA);
        srcA = srcc[slot(sA)];
        yA = 4 * sA + g < deg ? yc[slot(sA) * 16 + i16] : 0.f;
        cC = cA;
        sC = sA;
        gather(srcA, cC, xC);
        yC = yA;
        next(cA, sA);
        srcA = srcc[slot(sA)];
        yA = 4 * sA + g < deg ? yc[slot(sA) * 16 + i16] : 0.f;
    }
    v4f acc[4][4];
    for (int c = 0; c < nch; ++c) {
#pragma unroll
        for (int t = 0; t < 4; ++t)
#pragma unroll
            for (int j = 0; j < 4; ++j) acc[t][j] = v4f{0.f, 0.f, 0.f, 0.f};
        for (int s = 0; s < nst; ++s) {
            float4 xa[4];
#pragma unroll
            for (int t = 0; t < 4; ++t) {
                xa[t] = xB[t];
                xB[t] = xC[t];
            }
            const float ya = yB;
            yB = yC;
            next(cC, sC);  // stage C: gathers of the step two ahead
            gather(srcA, cC, xC);
            yC = yA;
            next(cA, sA);  // stage A: index and Y three steps ahead
            srcA = srcc[slot(sA)];
            {
                const float yv = yc[slot(sA) * 16 + i16];
                yA = 4 * sA + g < deg ? yv : 0.f;
            }
#pragma unroll
            for (int t = 0; t < 4; ++t) {
                acc[t][0] = mfma1(xa[t].x, ya, acc[t][0]);
                acc[t][1] = mfma1(xa[t].y, ya, acc[t][1]);
                acc[t][2] = mfma1(xa[t].z, ya, acc[t][2]);
                acc[t][3] = mfma1(xa[t].w, ya, acc[t][3]);
            }
        }
        if (c > 0) __syncthreads();  // the previous chunk's contraction reads are done
        // S[c0 + 4t + g][a = 4r + j][b = i16] -> LDS block (w, 4t + g), row b, quad r
#pragma unroll
        for (int t = 0; t < 4; ++t) {
            float* blk = sS + (w * 16 + 4 * t + g) * kPsStride + i16 * 16;
#pragma unroll
            for (int r = 0; r < 4; ++r)
                *reinterpret_cast<float4*>(blk + ((r ^ ps_swz(i16)) * 4)) =
                    make_float4(acc[t][0][r], acc[t][1][r], acc[t][2][r], acc[t][3][r]);
        }
        __syncthreads();
        // contraction: lane (dd, ch)
        // the 4 positions x 16 channels of one slot are 256 contiguous bytes of T
        const int dd = lane >> 4, ch = lane & 15;
        const int c0 = (ch0 + c) * 16;
        const int64_t pos = quad * 4 + dd;
        const bool store = pos < n_dst;
        const int64_t tchunk = npad * kNumSlots * 16;  // floats per chunk of T
        const __amdgpu_buffer_rsrc_t tr =
            buffer_rsrc(T + (int64_t)(ch0 + c) * tchunk, (uint32_t)(tchunk * 4));
        const int toff = (int)(pos >> 4) * kTBlockBytes + ((int)(pos & 15) * 16 + ch) * 4;
        const float* sSrow = sS + (dd * 16 + ch) * kPsStride;
        const bool chan_ok = c0 + ch < C;
        switch (w) {
            case 0: ps_contract<0>(sSrow, tr, toff, store, chan_ok); break;
            case 1: ps_contract<1>(sSrow, tr, toff, store, chan_ok); break;
            case 2: ps_contract<2>(sSrow, tr, toff, store, chan_ok); break;
            default: ps_contract<3>(sSrow, tr, toff, store, chan_ok); break;
        }
    }
}

// Mixing stage: out[order[r], co, o] = sum_{q: out(q) = o} sum_ci W[p(q), ci, co] T[., q, r, ci]
// over positions r.  One wave per (16 positions, output component o, 64 output
// channels), no LDS until the output: per slot q of o and 16-channel chunk, four
// k-steps of
//   D[r][co] += A[r][ci] B[ci][co],  A = T (lane (r = l % 16, k = l / 16): float4
//   over ci = 4k .. 4k + 3),  B = wt (lane (k, co = l % 16), the same four ci)
// for the four 16-channel tiles of co.  Each operand load is 1 KB contiguous.  A path
// reaches o through one slot only, so every slot brings its own W.  Operands are
// loaded kMixAhead slots ahead, across chunk boundaries.
constexpr int kMixAhead = 2;
constexpr int n_slots_out(int o) {
    int c = 0;
    for (int q = 0; q < kNumSlots; ++q) c += kSlotOut[q] == o ? 1 : 0;
    return c;
}
constexpr int slot_of_out(int o, int k) {
    for (int q = 0; q < kNumSlots; ++q)
        if (kSlotOut[q] == o) {
            if (k == 0) return q;
            --k;
        }
    return -1;
}

template <int O>
__device__ __forceinline__ void mix_component(const float* __restrict__ T,
                                              const float* __restrict__ wt, float* sOut, int64_t n,
                                              int64_t npad, int nchunk, int cout, int64_t row0,
                                              int co0) {
    constexpr int NS = n_slots_out(O);
    static_assert(NS >= kMixAhead, "ring deeper than the slot list");
    const int lane = threadIdx.x & 63, g4 = lane >> 4, i16 = lane & 15;
    // buffer loads: lane offsets in VGPRs, (chunk, slot, path) offsets in SGPRs
    const int64_t tchunk = (int64_t)kNumSlots * npad * 16;  // floats per chunk of T
    const uint32_t tchunk_bytes = (uint32_t)(tchunk * sizeof(float));
    const int toff = ((int)min<int64_t>(i16, n - 1 - row0) * 16 + 4 * g4) * 4;
    const int tblock = (int)(row0 >> 4) * kTBlockBytes;  // bytes of the tile's block
    const __amdgpu_buffer_rsrc_t wr =
        buffer_rsrc(wt, (uint32_t)((int64_t)nchunk * kNumPaths * cout * 64));
    const int wpath = cout * 64, wchunk = kNumPaths * cout * 64;
    int wco[4];
#pragma unroll
    for (int t = 0; t < 4; ++t) wco[t] = (min(co0 + 16 * t + i16, cout - 1) * 16 + 4 * g4) * 4;
    v4f acc[4];
#pragma unroll
    for (int t = 0; t < 4; ++t) acc[t] = v4f{0.f, 0.f, 0.f, 0.f};
    auto load = [&](int chunk, auto kk, float4& a, float4 (&b)[4]) {
        constexpr int k = decltype(kk)::value;
        constexpr int q = slot_of_out(O, k);
        constexpr int pos = fwd_slot_pos(q);
        constexpr int p = kSlotPath[q];
        const __amdgpu_buffer_rsrc_t tr = buffer_rsrc(T + chunk * tchunk, tchunk_bytes);
        a = buffer_ld4(tr, toff, tblock + pos * kTSlotBytes);
#pragma unroll
        for (int t = 0; t < 4; ++t) b[t] = buffer_ld4(wr, wco[t], chunk * wchunk + p * wpath);
    };
    float4 hA[kMixAhead], hB[kMixAhead][4];  // first slots of the current chunk
    static_for<kMixAhead>([&](auto jj) {
        constexpr int j = decltype(jj)::value;
        load(0, jj, hA[j], hB[j]);
    });
    for (int c = 0; c < nchunk; ++c) {
        float4 oA[NS], oB[NS][4];
        static_for<kMixAhead>([&](auto jj) {
            constexpr int j = decltype(jj)::value;
            oA[j] = hA[j];
#pragma unroll
            for (int t = 0; t < 4; ++t) oB[j][t] = hB[j][t];
        });
        static_for<NS>([&](auto kk) {
            constexpr int k = decltype(kk)::value;
            constexpr int kn = k + kMixAhead;
            if constexpr (kn < NS)
                load(c, std::integral_constant<int, kn>{}, oA[kn], oB[kn]);
            else
                load(min(c + 1, nchunk - 1), std::integral_constant<int, kn - NS>{}, hA[kn - NS],
                     hB[kn - NS]);
#pragma unroll
            for (int t = 0; t < 4; ++t) acc[t] = mfma4(oA[k], oB[k][t], acc[t]);
            // keep the ring: no load moves ahead of the slot it belongs to
            __builtin_amdgcn_sched_barrier(0);
        });
    }
    // D[4 g4 + r][i16]: position 4 g4 + r of the tile, channel 16 t + i16 of the 64; the
    // workgroup's four components of one (position, channel) meet in LDS
    const int w = threadIdx.x >> 6;
#pragma unroll
    for (int t = 0; t < 4; ++t)
#pragma unroll
        for (int r = 0; r < 4; ++r) sOut[((4 * g4 + r) * 64 + 16 * t + i16) * 4 + w] = acc[t][r];
}

// grid (4 x 16-position tiles, 64-channel tiles of C_out): block x is group G = x % 4 of
// tile x / 4 (a tile's four blocks are dispatched together), wave w takes o = 4 G + w,
// and the block stores float4 (o = 4 G .. 4 G + 3) per (destination, channel).
__global__ __launch_bounds__(256) void mp_weighted_mix_kernel(const float* __restrict__ T,
                                                              const float* __restrict__ wt,
                                                              const int64_t* __restrict__ order,
                                                              float* __restrict__ out, int64_t n,
                                                              int64_t npad, int nchunk, int cout) {
    __shared__ __attribute__((aligned(16))) float sOut[16 * 64 * 4];
    const int G = blockIdx.x & 3;
    const int64_t row0 = (int64_t)(blockIdx.x >> 2) * 16;
    const int co0 = blockIdx.y * 64;
    switch (G * 4 + (threadIdx.x >> 6)) {
#define BM_MIX_CASE(o) \
    case o: mix_component<o>(T, wt, sOut, n, npad, nchunk, cout, row0, co0); break;
        BM_MIX_CASE(0) BM_MIX_CASE(1) BM_MIX_CASE(2) BM_MIX_CASE(3)
        BM_MIX_CASE(4) BM_MIX_CASE(5) BM_MIX_CASE(6) BM_MIX_CASE(7)
        BM_MIX_CASE(8) BM_MIX_CASE(9) BM_MIX_CASE(10) BM_MIX_CASE(11)
        BM_MIX_CASE(12) BM_MIX_CASE(13) BM_MIX_CASE(14)
#undef BM_MIX_CASE
        default: mix_component<15>(T, wt, sOut, n, npad, nchunk, cout, row0, co0); break;
    }
    __syncthreads();
    // 16 positions x 64 channels of float4: four per thread
#pragma unroll
    for (int k = 0; k < 4; ++k) {
        const int i = threadIdx.x + 256 * k;  // position i / 64, channel i % 64
        const int64_t r = row0 + (i >> 6);
        const int co = co0 + (i & 63);
        if (r < n && co < cout) {
            const int64_t d = order ? order[r] : r;
            if (d >= 0 && d < n)  // an order entry out of range is not written
                *reinterpret_cast<float4*>(out + (d * cout + co) * 16 + 4 * G) =
                    *reinterpret_cast<const float4*>(sOut + i * 4);
        }
    }
}

static size_t align256(size_t b) { return (b + 255) & ~(size_t)255; }

}  // namespace bmhip

extern "C" size_t batteries_sh_tp_scatter_weighted_workspace_bytes(int64_t N_dst, int64_t N_edges,
                                                                   int C_in, int C_out) {
    if (N_dst < 0 || N_edges < 0 || C_in <= 0 || C_out <= 0) return 0;
    const size_t cp = (size_t)((C_in + 15) / 16) * 16;
    const size_t npad = (size_t)((N_dst + 15) / 16) * 16;
    return align256((size_t)N_edges * 16 * sizeof(float)) + align256((size_t)N_edges * sizeof(int)) +
           align256(npad * kNumSlots * cp * sizeof(float)) +
           align256((size_t)kNumPaths * C_out * cp * sizeof(float));
}

extern "C" int batteries_sh_tp_scatter_weighted(
    const float* edge_vectors, const float* node_features, const float* weights,
    const int64_t* source_idx, const int64_t* perm, const int64_t* row_ptr, const int64_t* order,
    float* node_output, int64_t N_src, int64_t N_dst, int64_t N_edges, int C_in, int C_out,
    int normalize, void* workspace, size_t workspace_bytes, hipStream_t stream) {
    if (N_src < 0 || N_dst < 0 || N_edges < 0 || C_in <= 0 || C_out <= 0) return BM_ERR_ARG;
    if (N_edges > 0 && N_src == 0) return BM_ERR_ARG;
    if (N_dst == 0) return BM_OK;
    if (N_edges > INT32_MAX || N_src > INT32_MAX) return BM_ERR_ARG;  // int32 source rows in workspace
    if ((int64_t)kNumPaths * C_in * C_out * 4 > INT32_MAX) return BM_ERR_ARG;  // W via 32-bit offsets
    if (ceil_div(N_dst, 16) > INT32_MAX || ceil_div(C_out, 64) > 65535) return BM_ERR_ARG;
    if ((reinterpret_cast<uintptr_t>(node_features) | reinterpret_cast<uintptr_t>(node_output) |
         reinterpret_cast<uintptr_t>(workspace)) & 15)
        return BM_ERR_ARG;
    const size_t need =
        batteries_sh_tp_scatter_weighted_workspace_bytes(N_dst, N_edges, C_in, C_out);
    if (!workspace || workspace_bytes < need) return BM_ERR_WORKSPACE;
    const int cp = (C_in + 15) / 16 * 16;
    const int64_t npad = ceil_div(N_dst, 16) * 16;
    // 32-bit byte offsets inside one chunk of T and inside wt
    if ((int64_t)kNumSlots * npad * 64 > INT32_MAX) return BM_ERR_ARG;
    if ((int64_t)kNumPaths * C_out * cp * 4 > INT32_MAX) return BM_ERR_ARG;
    char* ws = static_cast<char*>(workspace);
    float* yc = reinterpret_cast<float*>(ws);
    ws += align256((size_t)N_edges * 16 * sizeof(float));
    int* srcc = reinterpret_cast<int*>(ws);
    ws += align256((size_t)N_edges * sizeof(int));
    float* tsum = reinterpret_cast<float*>(ws);
    ws += align256((size_t)npad * kNumSlots * cp * sizeof(float));
    float* wt = reinterpret_cast<float*>(ws);
    const int64_t edge_blocks = ceil_div(N_edges, 256);
    const int64_t wt_blocks = ceil_div((int64_t)kNumPaths * C_out * cp, 256);
    if (edge_blocks + wt_blocks > INT32_MAX) return BM_ERR_ARG;
    mp_edge_prep_kernel<<<(unsigned)(edge_blocks + wt_blocks), 256, 0, stream>>>(
        edge_vectors, source_idx, perm, N_edges, normalize, yc, srcc, edge_blocks, weights, wt,
        C_in, C_out, cp);
    const int64_t nquad = ceil_div(N_dst, 4);
    const int nchunk = (C_in + 15) / 16;
    const int cpw = std::min(nchunk, 2);  // 16-channel chunks per workgroup
    const int64_t n_units = nquad * ceil_div(nchunk, cpw);
    const int64_t grid = ceil_div(n_units, 8) * 8;
    if (grid > INT32_MAX) return BM_ERR_ARG;
    mp_path_sums_kernel<<<(unsigned)grid, 256, 0, stream>>>(
        yc, srcc, node_features, row_ptr, order, tsum, N_dst, npad, C_in, cpw, n_units);
    if (ceil_div(N_dst, 16) * 4 > INT32_MAX) return BM_ERR_ARG;
    dim3 mgrid((unsigned)(ceil_div(N_dst, 16) * 4), (unsigned)ceil_div(C_out, 64), 1);
    mp_weighted_mix_kernel<<<mgrid, 256, 0, stream>>>(tsum, wt, order, node_output, N_dst, npad,
                                                      nchunk, C_out);
    return (int)hipGetLastError();
}
