// Graph build for the fused message-passing kernels in four kernels: the neighbor
// list in the message-passing layout (edges grouped by destination, sources
// ascending), the spatial order of the atoms and the processing schedule of the
// fused scatter kernel, for systems of up to kGbMaxAtoms atoms.
//
// Replaces, for batmobile.Graph, the cell-list passes of nl.hip (binning, count,
// scan, write, row sort: reference src/neighbor_list/neighbor_list.cu:242-430 and
// the e2e pipeline's per-step neighbor list, benchmarks/benchmark_e2e_mace.py:192-278),
// the serpentine order and batteries_mp_schedule (mp.hip), with the same results:
// gb_bin_kernel, gb_cell_kernel (which also writes the spatial order) and
// gb_rows_kernel of nl_cells.h, and between the last two
//
//   gb_sched_kernel  one workgroup per schedule group: each computes the row offsets
//                    (exclusive sums of the counts), the degrees in spatial order and
//                    their sums and the group bounds in LDS, then balances its group
//                    (mp_schedule.h) with four waves on a compute unit of its own and
//                    writes every scheduled destination's slot offset for the row
//                    kernel (edge_perm); the first one writes the row offsets.
#include "common.h"
#include "batmobile_hip.h"
#include "nl_geom.h"
#include "mp_schedule.h"
#include "nl_cells.h"

namespace bmhip {

constexpr int kGsThreads = 1024;               // the schedule workgroup
constexpr int kGsPer = kGbMaxAtoms / kGsThreads;
constexpr int kGsMaxGroups = 256;               // schedule groups (8 per generation)
constexpr int kGsFastGroups = 32;               // up to this many: targets found in parallel

// Exclusive sums of s[0 .. n) in place (s[n] = total), n <= kGbMaxAtoms, by the
// kGsThreads threads of the workgroup: thread t sums its run s[8t .. 8t + 8) (two
// 16-byte reads), the run totals are scanned within each wave, then across the
// waves.  s is 16-byte aligned.  Returns the total.
__device__ int gb_lds_scan(int* s, int n, int* sWsum) {
    static_assert(kGsPer == 8, "two int4 per thread");
    const int t = threadIdx.x, lane = t & 63, w = t >> 6;
    const int i0 = t * kGsPer;
    const int4 r0 = reinterpret_cast<const int4*>(s + i0)[0];
    const int4 r1 = reinterpret_cast<const int4*>(s + i0)[1];
    int v[kGsPer] = {r0.x, r0.y, r0.z, r0.w, r1.x, r1.y, r1.z, r1.w};
    int sum = 0;
#pragma unroll
    for (int q = 0; q < kGsPer; ++q) {
        v[q] = i0 + q < n ? v[q] : 0;
        sum += v[q];
    }
    const int x = wave_incl_scan(sum);
    if (lane == 63) sWsum[w] = x;
    __syncthreads();
    int before = 0, total = 0;
#pragma unroll
    for (int k = 0; k < kGsThreads / 64; ++k) {
        const int ws = sWsum[k];
        before += k < w ? ws : 0;
        total += ws;
    }
    int run = before + x - sum;
    int o[kGsPer];
#pragma unroll
    for (int q = 0; q < kGsPer; ++q) {
        o[q] = run;
        run += v[q];
    }
    if (i0 + kGsPer <= n) {
        reinterpret_cast<int4*>(s + i0)[0] = make_int4(o[0], o[1], o[2], o[3]);
        reinterpret_cast<int4*>(s + i0)[1] = make_int4(o[4], o[5], o[6], o[7]);
    } else {
#pragma unroll
        for (int q = 0; q < kGsPer; ++q)
            if (i0 + q < n) s[i0 + q] = o[q];
    }
    if (t == 0) s[n] = total;
    __syncthreads();
    return total;
}

__global__ __launch_bounds__(kGsThreads) void gb_sched_kernel(
    const int* __restrict__ cnt, const int64_t* __restrict__ order, int n, uint64_t cap, int P,
    int Q, int R, int64_t* __restrict__ offsets, int* __restrict__ overflow,
    int64_t* __restrict__ row_dst, int64_t* __restrict__ row_ptr_s, int64_t* __restrict__ soff) {
    __shared__ __attribute__((aligned(16))) int sOff[kGbMaxAtoms + 4];  // row offsets, atom order
    __shared__ __attribute__((aligned(16))) int sCum[kGbMaxAtoms + 4];  // running sums, spatial order
    __shared__ int sOrd[kGbMaxAtoms];                                   // the spatial order
    __shared__ int sWsum[kGsThreads / 64];
    __shared__ int sPos[kGsMaxGroups];
    __shared__ int sGb[kGsMaxGroups + 1];
    __shared__ int sQg[kGsMaxGroups];
    __shared__ int sWend[kGsMaxGroups];
    __shared__ double sTgt[kGsMaxGroups];
    __shared__ __attribute__((aligned(16))) SchedLds<int> sL;
    const int t = threadIdx.x, lane = t & 63;
    const int w = __builtin_amdgcn_readfirstlane(t >> 6);
    int cv[kGsPer];
    int64_t ov[kGsPer];
#pragma unroll
    for (int j = 0; j < kGsPer; ++j) {
        const int i = min(j * kGsThreads + t, n - 1);
        cv[j] = cnt[i];
        ov[j] = order[i];
    }
    const int G = (P + Q - 1) / Q;
    for (int gi = t; gi < 8 * G; gi += kGsThreads) {
        const SchedGroup s = sched_group(gi, P, Q);
        sQg[gi] = s.Qg;
        sWend[gi] = (int)s.w_end;
    }
#pragma unroll
    for (int j = 0; j < kGsPer; ++j) {
        const int i = j * kGsThreads + t;
        if (i < n) {
            sOff[i] = cv[j];
            sOrd[i] = (int)ov[j];
        }
    }
    __syncthreads();
    const int E0 = gb_lds_scan(sOff, n, sWsum);
    // capacity mode: when the edges outgrew the arrays every row is empty (so that no
    // later kernel reads past them) and the flag is raised
    const bool over = (uint64_t)E0 > cap;
    const int E = over ? 0 : E0;
    const bool first = blockIdx.x == 0;  // writes the row offsets, the flag and E
#pragma unroll
    for (int j = 0; j < kGsPer; ++j) {
        const int m = j * kGsThreads + t;
        if (m < n) sCum[m] = over ? 0 : sOff[ov[j] + 1] - sOff[ov[j]];
    }
    if (first) {
        for (int i = t; i <= n; i += kGsThreads) offsets[i] = over ? 0 : sOff[i];
        if (t == 0 && overflow) *overflow = over ? 1 : 0;
    }
    // each group's edge share, for the search below
    for (int gi = t; gi < 8 * G; gi += kGsThreads)
        sTgt[gi] = (double)E * (double)sWend[gi] / (8.0 * (double)P);
    __syncthreads();
    gb_lds_scan(sCum, n, sWsum);
    if (8 * G <= kGsFastGroups) {
        // the target position of every group (the search of sched_group_target: the first
        // position whose running sum reaches the share, or the one before it when that is
        // closer), found by the thread whose run holds it: positions m in [8t, 8t + 8),
        // and the last thread also n (sCum[n] = E reaches every share).  A running sum
        // (an integer) reaches the share when it reaches the share rounded up.
        const int m0 = t * kGsPer;
        const int m1 = t == kGsThreads - 1 ? n + 1 : min(m0 + kGsPer, n + 1);
        if (m0 < m1) {
            const int before = m0 > 0 ? sCum[m0 - 1] : -1;
            const int last = sCum[m1 - 1];
            for (int gi = 0; gi < 8 * G; ++gi) {
                const double target = sTgt[gi];
                const int64_t need = (int64_t)ceil(target);
                if (before < need && last >= need) {  // the crossing is in this run
                    int m = m0, prev = before;
                    while (sCum[m] < need) prev = sCum[m++];
                    sPos[gi] = (m > 0 && target - (double)prev < (double)sCum[m] - target) ? m - 1 : m;
                }
            }
        }
    } else {
        for (int gi = t; gi < 8 * G; gi += kGsThreads)
            sPos[gi] = (int)sched_group_target(gi, P, Q, n, (double)E,
                                               [&](int64_t m) { return (int64_t)sCum[m]; });
    }
    __syncthreads();
    if (t == 0) {
        sched_clamp_groups(
            P, Q, R, n, [&](int gi) { return (int64_t)sPos[gi]; },
            [&](int i, int64_t v) { sGb[i] = (int)v; },
            [&](int gi) { return SchedGroup{sQg[gi], 0, (int64_t)sWend[gi]}; });
        if (first) row_ptr_s[(int64_t)8 * P * R] = E;
    }
    __syncthreads();
    // workgroup gi balances group gi with its first four waves (a compute unit of its own)
    const int gi = blockIdx.x;
    const int s0 = sGb[gi], s1 = sGb[gi + 1];
    const int Qg = sQg[gi];
    sched_balance_group<int>(
        w, lane, Qg, R, s1 - s0, sCum[s0], (int64_t)sWend[gi] - Qg,
        [&](int q) { return sCum[s0 + q + 1] - sCum[s0 + q]; },
        [&](int q) -> int64_t { return sOrd[s0 + q]; }, row_dst, row_ptr_s,
        [&](int64_t d, int64_t o) { soff[d] = o; }, sL);
}

// Within the limits of the four-kernel build: atoms, cells, the sweeps' work, and the
// schedule's groups (those of batteries_mp_schedule_shape(N, C)) for its one workgroup.
static bool gb_supported(int64_t N, const BinCfg& c, int C) {
    if (!cells_supported(N, c) || C <= 0) return false;
    int nb = 0, rpb = 0;
    if (batteries_mp_schedule_shape(N, C, &nb, &rpb) != BM_OK) return false;
    const int P = nb / 8, Q = schedule_group_size(nb, C);
    return Q >= 1 && 8 * ((P + Q - 1) / Q) <= kGsMaxGroups;
}

}  // namespace bmhip

using namespace bmhip;

extern "C" size_t batteries_graph_build_workspace_bytes(int64_t N, const float* box, float cutoff,
                                                        int C, int row_capacity) {
    if (N < 0 || !box || !valid_box(box, cutoff) || row_capacity < 0) return 0;
    const BinCfg c = make_bin_cfg(box, cutoff);
    if (!gb_supported(N, c, C)) return 0;
    return gb_layout(N, gb_row_cap(N, box, cutoff, row_capacity)).total;
}

extern "C" int batteries_graph_build_count(const float* positions, const float* box, int64_t N,
                                           float cutoff, int self_loops, int C, int n_blocks,
                                           int rows_per_block, int64_t capacity,
                                           int row_capacity, void* workspace,
                                           size_t workspace_bytes, int64_t* row_offsets,
                                           int64_t* order, int64_t* row_ptr_s, int64_t* row_dst,
                                           int* overflow, hipStream_t stream) {
    if (N < 0 || !box || !valid_box(box, cutoff) || row_capacity < 0 || C <= 0) return BM_ERR_ARG;
    const BinCfg c = make_bin_cfg(box, cutoff);
    if (!gb_supported(N, c, C)) return BM_ERR_ARG;
    if (n_blocks <= 0 || n_blocks % 8 || rows_per_block <= 0 || rows_per_block > kScatterRows ||
        (int64_t)n_blocks * rows_per_block < N)
        return BM_ERR_ARG;
    const int P = n_blocks / 8;
    const int Q = schedule_group_size(n_blocks, C);
    if (Q < 1 || 8 * ((P + Q - 1) / Q) > kGsMaxGroups) return BM_ERR_ARG;
    const int rc = gb_row_cap(N, box, cutoff, row_capacity);
    const GbLayout L = gb_layout(N, rc);
    if (!workspace || workspace_bytes < L.total) return BM_ERR_WORKSPACE;
    if (!row_offsets || !order || !row_ptr_s || !row_dst) return BM_ERR_ARG;
    char* ws = static_cast<char*>(workspace);
    int* pk = reinterpret_cast<int*>(ws + L.pk);
    int* cnt = reinterpret_cast<int*>(ws + L.cnt);
    int64_t* soff = reinterpret_cast<int64_t*>(ws + L.soff);
    float4* slab = reinterpret_cast<float4*>(ws + L.slab);
    const uint64_t cap = capacity < 0 ? ~0ull : (uint64_t)capacity;
    const int n = (int)N;
    gb_bin_kernel<<<(unsigned)ceil_div(N, 256), 256, 0, stream>>>(positions, c, n, pk);
    gb_cell_kernel<<<(unsigned)c.total, kGbBlock, 0, stream>>>(positions, c, n, cutoff * cutoff,
                                                               self_loops, pk, rc, slab, cnt,
                                                               order);
    gb_sched_kernel<<<(unsigned)(8 * ((P + Q - 1) / Q)), kGsThreads, 0, stream>>>(
        cnt, order, n, cap, P, Q, rows_per_block, row_offsets, overflow, row_dst, row_ptr_s, soff);
    return (int)hipGetLastError();
}

extern "C" int batteries_graph_build_write(const float* positions, const float* box, int64_t N,
                                           float cutoff, int self_loops, int row_capacity,
                                           void* workspace, size_t workspace_bytes,
                                           const int64_t* row_offsets, const int* overflow,
                                           int64_t* src, int64_t* dst, float* edge_vectors,
                                           int64_t* edge_perm, hipStream_t stream) {
    if (N < 0 || !box || !valid_box(box, cutoff) || row_capacity < 0) return BM_ERR_ARG;
    const BinCfg c = make_bin_cfg(box, cutoff);
    if (!cells_supported(N, c)) return BM_ERR_ARG;
    const int rc = gb_row_cap(N, box, cutoff, row_capacity);
    const GbLayout L = gb_layout(N, rc);
    if (!workspace || workspace_bytes < L.total || !row_offsets) return BM_ERR_WORKSPACE;
    char* ws = static_cast<char*>(workspace);
    const int* pk = reinterpret_cast<const int*>(ws + L.pk);
    const int* cnt = reinterpret_cast<const int*>(ws + L.cnt);
    const int64_t* soff = reinterpret_cast<const int64_t*>(ws + L.soff);
    const float4* slab = reinterpret_cast<const float4*>(ws + L.slab);
    gb_rows_kernel<false, int64_t><<<(unsigned)ceil_div(N, 4), 256, 0, stream>>>(
        positions, c, (int)N, cutoff * cutoff, self_loops, pk, rc, slab, cnt, row_offsets, soff,
        overflow, src, dst, edge_vectors, edge_perm);
    return (int)hipGetLastError();
}
