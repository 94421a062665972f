// Destination schedule of the fused scatter kernel, shared by the schedule
// kernels (mp.hip) and the one-workgroup schedule of the graph build (graph.hip).
//
// The fused scatter kernel runs n_blocks = 8 P workgroups of R row slots; slot t of
// workgroup b is scheduled row q = b * R + t.  Workgroup b = x * P + k runs on XCD
// x, and the workgroups of an XCD run in generations of Q resident ones.
//
//   - Each (XCD, generation) group owns a contiguous range of the processing (spatial)
//     order, cut so that every group holds edges in proportion to its number of
//     workgroups (at most Qg * R rows).
//   - Inside a group, slot t of workgroup k first takes the group's row t * Qg + k:
//     slice t (Qg consecutive spatial positions) goes to slot t of all the group's
//     workgroups, so the rows in flight on an XCD at one time stay spatially compact
//     and their source rows stay in L2.
//   - kSchedSwapRounds rounds of pairwise exchanges then even out the workgroups'
//     edge counts: workgroup k pairs with k ^ m (m = 32, 16, 8, 4, 2, 1, 32, 16), and
//     the pair exchanges the rows of the one slot whose exchange brings their counts
//     closest (if any exchange reduces the difference).  The pairs need no ranking,
//     only lane permutes.
//
// The kernel time is that of the busiest compute unit, so equal edge counts per
// workgroup matter.  In a host simulation at configs[3] (5000 destinations, 512
// workgroups of 11 slots, 294 edges per workgroup on average, three seeds) the largest
// workgroup holds about 370 edges with the slices alone and 297-298 after the eight
// rounds; pairing the i-th lightest with the i-th heaviest after a ranking of the
// loads (four rounds) gave 296-301 at about three times the cost, and the
// heaviest-row-to-lightest-workgroup dealing used before 298.  On a density gradient
// (387 edges per workgroup on average) the eight rounds give 396, the ranked pairs
// 410, the dealing 413.  Every destination is still summed by one wave in ascending
// edge order, so the result does not depend on the schedule.
#pragma once

#include "common.h"

namespace bmhip {

constexpr int kScatterRows = 11;      // row slots per workgroup
constexpr int kSchedMaxQ = 64;        // workgroups of one group: the lanes of one wave

// Workgroups of one group for a launch of n_blocks workgroups over C channels (mp.hip).
int schedule_group_size(int n_blocks, int C);

// Group gi (of 8 G, G = ceil(P / Q) generations per XCD): its workgroup count Qg,
// its first workgroup and the number of workgroups up to its end.
struct SchedGroup {
    int Qg;
    int64_t b0, w_end;
};
__host__ __device__ inline SchedGroup sched_group(int gi, int P, int Q) {
    const int G = (P + Q - 1) / Q;
    const int x = gi / G, gen = gi - x * G;
    SchedGroup s;
    s.Qg = min(Q, P - gen * Q);
    s.b0 = (int64_t)x * P + (int64_t)gen * Q;
    s.w_end = s.b0 + s.Qg;
    return s;
}

// Target end of group gi: the first position whose running edge count reaches the
// group's share E * w_end / (8 P), or the one before it when that is closer.
// cum(m) is the exclusive running sum at position m (cum(n_dst) = E).
template <class CumF>
__device__ inline int64_t sched_group_target(int gi, int P, int Q, int64_t n_dst, double E,
                                             CumF cum) {
    const SchedGroup s = sched_group(gi, P, Q);
    const double target = E * (double)s.w_end / (8.0 * (double)P);
    int64_t lo = 0, hi = n_dst;
    while (lo < hi) {
        const int64_t mid = (lo + hi) >> 1;
        if ((double)cum(mid) < target) lo = mid + 1;
        else hi = mid;
    }
    if (lo > 0 && target - (double)cum(lo - 1) < (double)cum(lo) - target) --lo;
    return lo;
}

// The targets clamped in group order, by one thread: every group fits its Qg * R
// slots and leaves room for the later groups.  gb[0 .. 8 G] (gb[0] = 0).  group(gi)
// gives sched_group(gi, P, Q) (or the same values precomputed).
template <class TargetF, class PutF, class GroupF>
__device__ inline void sched_clamp_groups(int P, int Q, int R, int64_t n_dst, TargetF target,
                                          PutF put, GroupF group) {
    const int G = (P + Q - 1) / Q;
    const int64_t total_wg = 8LL * P;
    int64_t start = 0;
    put(0, (int64_t)0);
    for (int gi = 0; gi < 8 * G; ++gi) {
        const SchedGroup s = group(gi);
        const int64_t low = max(start, n_dst - (total_wg - s.w_end) * (int64_t)R);
        const int64_t high = min(n_dst, start + (int64_t)s.Qg * R);
        const int64_t pos = max(low, min(high, target(gi)));
        put(gi + 1, pos);
        start = pos;
    }
}
template <class TargetF, class PutF>
__device__ inline void sched_clamp_groups(int P, int Q, int R, int64_t n_dst, TargetF target,
                                          PutF put) {
    sched_clamp_groups(P, Q, R, n_dst, target, put,
                       [&](int gi) { return sched_group(gi, P, Q); });
}

// The exchange rounds: in round r lane k (workgroup k) pairs with lane k ^ m_r, and the
// pair exchanges the rows of the one slot whose exchange brings their edge counts
// closest (if any exchange reduces the difference).  The partner's slot degrees and
// load come by lane permutes; both lanes of a pair compute the same choice from the
// same values, so each takes the partner's row of that slot.
constexpr int kSchedSwapRounds = 8;
__device__ __forceinline__ int sched_swap_mask(int r) { return 32 >> (r % 6); }

template <typename TD>
__device__ inline void sched_swap_rounds(int k, int Qg, int T, int (&pos)[kScatterRows],
                                         TD (&a)[kScatterRows], TD& load) {
#pragma unroll
    for (int rd = 0; rd < kSchedSwapRounds; ++rd) {
        const int m = sched_swap_mask(rd);
        TD pa[kScatterRows];
        static_for<kScatterRows>([&](auto tt) {
            constexpr int t = decltype(tt)::value;
            pa[t] = __shfl_xor(a[t], m, 64);
        });
        const TD pl = __shfl_xor(load, m, 64);
        const int kp = k ^ m;
        const bool heavy = load > pl || (load == pl && k > kp);
        const TD diff = heavy ? load - pl : pl - load;
        int best = -1;
        TD bv = diff;
        static_for<kScatterRows>([&](auto tt) {
            constexpr int t = decltype(tt)::value;
            if (t < T) {
                const TD d = heavy ? a[t] - pa[t] : pa[t] - a[t];
                if (d > 0 && d < diff) {
                    const TD dv = diff > 2 * d ? diff - 2 * d : 2 * d - diff;
                    if (dv < bv) {
                        bv = dv;
                        best = t;
                    }
                }
            }
        });
        int mine = -1;  // this lane's row in the chosen slot, for the partner
        static_for<kScatterRows>([&](auto tt) {
            constexpr int t = decltype(tt)::value;
            if (t == best) mine = pos[t];
        });
        const int theirs = __shfl_xor(mine, m, 64);
        if (k < Qg && kp < Qg && best >= 0) {
            static_for<kScatterRows>([&](auto tt) {
                constexpr int t = decltype(tt)::value;
                if (t == best) {
                    const TD d = heavy ? a[t] - pa[t] : pa[t] - a[t];
                    a[t] = pa[t];
                    pos[t] = theirs;
                    load += heavy ? -d : d;
                }
            });
        }
    }
}

// One wave balances one group: lane k is workgroup b0 + k (k < Qg <= 64), holding
// its R slots in registers.  The group's rows are positions [0, n) of its range of
// the processing order: deg(r) is the degree of row r, dst(r) its destination (-1:
// none, degree 0); both are called for every slot with r clamped into [0, n), so
// that their loads are all in flight together.  base is the number of edges before
// the group.  Writes row_dst and row_ptr_s for the group's slots and calls
// put_soff(d, offset) for every scheduled destination d.
template <typename TD, class DegF, class DstF, class SoffF>
__device__ inline void sched_balance_wave(int k, int Qg, int R, int n, int64_t base, int64_t b0,
                                          DegF deg, DstF dst, int64_t* __restrict__ row_dst,
                                          int64_t* __restrict__ row_ptr_s, SoffF put_soff) {
    const int T = n > 0 ? (n + Qg - 1) / Qg : 0;  // <= R: a group holds at most Qg * R rows
    int pos[kScatterRows];
    TD a[kScatterRows];
    TD load = 0;
    if (T > 0) {
        TD dv[kScatterRows];
        static_for<kScatterRows>([&](auto tt) {
            constexpr int t = decltype(tt)::value;
            dv[t] = deg(min(t * Qg + k, n - 1));
        });
        static_for<kScatterRows>([&](auto tt) {
            constexpr int t = decltype(tt)::value;
            const int p = t * Qg + k;
            const bool live = k < Qg && t < T && p < n;
            pos[t] = live ? p : -1;
            a[t] = live ? dv[t] : TD(0);
            load += a[t];
        });
        sched_swap_rounds(k, Qg, T, pos, a, load);
    } else {
        static_for<kScatterRows>([&](auto tt) {
            constexpr int t = decltype(tt)::value;
            pos[t] = -1;
            a[t] = 0;
        });
    }
    // destinations of the slots (loads issued together), then the slot offsets: the
    // group's slots follow the edges of the earlier groups, in workgroup order
    int64_t dd[kScatterRows];
    static_for<kScatterRows>([&](auto tt) {
        constexpr int t = decltype(tt)::value;
        dd[t] = T > 0 ? dst(max(pos[t], 0)) : -1;
    });
    int64_t wl = 0;
    static_for<kScatterRows>([&](auto tt) {
        constexpr int t = decltype(tt)::value;
        if (pos[t] < 0) dd[t] = -1;
        if (dd[t] < 0) a[t] = 0;
        wl += a[t];
    });
    int64_t xs = wl;  // inclusive scan of the workgroup loads over the lanes
#pragma unroll
    for (int off = 1; off < 64; off <<= 1) {
        const int64_t y = __shfl_up(xs, off, 64);
        if (k >= off) xs += y;
    }
    int64_t off = base + (xs - wl);
    if (k < Qg) {
        const int64_t b = b0 + k;
        static_for<kScatterRows>([&](auto tt) {
            constexpr int t = decltype(tt)::value;
            if (t < R) {
                row_dst[b * R + t] = dd[t];
                row_ptr_s[b * R + t] = off;
                if (dd[t] >= 0) put_soff(dd[t], off);
                off += a[t];
            }
        });
    }
}

}  // namespace bmhip
