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
//     only lane permutes; four waves share a group's slots.
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

// The exchange rounds: in round r workgroup k pairs with workgroup k ^ m_r, and the pair
// exchanges the rows of the one slot whose exchange brings their edge counts closest
// (if any exchange reduces the difference; the first such slot on a tie).
constexpr int kSchedSwapRounds = 8;
__device__ __forceinline__ int sched_swap_mask(int r) { return 32 >> (r % 6); }

// Four waves balance one group: lane k of every wave is workgroup b0 + k (k < Qg <= 64),
// and wave v holds its slots t = v, v + 4, v + 8 in registers.  In a round each wave
// takes the partner's degrees of its slots by lane permutes and proposes its best slot;
// the four proposals meet in LDS (one barrier per round, buffers alternating by round)
// and every wave applies the best, the owner of the slot taking the partner's row.
// Both lanes of a pair see the same values, so they make the same choice.
constexpr int kSchedWaves = 4;
constexpr int kSchedSlotsPerWave = (kScatterRows + kSchedWaves - 1) / kSchedWaves;

template <typename TD>
struct SchedLds {
    int64_t key[2][kSchedWaves][64];  // (round parity, wave, lane): dv * 16 + t of its best slot
    TD d[2][kSchedWaves][64];         // that slot's degree difference
    TD a[kScatterRows][64];           // the final slot degrees
    TD part[kSchedWaves][64];         // the waves' partial loads
};

// Every thread of the workgroup calls it (it holds barriers); waves v >= kSchedWaves take
// part in the barriers only.  The group's rows are positions [0, n) of its range of the
// processing order: deg(r) is the degree of row r, dst(r) its destination (-1: none,
// degree 0); both are called with r clamped into [0, n), so that their loads are all in
// flight together.  base is the number of edges before the group.  Writes row_dst and
// row_ptr_s for the group's slots and calls put_soff(d, offset) for every scheduled
// destination d.
template <typename TD, class DegF, class DstF, class SoffF>
__device__ inline void sched_balance_group(int v, int k, int Qg, int R, int n, int64_t base,
                                           int64_t b0, DegF deg, DstF dst,
                                           int64_t* __restrict__ row_dst,
                                           int64_t* __restrict__ row_ptr_s, SoffF put_soff,
                                           SchedLds<TD>& L) {
    constexpr int J = kSchedSlotsPerWave;
    const int T = n > 0 ? (n + Qg - 1) / Qg : 0;  // <= R: a group holds at most Qg * R rows
    const bool act = v < kSchedWaves;
    int pos[J];
    TD a[J];
    TD part = 0;
    {
        TD dv[J];
        static_for<J>([&](auto jj) {
            constexpr int j = decltype(jj)::value;
            dv[j] = (act && T > 0) ? deg(min((v + 4 * j) * Qg + k, n - 1)) : TD(0);
        });
        static_for<J>([&](auto jj) {
            constexpr int j = decltype(jj)::value;
            const int t = v + 4 * j, p = t * Qg + k;
            const bool live = act && k < Qg && t < T && p < n;
            pos[j] = live ? p : -1;
            a[j] = live ? dv[j] : TD(0);
            part += a[j];
        });
    }
    if (act) L.part[v][k] = part;
    __syncthreads();
    TD load = 0;
    if (act)
#pragma unroll
        for (int q = 0; q < kSchedWaves; ++q) load += L.part[q][k];
    for (int rd = 0; rd < kSchedSwapRounds && T > 0; ++rd) {
        const int m = sched_swap_mask(rd), kp = k ^ m, par = rd & 1;
        TD pa[J];
        bool heavy = false;
        if (act) {
            static_for<J>([&](auto jj) {
                constexpr int j = decltype(jj)::value;
                pa[j] = __shfl_xor(a[j], m, 64);
            });
            const TD pl = __shfl_xor(load, m, 64);
            heavy = load > pl || (load == pl && k > kp);
            const TD diff = heavy ? load - pl : pl - load;
            int64_t bkey = INT64_MAX;
            TD bd = 0;
            static_for<J>([&](auto jj) {
                constexpr int j = decltype(jj)::value;
                const int t = v + 4 * j;
                const TD d = heavy ? a[j] - pa[j] : pa[j] - a[j];
                if (t < T && d > 0 && d < diff) {
                    const TD dv = diff > 2 * d ? diff - 2 * d : 2 * d - diff;
                    const int64_t key = (int64_t)dv * 16 + t;
                    if (key < bkey) {
                        bkey = key;
                        bd = d;
                    }
                }
            });
            L.key[par][v][k] = bkey;
            L.d[par][v][k] = bd;
        }
        __syncthreads();
        if (act) {
            int64_t best = INT64_MAX;
            TD bd = 0;
#pragma unroll
            for (int q = 0; q < kSchedWaves; ++q) {
                const int64_t key = L.key[par][q][k];
                if (key < best) {
                    best = key;
                    bd = L.d[par][q][k];
                }
            }
            const bool swap = k < Qg && kp < Qg && best != INT64_MAX;
            const int tb = swap ? (int)(best & 15) : -1;
            int mine = -1;  // this lane's row in the chosen slot (in its owner wave), for the partner
            static_for<J>([&](auto jj) {
                constexpr int j = decltype(jj)::value;
                if (v + 4 * j == tb) mine = pos[j];
            });
            const int theirs = __shfl_xor(mine, m, 64);
            if (swap) {
                load += heavy ? -bd : bd;
                static_for<J>([&](auto jj) {
                    constexpr int j = decltype(jj)::value;
                    if (v + 4 * j == tb) {
                        a[j] = pa[j];
                        pos[j] = theirs;
                    }
                });
            }
        }
    }
    // destinations of the slots (loads issued together); the slots' degrees to LDS
    int64_t dd[J];
    static_for<J>([&](auto jj) {
        constexpr int j = decltype(jj)::value;
        dd[j] = (act && T > 0) ? dst(max(pos[j], 0)) : -1;
    });
    static_for<J>([&](auto jj) {
        constexpr int j = decltype(jj)::value;
        const int t = v + 4 * j;
        if (pos[j] < 0) dd[j] = -1;
        if (dd[j] < 0) a[j] = 0;
        if (act && t < kScatterRows) L.a[t][k] = a[j];
    });
    __syncthreads();
    if (!act) return;
    // slot offsets: the group's slots follow the edges of the earlier groups, in workgroup
    // order, then slot order
    TD run[kScatterRows + 1];
    run[0] = 0;
#pragma unroll
    for (int t = 0; t < kScatterRows; ++t) run[t + 1] = run[t] + (t < R ? L.a[t][k] : TD(0));
    const int64_t wl = run[kScatterRows];
    int64_t xs;  // inclusive scan of the workgroup loads over the lanes
    if constexpr (sizeof(TD) == 4) {
        xs = wave_incl_scan((int)wl);
    } else {
        xs = wl;
#pragma unroll
        for (int off = 1; off < 64; off <<= 1) {
            const int64_t y = __shfl_up(xs, off, 64);
            if (k >= off) xs += y;
        }
    }
    const int64_t off0 = base + (xs - wl);
    if (k < Qg) {
        const int64_t b = b0 + k;
        static_for<J>([&](auto jj) {
            constexpr int j = decltype(jj)::value;
            const int t = v + 4 * j;
            if (t < R) {
                int64_t o = off0;
                static_for<kScatterRows>([&](auto uu) {
                    constexpr int u = decltype(uu)::value;
                    if (u == t) o += run[u];
                });
                row_dst[b * R + t] = dd[j];
                row_ptr_s[b * R + t] = o;
                if (dd[j] >= 0) put_soff(dd[j], o);
            }
        });
    }
}

}  // namespace bmhip
