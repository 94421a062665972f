// Graph build for the fused message-passing kernels in four kernels: the neighbor
// list in the message-passing layout (edges grouped by destination, sources
// ascending), the spatial order of the atoms and the processing schedule of the
// fused scatter kernel, for systems of up to kGbMaxAtoms atoms.
//
// Replaces, for batmobile.Graph, the cell-list passes of nl.hip (binning, count,
// scan, write, row sort: reference src/neighbor_list/neighbor_list.cu:242-430 and
// the e2e pipeline's per-step neighbor list, benchmarks/benchmark_e2e_mace.py:192-278),
// the serpentine order and batteries_mp_schedule (mp.hip), with the same results:
//
//   gb_bin_kernel    per atom: its cell and the cell's position on the serpentine
//                    path (nl_geom.h), packed in one int.
//   gb_cell_kernel   one workgroup per cell (path position p): a sweep over all the
//                    atoms sets a bit per atom of the 27 stencil cells and per atom of
//                    the cell itself; the bits' ranks list both in atom index order
//                    (each cell of the stencil is distinct with at least three cells
//                    per axis, so every atom is listed at most once).  The sweep also
//                    counts the atoms on earlier path cells, which is where the
//                    cell's atoms start in the spatial order.  Each own
//                    atom i then tests the listed candidates in index order; the kept
//                    ones come out sorted by j, with no sort, and go to row i of a
//                    slab of row_cap entries per atom (edges past row_cap are only
//                    counted).
//   gb_sched_kernel  one workgroup per schedule group: each computes the row offsets
//                    (exclusive sums of the counts), the degrees in spatial order and
//                    their sums and the group bounds in LDS, then balances its group
//                    (mp_schedule.h) with four waves on a compute unit of its own and
//                    writes every scheduled destination's slot offset for the next
//                    kernel; the first one writes the row offsets.
//   gb_rows_kernel   one wave per row: the slab row copied to the edge arrays and to
//                    edge_perm (the slot offsets); a row that outgrew its slab row is
//                    found again by a sweep over all atoms in index order, written in
//                    place.
//
// The distances are those of nl.hip (min_image in nl_geom.h), so the edges, vectors,
// row offsets, order and schedule are bit-identical to the general path's.
#include "common.h"
#include "batmobile_hip.h"
#include "nl_geom.h"
#include "mp_schedule.h"

namespace bmhip {

constexpr int kGbMaxAtoms = 8192;
constexpr int kGbMaxCells = 4096;              // 12-bit cell ids in the packed bins
constexpr int64_t kGbMaxSweep = 1LL << 23;     // atoms x cells: the sweeps' total work
constexpr int kGbWaves = 8;                    // waves per cell
constexpr int kGbBlock = 64 * kGbWaves;
constexpr int kGbPer = kGbMaxAtoms / kGbBlock;  // packed bins held per thread
constexpr int kGbCap = 2048;                   // candidates staged per chunk (32 KB)
constexpr int kGbHomeCap = 256;                // own atoms per chunk
constexpr int kGsThreads = 1024;               // the schedule workgroup
constexpr int kGsPer = kGbMaxAtoms / kGsThreads;
constexpr int kGsMaxGroups = 256;               // schedule groups (8 per generation)
constexpr int kGsFastGroups = 32;               // up to this many: targets found in parallel

__device__ __forceinline__ uint64_t lanes_below(int lane) { return (1ull << lane) - 1ull; }

__global__ __launch_bounds__(256) void gb_bin_kernel(const float* __restrict__ pos, BinCfg c,
                                                     int n, int* __restrict__ pk) {
    const int i = blockIdx.x * 256 + threadIdx.x;
    if (i >= n) return;
    int b[3];
    bin_coords(pos[(int64_t)i * 3], pos[(int64_t)i * 3 + 1], pos[(int64_t)i * 3 + 2], c, b);
    const int cell = b[0] + b[1] * c.nb[0] + b[2] * c.nb[0] * c.nb[1];
    pk[i] = cell | (serpentine_pos(b[0], b[1], b[2], c) << 12);
}

__global__ __launch_bounds__(kGbBlock) void gb_cell_kernel(
    const float* __restrict__ pos, BinCfg c, int n, float rc2, int self_loops,
    const int* __restrict__ pk, int row_cap, float4* __restrict__ slab, int* __restrict__ cnt,
    int64_t* __restrict__ order) {
    constexpr int kWords = kGbMaxAtoms / 32;  // bitmap words: one per thread of the first ones
    static_assert(kWords <= kGbBlock, "one bitmap word per thread");
    __shared__ float4 sCand[kGbCap];
    __shared__ int sCidx[kGbCap];
    __shared__ float4 sHome[kGbHomeCap];
    __shared__ int sHidx[kGbHomeCap];
    __shared__ int sW[kGbHomeCap];
    __shared__ uint32_t sBits[kGbMaxCells / 32];  // the 27 stencil cells
    __shared__ uint32_t sMem[kWords];             // atoms in the stencil cells (members)
    __shared__ uint32_t sOwn[kWords];             // atoms in this cell
    __shared__ int sWave[kGbWaves];
    __shared__ int sBef[kGbWaves];
    const int t = threadIdx.x, lane = t & 63;
    const int wv = __builtin_amdgcn_readfirstlane(t >> 6);
    const int p = blockIdx.x;
    const int hc = serpentine_cell(p, c);
    const int nx = c.nb[0], ny = c.nb[1], nz = c.nb[2];
    const int hx = hc % nx, hy = (hc / nx) % ny, hz = hc / (nx * ny);
    // atom (wv + kGbWaves k) * 64 + lane in slot k: every packed bin loaded up front
    // (clamped, unconditional)
    int v[kGbPer];
#pragma unroll
    for (int k = 0; k < kGbPer; ++k) {
        const int a = (wv + kGbWaves * k) * 64 + lane;
        v[k] = pk[min(a, n - 1)];
        if (a >= n) v[k] = -1;
    }
    for (int q = t; q < kGbMaxCells / 32; q += kGbBlock) sBits[q] = 0;
    if (t < kWords) {
        sMem[t] = 0;
        sOwn[t] = 0;
    }
    __syncthreads();
    if (t < 27) {
        const int dz = t / 9 - 1, dy = (t / 3) % 3 - 1, dx = t % 3 - 1;
        const int kk = wrap_bin(hx + dx, nx) + wrap_bin(hy + dy, ny) * nx +
                       wrap_bin(hz + dz, nz) * nx * ny;
        atomicOr(&sBits[kk >> 5], 1u << (kk & 31));
    }
    __syncthreads();
    // The sweep: each atom of a stencil cell sets its bit in sMem, each atom of this
    // cell in sOwn, so that the bit ranks give both lists in atom index order; the
    // atoms on earlier path cells are counted (where this cell's atoms start in the
    // spatial order).
    int bef = 0;
    static_for<kGbPer>([&](auto kk) {
        constexpr int k = decltype(kk)::value;
        const int x = v[k];
        const int cell = x & 0xfff;
        const uint32_t word = sBits[cell >> 5];
        const int a = (wv + kGbWaves * k) * 64 + lane;
        if (x >= 0) {
            if ((word >> (cell & 31)) & 1u) atomicOr(&sMem[a >> 5], 1u << (a & 31));
            if (cell == hc) atomicOr(&sOwn[a >> 5], 1u << (a & 31));
            bef += (x >> 12) < p ? 1 : 0;
        }
    });
    bef = wave_incl_scan(bef);
    if (lane == 63) sBef[wv] = bef;
    __syncthreads();
    // ranks: word t's members and own atoms follow those of the words before it (packed
    // counts, members | own << 16, scanned over the workgroup)
    const uint32_t mw = t < kWords ? sMem[t] : 0u, ow = t < kWords ? sOwn[t] : 0u;
    const int cw = __popc(mw) | (__popc(ow) << 16);
    const int incl = wave_incl_scan(cw);
    if (lane == 63) sWave[wv] = incl;
    __syncthreads();
    int before = 0, tot = 0;
    int base_p = 0;
#pragma unroll
    for (int q = 0; q < kGbWaves; ++q) {
        before += q < wv ? sWave[q] : 0;
        tot += sWave[q];
        base_p += sBef[q];
    }
    const int excl = before + incl - cw;
    const int T = tot & 0xffff, H = tot >> 16;
    if (H == 0) return;  // uniform: no atoms in this cell
    // lists the members with rank in [c_lo, c_lo + kGbCap) and the own atoms with rank
    // in [h_lo, h_lo + kGbHomeCap) from this thread's words
    auto extract = [&](int c_lo, int h_lo) {
        uint32_t m = mw;
        int r = (excl & 0xffff) - c_lo;
        while (m) {
            const int bit = __ffs(m) - 1;
            if (r >= 0 && r < kGbCap) sCidx[r] = t * 32 + bit;
            ++r;
            m &= m - 1;
        }
        m = ow;
        r = (excl >> 16) - h_lo;
        while (m) {
            const int bit = __ffs(m) - 1;
            if (r >= 0 && r < kGbHomeCap) sHidx[r] = t * 32 + bit;
            ++r;
            m &= m - 1;
        }
    };
    // own atoms in chunks of kGbHomeCap, each against the members in chunks of kGbCap
    // (one chunk of each unless the system is denser than any at an interatomic cutoff)
    for (int h_lo = 0; h_lo < H; h_lo += kGbHomeCap) {
        const int nh = min(kGbHomeCap, H - h_lo);
        for (int c_lo = 0; c_lo < T; c_lo += kGbCap) {
            const int nc = min(kGbCap, T - c_lo);
            if (h_lo > 0 || c_lo > 0) __syncthreads();  // the previous chunk is processed
            extract(c_lo, h_lo);
            __syncthreads();
            for (int q = t; q < nc; q += kGbBlock) {
                const int64_t j = sCidx[q];
                sCand[q] = make_float4(pos[j * 3], pos[j * 3 + 1], pos[j * 3 + 2],
                                       __int_as_float((int)j));
            }
            if (c_lo == 0)
                for (int q = t; q < nh; q += kGbBlock) {
                    const int64_t i = sHidx[q];
                    sHome[q] = make_float4(pos[i * 3], pos[i * 3 + 1], pos[i * 3 + 2],
                                           __int_as_float((int)i));
                    order[base_p + h_lo + q] = i;
                }
            __syncthreads();
            const bool last = c_lo + kGbCap >= T;
            for (int hh = wv; hh < nh; hh += kGbWaves) {
                const float4 ci = sHome[hh];
                const int i = __builtin_amdgcn_readfirstlane(__float_as_int(ci.w));
                const float pi[3] = {ci.x, ci.y, ci.z};
                int w = c_lo == 0 ? 0 : sW[hh];
                // candidates 64 at a time, the next batch's read issued before this
                // batch's tests (past the end it rereads the last candidate, unused)
                float4 nxt = sCand[min(lane, nc - 1)];
                for (int c0 = 0; c0 < nc; c0 += 64) {
                    const float4 cj = nxt;
                    nxt = sCand[min(c0 + 64 + lane, nc - 1)];
                    const int j = __float_as_int(cj.w);
                    const float pj[3] = {cj.x, cj.y, cj.z};
                    float d[3];
                    const float r2 = min_image(pi, pj, c, d);
                    const bool keep = c0 + lane < nc && (self_loops || j != i) && r2 <= rc2;
                    const uint64_t m = __ballot(keep);
                    const int at = w + __popcll(m & lanes_below(lane));
                    if (keep && at < row_cap)
                        slab[(int64_t)i * row_cap + at] =
                            make_float4(-d[0], -d[1], -d[2], __int_as_float(j));
                    w += __popcll(m);
                }
                if (lane == 0) {
                    if (last) cnt[i] = w;
                    else sW[hh] = w;
                }
            }
        }
    }
}

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

__device__ __forceinline__ bool gb_near(int b, int h, int nb) {
    const int d = b - h;
    return d == 0 || d == 1 || d == -1 || d == nb - 1 || d == 1 - nb;
}

__global__ __launch_bounds__(256) void gb_rows_kernel(
    const float* __restrict__ pos, BinCfg c, int n, float rc2, int self_loops,
    const int* __restrict__ pk, int row_cap, const float4* __restrict__ slab,
    const int* __restrict__ cnt, const int64_t* __restrict__ offsets,
    const int64_t* __restrict__ soff, const int* __restrict__ overflow, int64_t* __restrict__ src,
    int64_t* __restrict__ dst, float* __restrict__ vec, int64_t* __restrict__ edge_perm) {
    const int lane = threadIdx.x & 63;
    const int i = blockIdx.x * 4 + (threadIdx.x >> 6);
    if (i >= n) return;  // uniform per wave
    if (overflow && *overflow) return;
    const int64_t s = offsets[i], so = soff[i];
    const int len = cnt[i];
    if (len <= row_cap) {
        for (int k = lane; k < len; k += 64) {
            const float4 e = slab[(int64_t)i * row_cap + k];
            const int64_t at = s + k;
            src[at] = __float_as_int(e.w);
            dst[at] = i;
            vec[at * 3] = e.x;
            vec[at * 3 + 1] = e.y;
            vec[at * 3 + 2] = e.z;
            edge_perm[so + k] = at;
        }
        return;
    }
    // the row outgrew its slab row: every atom in index order, tested for the stencil
    // and the cutoff, kept ones written at their place
    const int nx = c.nb[0], ny = c.nb[1], nz = c.nb[2];
    const int hc = pk[i] & 0xfff;
    const int hx = hc % nx, hy = (hc / nx) % ny, hz = hc / (nx * ny);
    const float pi[3] = {pos[(int64_t)i * 3], pos[(int64_t)i * 3 + 1], pos[(int64_t)i * 3 + 2]};
    int64_t w = 0;
    for (int a0 = 0; a0 < n; a0 += 64) {
        const int a = a0 + lane;
        bool keep = false;
        float d[3] = {0.f, 0.f, 0.f};
        if (a < n) {
            const int cell = pk[a] & 0xfff;
            const int bx = cell % nx, by = (cell / nx) % ny, bz = cell / (nx * ny);
            if (gb_near(bx, hx, nx) && gb_near(by, hy, ny) && gb_near(bz, hz, nz)) {
                const float pj[3] = {pos[(int64_t)a * 3], pos[(int64_t)a * 3 + 1],
                                     pos[(int64_t)a * 3 + 2]};
                keep = (self_loops || a != i) && min_image(pi, pj, c, d) <= rc2;
            }
        }
        const uint64_t m = __ballot(keep);
        if (keep) {
            const int64_t k = w + __popcll(m & lanes_below(lane));
            src[s + k] = a;
            dst[s + k] = i;
            vec[(s + k) * 3] = -d[0];
            vec[(s + k) * 3 + 1] = -d[1];
            vec[(s + k) * 3 + 2] = -d[2];
            edge_perm[so + k] = s + k;
        }
        w += __popcll(m);
    }
}

struct GbLayout {
    size_t pk, cnt, soff, slab, total;
};
static GbLayout gb_layout(int64_t n, int row_cap) {
    auto al = [](size_t x) { return (x + 255) & ~size_t(255); };
    GbLayout L;
    size_t o = 0;
    L.pk = o; o = al(o + sizeof(int) * (size_t)n);
    L.cnt = o; o = al(o + sizeof(int) * (size_t)n);
    L.soff = o; o = al(o + sizeof(int64_t) * (size_t)n);
    L.slab = o; o = al(o + sizeof(float4) * (size_t)n * (size_t)row_cap);
    L.total = o;
    return L;
}

// Within the limits of the four-kernel build: atoms, cells, the sweeps' work, and the
// schedule's groups (those of batteries_mp_schedule_shape(N, C)) for its one workgroup.
static bool gb_supported(int64_t N, const BinCfg& c, int C) {
    if (!(N >= 1 && N <= kGbMaxAtoms && c.total <= kGbMaxCells &&
          N * (int64_t)c.total <= kGbMaxSweep && C > 0))
        return false;
    int nb = 0, rpb = 0;
    if (batteries_mp_schedule_shape(N, C, &nb, &rpb) != BM_OK) return false;
    const int P = nb / 8, Q = schedule_group_size(nb, C);
    return Q >= 1 && 8 * ((P + Q - 1) / Q) <= kGsMaxGroups;
}

// Slab row capacity from the density: twice the expected neighbor count plus 16,
// in multiples of 16, between 32 and 1024 entries (rows past it are found again
// by gb_rows_kernel, correct at any density).
static int gb_row_cap(int64_t N, const float* box, float cutoff, int requested) {
    if (requested > 0) return requested;
    const double vol = (double)box[0] * (double)box[1] * (double)box[2];
    const double expect = (double)N / vol * 4.18879020478639 * (double)cutoff * cutoff * cutoff;
    int cap = (int)(2.0 * expect + 16.0);
    cap = (cap + 15) & ~15;
    return std::min(1024, std::max(32, cap));
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
    if (!(N >= 1 && N <= kGbMaxAtoms && c.total <= kGbMaxCells)) return BM_ERR_ARG;
    const int rc = gb_row_cap(N, box, cutoff, row_capacity);
    const GbLayout L = gb_layout(N, rc);
    if (!workspace || workspace_bytes < L.total || !row_offsets) return BM_ERR_WORKSPACE;
    char* ws = static_cast<char*>(workspace);
    const int* pk = reinterpret_cast<const int*>(ws + L.pk);
    const int* cnt = reinterpret_cast<const int*>(ws + L.cnt);
    const int64_t* soff = reinterpret_cast<const int64_t*>(ws + L.soff);
    const float4* slab = reinterpret_cast<const float4*>(ws + L.slab);
    gb_rows_kernel<<<(unsigned)ceil_div(N, 4), 256, 0, stream>>>(
        positions, c, (int)N, cutoff * cutoff, self_loops, pk, rc, slab, cnt, row_offsets, soff,
        overflow, src, dst, edge_vectors, edge_perm);
    return (int)hipGetLastError();
}
