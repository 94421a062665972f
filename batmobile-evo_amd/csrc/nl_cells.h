// The cell-list kernels of the four-kernel neighbor list and graph build (graph.hip and,
// for the neighbor list alone, nl.hip), for systems of up to kGbMaxAtoms atoms and
// kGbMaxCells cells with atoms x cells <= kGbMaxSweep:
//
//   gb_bin_kernel    per atom: its cell and the cell's position on the serpentine
//                    path (nl_geom.h), packed in one int.
//   gb_cell_kernel   one workgroup per cell (path position p): a sweep over all the
//                    atoms sets a bit per atom of the 27 stencil cells and per atom of
//                    the cell itself; the bits' ranks list both in atom index order
//                    (each cell of the stencil is distinct with at least three cells
//                    per axis, so every atom is listed at most once).  The sweep also
//                    counts the atoms on earlier path cells, which is where the
//                    cell's atoms start in the spatial order.  Each own atom i then
//                    tests the listed candidates in index order; the kept ones come
//                    out sorted by j, with no sort, and go to row i of a slab of
//                    row_cap entries per atom (edges past row_cap are only counted).
//   gb_rows_kernel   one wave per row: the slab row copied to the edge arrays (and in
//                    the message-passing layout to edge_perm); a row that outgrew its
//                    slab row is found again by a sweep over all atoms in index order,
//                    written in place.
//
// The distances are those of nl.hip (min_image in nl_geom.h), so the neighbor sets and
// vectors are bit-identical to the general passes'.  Replaces, for these systems, the
// reference's binning, count and write passes (src/neighbor_list/neighbor_list.cu:242-430).
// Everything here has internal linkage: each including file has its own copy.
#pragma once

#include "common.h"
#include "nl_geom.h"

namespace bmhip {
namespace {

constexpr int kGbMaxAtoms = 8192;
constexpr int kGbMaxCells = 4096;              // 12-bit cell ids in the packed bins
constexpr int64_t kGbMaxSweep = 1LL << 23;     // atoms x cells: the sweeps' total work
constexpr int kGbWaves = 8;                    // waves per cell
constexpr int kGbBlock = 64 * kGbWaves;
constexpr int kGbPer = kGbMaxAtoms / kGbBlock;  // packed bins held per thread
constexpr int kGbCap = 2048;                   // candidates staged per chunk (32 KB)
constexpr int kGbHomeCap = 256;                // own atoms per chunk
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
                    if (order) order[base_p + h_lo + q] = i;
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

__device__ __forceinline__ bool gb_near(int b, int h, int nb) {
    const int d = b - h;
    return d == 0 || d == 1 || d == -1 || d == nb - 1 || d == 1 - nb;
}

// REF: the neighbor list's own orientation (src = i, dst = j, the vector r_j - r_i;
// edge_perm and soff unused), else the message-passing layout (src = j, dst = i, the
// vector r_i - r_j as the slab holds it, edge_perm at the row's slot offset).
template <bool REF, typename TI>
__global__ __launch_bounds__(256) void gb_rows_kernel(
    const float* __restrict__ pos, BinCfg c, int n, float rc2, int self_loops,
    const int* __restrict__ pk, int row_cap, const float4* __restrict__ slab,
    const int* __restrict__ cnt, const int64_t* __restrict__ offsets,
    const int64_t* __restrict__ soff, const int* __restrict__ overflow, TI* __restrict__ src,
    TI* __restrict__ dst, float* __restrict__ vec, int64_t* __restrict__ edge_perm) {
    const int lane = threadIdx.x & 63;
    const int i = blockIdx.x * 4 + (threadIdx.x >> 6);
    if (i >= n) return;  // uniform per wave
    if (overflow && *overflow) return;
    const int64_t s = offsets[i], so = REF ? 0 : soff[i];
    const int len = cnt[i];
    auto put = [&](int64_t at, int j, float v0, float v1, float v2) {  // v: r_i - r_j
        src[at] = REF ? i : j;
        dst[at] = REF ? j : i;
        vec[at * 3] = REF ? -v0 : v0;
        vec[at * 3 + 1] = REF ? -v1 : v1;
        vec[at * 3 + 2] = REF ? -v2 : v2;
        if (!REF) edge_perm[so + (at - s)] = at;
    };
    if (len <= row_cap) {
        for (int k = lane; k < len; k += 64) {
            const float4 e = slab[(int64_t)i * row_cap + k];
            put(s + k, __float_as_int(e.w), e.x, e.y, e.z);
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
        if (keep) put(s + w + __popcll(m & lanes_below(lane)), a, -d[0], -d[1], -d[2]);
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

// Within the limits of the sweep: atoms, cells and atoms x cells.
static bool cells_supported(int64_t N, const BinCfg& c) {
    return N >= 1 && N <= kGbMaxAtoms && c.total <= kGbMaxCells &&
           N * (int64_t)c.total <= kGbMaxSweep;
}

}  // namespace
}  // namespace bmhip
