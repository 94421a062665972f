// Cell-list neighbor list with periodic (orthorhombic) boundaries, and the
// exclusive prefix scan used by it and by the CSR conversion.
//
// Replaces reference src/neighbor_list/neighbor_list.cu:18-478.
// Same geometry as the reference: box = cell diagonal, bins per axis =
// max(3, int(L / r_c)), bin = min(int(wrap(p) / b), bins - 1) with
// wrap(p) = p - floorf(p * (1/L)) * L, minimum image d -= rintf(d * (1/L)) * L,
// keep d.d <= r_c^2 (inclusive), j != i unless self loops, emit src = i,
// dst = j, vec = d grouped by i.
//
// Unlike the reference the result is deterministic: atoms inside a bin are
// ordered by index and each atom's neighbors are sorted by j, so the output is
// sorted by (i, j).  All distance arithmetic is evaluated without FMA
// contraction in one fixed order, so the kept pairs are a function of the
// fp32 inputs alone.
#include "common.h"
#include "batmobile_hip.h"
#include "nl_geom.h"
#include "nl_cells.h"

#include <cstring>
#include <vector>

namespace bmhip {

__global__ void nl_zero_i32_kernel(int* __restrict__ p, int64_t n) {
    const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (i < n) p[i] = 0;
}

__global__ void nl_assign_kernel(const float* __restrict__ pos, BinCfg c, int* __restrict__ bin_of,
                                 int* __restrict__ bin_count, int64_t n) {
    const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (i >= n) return;
    int b[3];
    bin_coords(pos[i * 3], pos[i * 3 + 1], pos[i * 3 + 2], c, b);
    const int k = b[0] + b[1] * c.nb[0] + b[2] * c.nb[0] * c.nb[1];
    bin_of[i] = k;
    atomicAdd(bin_count + k, 1);
}

__global__ void nl_place_kernel(const int* __restrict__ bin_of, const int64_t* __restrict__ bin_start,
                                int* __restrict__ cursor, int* __restrict__ order, int64_t n) {
    const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (i >= n) return;
    const int k = bin_of[i];
    const int pos = atomicAdd(cursor + k, 1);
    order[bin_start[k] + pos] = (int)i;
}

// ascending atom index inside each bin
__global__ void nl_sort_bins_kernel(const int64_t* __restrict__ bin_start, int* __restrict__ order,
                                    int total) {
    const int k = blockIdx.x * blockDim.x + threadIdx.x;
    if (k >= total) return;
    const int64_t s = bin_start[k], e = bin_start[k + 1];
    for (int64_t i = s + 1; i < e; ++i) {
        const int v = order[i];
        int64_t j = i - 1;
        while (j >= s && order[j] > v) {
            order[j + 1] = order[j];
            --j;
        }
        order[j + 1] = v;
    }
}

// The same with one wave per bin (bins of a few atoms each, as many bins as a few
// workgroups per compute unit): each atom index goes to its rank, the number of
// smaller indices in the bin (indices in a bin are distinct).  Bins of at most
// kBinSortCap atoms are staged in LDS and written back in place.  Larger bins
// (cells much larger than the density needs) are ranked against the bin read
// again from memory, 64 indices at a time, into spare[] (the binning's per-atom
// bin array, free once the atoms are placed), then copied back.
constexpr int kBinSortCap = 1024;
__global__ __launch_bounds__(64) void nl_sort_bins_wave_kernel(const int64_t* __restrict__ bin_start,
                                                               int* __restrict__ order,
                                                               int* __restrict__ spare, int total) {
    __shared__ int sv[kBinSortCap];
    const int k = blockIdx.x;
    if (k >= total) return;
    const int64_t s = bin_start[k];
    const int n = (int)(bin_start[k + 1] - s);
    const int lane = threadIdx.x;
    if (n <= 1) return;
    if (n > kBinSortCap) {
        for (int base = 0; base < n; base += 64) {
            const int a = base + lane;
            const int v = a < n ? order[s + a] : 0;
            int r = 0;
            for (int c0 = 0; c0 < n; c0 += 64) {
                const int x = c0 + lane < n ? order[s + c0 + lane] : 0;
                const int m_end = min(64, n - c0);
                for (int m = 0; m < m_end; ++m) r += __builtin_amdgcn_readlane(x, m) < v ? 1 : 0;
            }
            if (a < n) spare[s + r] = v;
        }
        __syncthreads();  // the wave's stores to spare[] are complete and visible to it
        for (int i = lane; i < n; i += 64) order[s + i] = spare[s + i];
        return;
    }
    for (int i = lane; i < n; i += 64) sv[i] = order[s + i];
    __syncthreads();
    for (int i = lane; i < n; i += 64) {
        const int v = sv[i];
        int r = 0;
        for (int u = 0; u < n; ++u) r += sv[u] < v ? 1 : 0;
        order[s + r] = v;
    }
}

// Binning of a small system in one workgroup, in place of the zero / assign /
// scan / zero / place / sort-bins sequence (six launches of a few microseconds
// each) when the atoms and bins fit in LDS: bins counted with LDS atomics and
// scanned in LDS, atoms placed in arbitrary order within their bin, then each
// atom written at its bin's start plus its rank in the bin (the number of its
// atoms with a smaller index).  The same bin_start and order as the sequence.
constexpr int kBinSmallBlock = 1024;
constexpr int kBinSmallAtoms = 8192;
constexpr int kBinSmallBins = 4096;
constexpr int kBinSmallPer = kBinSmallAtoms / kBinSmallBlock;  // atoms per thread
static_assert(kBinSmallBins == 4 * kBinSmallBlock, "four bins per thread in the scan");

__global__ __launch_bounds__(kBinSmallBlock) void nl_bin_small_kernel(
    const float* __restrict__ pos, BinCfg c, int n, int64_t* __restrict__ bin_start,
    int* __restrict__ order) {
    __shared__ int sCnt[kBinSmallBins];
    __shared__ int sStart[kBinSmallBins + 1];
    __shared__ int sPlace[kBinSmallAtoms];
    __shared__ int sWave[kBinSmallBlock / 64];
    const int t = threadIdx.x, lane = t & 63, wv = t >> 6;
    const int total = c.total;
    // every position load issued before any is used (clamped, unconditional: a load
    // under a branch would be waited for before the next one is issued)
    float p[kBinSmallPer][3];
#pragma unroll
    for (int j = 0; j < kBinSmallPer; ++j) {
        const int64_t i = max(min(t + j * kBinSmallBlock, n - 1), 0);
#pragma unroll
        for (int d = 0; d < 3; ++d) p[j][d] = n > 0 ? pos[i * 3 + d] : 0.0f;
    }
    for (int k = t; k < kBinSmallBins; k += kBinSmallBlock) sCnt[k] = 0;
    __syncthreads();
    int bin[kBinSmallPer];
#pragma unroll
    for (int j = 0; j < kBinSmallPer; ++j) {
        bin[j] = -1;
        if (t + j * kBinSmallBlock < n) {
            int b[3];
            bin_coords(p[j][0], p[j][1], p[j][2], c, b);
            bin[j] = b[0] + b[1] * c.nb[0] + b[2] * c.nb[0] * c.nb[1];
            atomicAdd(&sCnt[bin[j]], 1);
        }
    }
    __syncthreads();
    // exclusive scan of the counts: four bins per thread, shuffles within a wave,
    // then the wave totals
    int v[4], sum = 0;
#pragma unroll
    for (int q = 0; q < 4; ++q) {
        v[q] = sCnt[4 * t + q];
        sum += v[q];
    }
    int incl = sum;
#pragma unroll
    for (int off = 1; off < 64; off <<= 1) {
        const int u = __shfl_up(incl, off, 64);
        if (lane >= off) incl += u;
    }
    if (lane == 63) sWave[wv] = incl;
    __syncthreads();
    int base = 0;
    for (int w = 0; w < wv; ++w) base += sWave[w];
    int run = base + incl - sum;
#pragma unroll
    for (int q = 0; q < 4; ++q) {
        const int k = 4 * t + q;
        sStart[k] = run;
        if (k < total) bin_start[k] = run;
        sCnt[k] = 0;  // the placement cursor from here on
        run += v[q];
    }
    if (t == 0) {
        sStart[kBinSmallBins] = n;
        bin_start[total] = n;
    }
    __syncthreads();
    // every placement's atomic issued before the writes that use them
    int slot[kBinSmallPer];
#pragma unroll
    for (int j = 0; j < kBinSmallPer; ++j)
        slot[j] = bin[j] >= 0 ? sStart[bin[j]] + atomicAdd(&sCnt[bin[j]], 1) : 0;
#pragma unroll
    for (int j = 0; j < kBinSmallPer; ++j)
        if (bin[j] >= 0) sPlace[slot[j]] = t + j * kBinSmallBlock;
    __syncthreads();
    // rank in the bin, four LDS reads in flight per step
#pragma unroll
    for (int j = 0; j < kBinSmallPer; ++j) {
        if (bin[j] < 0) continue;
        const int i = t + j * kBinSmallBlock;
        const int b0 = sStart[bin[j]], b1 = sStart[bin[j] + 1];
        int r = 0;
        for (int u = b0; u < b1; u += 4) {
            int x[4];
#pragma unroll
            for (int q = 0; q < 4; ++q) x[q] = sPlace[min(u + q, b1 - 1)];
#pragma unroll
            for (int q = 0; q < 4; ++q) r += (u + q < b1 && x[q] < i) ? 1 : 0;
        }
        order[b0 + r] = i;
    }
}

// ---------------------------------------------------------------------------
// Stencil passes (count, then write): one workgroup of kNlWaves waves per home
// cell.  The atoms of the 27 cells around it (reference order: dz, dy, dx from
// -1 to 1, atoms of a cell in ascending index) are staged in LDS as (x, y, z, j)
// by all its threads; then each wave takes every kNlWaves-th home atom i (read
// from the staged home cell), its lanes test 64 candidates at a time, and a
// ballot gives every kept pair its slot, so row i lists its neighbors in stencil
// order.  Candidate lists longer than the LDS buffer are processed in chunks.
// esrc may be null (the row is the source).
// ---------------------------------------------------------------------------
constexpr int kNlCap = 2048;  // candidates staged per chunk (32 KB)
constexpr int kNlWaves = 4;   // waves per cell

template <bool WRITE>
__global__ __launch_bounds__(64 * kNlWaves) void nl_cell_kernel(const float* __restrict__ pos, BinCfg c,
                                                                float rc2, int self_loops,
                                                                const int64_t* __restrict__ bin_start,
                                                                const int* __restrict__ order,
                                                                int64_t* __restrict__ counts,
                                                                const int64_t* __restrict__ offsets,
                                                                int* __restrict__ esrc,
                                                                int* __restrict__ edst,
                                                                float* __restrict__ evec,
                                                                uint64_t cap) {
    __shared__ float4 sCand[kNlCap];
    __shared__ int sStart[27], sPre[28];
    const int tid = threadIdx.x, lane = tid & 63;
    const int wv = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int k = blockIdx.x;
    const int bx = k % c.nb[0], by = (k / c.nb[0]) % c.nb[1], bz = k / (c.nb[0] * c.nb[1]);
    if (wv == 0) {
        int cnt_l = 0;
        if (lane < 27) {
            const int dz = lane / 9 - 1, dy = (lane / 3) % 3 - 1, dx = lane % 3 - 1;
            const int kk = wrap_bin(bx + dx, c.nb[0]) + wrap_bin(by + dy, c.nb[1]) * c.nb[0] +
                           wrap_bin(bz + dz, c.nb[2]) * c.nb[0] * c.nb[1];
            const int64_t s0 = bin_start[kk];
            sStart[lane] = (int)s0;
            cnt_l = (int)(bin_start[kk + 1] - s0);
        }
        // exclusive prefix of the 27 counts (wave-level, lanes 0..26)
        int incl = cnt_l;
#pragma unroll
        for (int off = 1; off < 32; off <<= 1) {
            const int v = __shfl_up(incl, off, 64);
            if (lane >= off) incl += v;
        }
        if (lane < 27) sPre[lane] = incl - cnt_l;
        if (lane == 26) sPre[27] = incl;
    }
    __syncthreads();
    const int T = sPre[27];
    const int home0 = sStart[13], H = sPre[14] - sPre[13];
    if (H == 0) return;  // uniform: no home atoms (the home cell is entry 13 of the stencil)

    // stage candidates [base, base + n) of the concatenated 27-cell list, all waves
    auto stage = [&](int base, int n) {
        for (int t = tid; t < n; t += 64 * kNlWaves) {
            const int idx = base + t;
            int cell = 0;
#pragma unroll
            for (int q = 1; q < 27; ++q) cell += sPre[q] <= idx ? 1 : 0;
            const int j = order[sStart[cell] + (idx - sPre[cell])];
            sCand[t] = make_float4(pos[(int64_t)j * 3], pos[(int64_t)j * 3 + 1],
                                   pos[(int64_t)j * 3 + 2], __int_as_float(j));
        }
    };
    // home atom hh against candidates [0, n) of the staged chunk; w counts its neighbors
    auto scan_cands = [&](int i, const float (&pi)[3], int n, int64_t& w) {
        for (int c0 = 0; c0 < n; c0 += 64) {
            const int t = c0 + lane;
            bool keep = false;
            float d[3] = {0.f, 0.f, 0.f};
            int j = 0;
            if (t < n) {
                const float4 cj = sCand[t];
                j = __float_as_int(cj.w);
                const float pj[3] = {cj.x, cj.y, cj.z};
                keep = (self_loops || j != i) && min_image(pi, pj, c, d) <= rc2;
            }
            const uint64_t m = __ballot(keep);
            if constexpr (WRITE) {
                const int64_t at = w + __popcll(m & ((1ull << lane) - 1ull));
                if (keep && (uint64_t)at < cap) {  // cap: the arrays' length (capacity mode)
                    if (esrc) esrc[at] = i;
                    edst[at] = j;
                    evec[at * 3 + 0] = d[0];
                    evec[at * 3 + 1] = d[1];
                    evec[at * 3 + 2] = d[2];
                }
            }
            w += __popcll(m);
        }
    };
    if (T <= kNlCap) {
        // one chunk: the waves share the staged candidates and take every kNlWaves-th
        // home atom, whose position is a staged candidate as well
        stage(0, T);
        __syncthreads();
        for (int hh = wv; hh < H; hh += kNlWaves) {
            const float4 ci = sCand[sPre[13] + hh];
            const int i = __builtin_amdgcn_readfirstlane(__float_as_int(ci.w));
            const float pi[3] = {ci.x, ci.y, ci.z};
            int64_t w = WRITE ? offsets[i] : 0;
            scan_cands(i, pi, T, w);
            if constexpr (!WRITE) {
                if (lane == 0) counts[i] = w;
            }
        }
        return;
    }
    // dense systems (more than kNlCap candidates): chunks staged by all waves, every
    // home atom walked by wave 0 (the other waves take part in staging and barriers)
    for (int hh = 0; hh < H; ++hh) {
        const int i = __builtin_amdgcn_readfirstlane(order[home0 + hh]);
        const float pi[3] = {pos[(int64_t)i * 3], pos[(int64_t)i * 3 + 1], pos[(int64_t)i * 3 + 2]};
        int64_t w = (WRITE && wv == 0) ? offsets[i] : 0;
        for (int base = 0; base < T; base += kNlCap) {
            const int n = min(kNlCap, T - base);
            __syncthreads();
            stage(base, n);
            __syncthreads();
            if (wv == 0) scan_cands(i, pi, n, w);
        }
        if constexpr (!WRITE) {
            if (wv == 0 && lane == 0) counts[i] = w;
        }
    }
}

// Sort each atom's neighbors by j: one wave per row, each entry written at its
// rank (the number of entries with a smaller j, ties by position in the row, so
// equal j from different periodic images keep the stencil order).  Rows of at
// most 64 * kRowRegs entries are held in registers (lane l owns entries l,
// l + 64, ...), all read before any is written.  Longer rows (denser than any
// system at an interatomic cutoff) are ranked against the row read again from
// memory, 64 entries at a time: GRAPH writes each entry at its rank in the
// output arrays; the in-place form keeps the ranks in esrc (the row's source
// column, which holds the row index and is restored afterwards), and one lane
// applies the permutation by following its cycles (one swap per entry); a caller
// that passes no source column gets an insertion sort by one lane instead.
// GRAPH: the sorted row goes to int64 arrays instead, edst / evec are left as
// they are: the message-passing layout (gsrc = j, gdst = i, gvec = the vector
// negated: edges grouped by destination i, each with vector r_i - r_j), or with
// ref the neighbor list's own (gsrc = i, gdst = j, gvec = the vector).
constexpr int kRowRegs = 8;
template <bool GRAPH>
__global__ __launch_bounds__(256) void nl_sort_rows_kernel(const int64_t* __restrict__ offsets,
                                                           int* __restrict__ esrc,
                                                           int* __restrict__ edst,
                                                           float* __restrict__ evec, int64_t n,
                                                           int64_t* __restrict__ gsrc,
                                                           int64_t* __restrict__ gdst,
                                                           float* __restrict__ gvec, int ref,
                                                           uint64_t cap) {
    const int lane = threadIdx.x & 63;
    const int64_t row = (int64_t)blockIdx.x * 4 + (threadIdx.x >> 6);
    if (row >= n) return;  // uniform per wave
    const int64_t s = offsets[row], e = offsets[row + 1];
    if ((uint64_t)e > cap) return;  // capacity mode: a row past the arrays (flagged later)
    const int len = (int)(e - s);
    auto put = [&](int64_t at, int j, float v0, float v1, float v2) {
        if constexpr (GRAPH) {
            if (ref) {  // uniform: the neighbor list itself with int64 indices
                gsrc[at] = row;
                gdst[at] = j;
                gvec[at * 3] = v0;
                gvec[at * 3 + 1] = v1;
                gvec[at * 3 + 2] = v2;
            } else {
                gsrc[at] = j;
                gdst[at] = row;
                gvec[at * 3] = -v0;
                gvec[at * 3 + 1] = -v1;
                gvec[at * 3 + 2] = -v2;
            }
        } else {
            edst[at] = j;
            evec[at * 3] = v0;
            evec[at * 3 + 1] = v1;
            evec[at * 3 + 2] = v2;
        }
    };
    if (len <= 64) {
        if (!GRAPH && len <= 1) return;
        int j = 0;
        float v0 = 0.f, v1 = 0.f, v2 = 0.f;
        if (lane < len) {
            j = edst[s + lane];
            v0 = evec[(s + lane) * 3];
            v1 = evec[(s + lane) * 3 + 1];
            v2 = evec[(s + lane) * 3 + 2];
        }
        int rank = 0;
        for (int m = 0; m < len; ++m) {
            const int jm = __builtin_amdgcn_readlane(j, m);
            rank += (jm < j || (jm == j && m < lane)) ? 1 : 0;
        }
        if (lane < len) put(s + rank, j, v0, v1, v2);
        return;
    }
    if (len <= 64 * kRowRegs) {
        const int nk = (len + 63) >> 6;
        int jk[kRowRegs], rk[kRowRegs];
        float xk[kRowRegs], yk[kRowRegs], zk[kRowRegs];
#pragma unroll
        for (int k = 0; k < kRowRegs; ++k) {
            const int a = k * 64 + lane;
            jk[k] = 0;
            rk[k] = 0;
            xk[k] = yk[k] = zk[k] = 0.f;
            if (a < len) {
                jk[k] = edst[s + a];
                xk[k] = evec[(s + a) * 3];
                yk[k] = evec[(s + a) * 3 + 1];
                zk[k] = evec[(s + a) * 3 + 2];
            }
        }
#pragma unroll
        for (int k2 = 0; k2 < kRowRegs; ++k2) {
            if (k2 < nk) {
                const int m_end = min(64, len - k2 * 64);
                for (int m = 0; m < m_end; ++m) {
                    const int jm = __builtin_amdgcn_readlane(jk[k2], m);
                    const int pm = k2 * 64 + m;
#pragma unroll
                    for (int k = 0; k < kRowRegs; ++k)
                        rk[k] += (jm < jk[k] || (jm == jk[k] && pm < k * 64 + lane)) ? 1 : 0;
                }
            }
        }
#pragma unroll
        for (int k = 0; k < kRowRegs; ++k)
            if (k * 64 + lane < len) put(s + rk[k], jk[k], xk[k], yk[k], zk[k]);
        return;
    }
    if constexpr (!GRAPH) {
        if (esrc == nullptr) {  // no source column to hold the ranks: insertion by one lane
            if (lane == 0)
                for (int64_t a = s + 1; a < e; ++a) {
                    const int v = edst[a];
                    const float v0 = evec[a * 3], v1 = evec[a * 3 + 1], v2 = evec[a * 3 + 2];
                    int64_t q = a - 1;
                    for (; q >= s && edst[q] > v; --q) {
                        edst[q + 1] = edst[q];
#pragma unroll
                        for (int d = 0; d < 3; ++d) evec[(q + 1) * 3 + d] = evec[q * 3 + d];
                    }
                    edst[q + 1] = v;
                    evec[(q + 1) * 3] = v0;
                    evec[(q + 1) * 3 + 1] = v1;
                    evec[(q + 1) * 3 + 2] = v2;
                }
            return;
        }
    }
    for (int base = 0; base < len; base += 64) {
        const int a = base + lane;
        const int ja = a < len ? edst[s + a] : 0;
        int r = 0;
        for (int c0 = 0; c0 < len; c0 += 64) {
            const int x = c0 + lane < len ? edst[s + c0 + lane] : 0;
            const int m_end = min(64, len - c0);
            for (int m = 0; m < m_end; ++m) {
                const int jm = __builtin_amdgcn_readlane(x, m);
                r += (jm < ja || (jm == ja && c0 + m < a)) ? 1 : 0;
            }
        }
        if (a < len) {
            if constexpr (GRAPH)
                put(s + r, ja, evec[(s + a) * 3], evec[(s + a) * 3 + 1], evec[(s + a) * 3 + 2]);
            else
                esrc[s + a] = r;
        }
    }
    if constexpr (!GRAPH) {
        __threadfence_block();  // the wave's rank stores are complete before lane 0 reads them
        if (lane == 0) {
            for (int a = 0; a < len; ++a) {
                int r = esrc[s + a];
                while (r != a) {  // the entry at a belongs at r: swap it there
                    const int64_t pa = s + a, pr = s + r;
                    const int tj = edst[pa];
                    edst[pa] = edst[pr];
                    edst[pr] = tj;
#pragma unroll
                    for (int d = 0; d < 3; ++d) {
                        const float tv = evec[pa * 3 + d];
                        evec[pa * 3 + d] = evec[pr * 3 + d];
                        evec[pr * 3 + d] = tv;
                    }
                    const int rr = esrc[pr];
                    esrc[pr] = r;
                    r = rr;
                }
            }
        }
        __threadfence_block();
        for (int a = lane; a < len; a += 64) esrc[s + a] = (int)row;
    }
}

// ---------------------------------------------------------------------------
// exclusive scan: out[0..n] (out[n] = total), one workgroup, no workspace.
// Tiles of kScanBlock * kScanPer elements: each thread sums its kScanPer
// consecutive elements in registers (all loads issued together), the thread
// sums are scanned within each wave by shuffles and across the waves through
// LDS (two barriers per tile), and each thread writes its run of prefixes.
// ---------------------------------------------------------------------------
constexpr int kScanBlock = 1024;
constexpr int kScanPer = 16;

template <typename TI>
__global__ __launch_bounds__(kScanBlock) void scan_exclusive_kernel(const TI* __restrict__ in,
                                                                    int64_t* __restrict__ out,
                                                                    int64_t n,
                                                                    int64_t* __restrict__ total_out) {
    constexpr int kWaves = kScanBlock / 64;
    __shared__ int64_t wsum[kWaves];
    const int t = threadIdx.x, lane = t & 63, w = t >> 6;
    int64_t carry = 0;  // total of the previous tiles (the same in every thread)
    for (int64_t base = 0; base < n; base += (int64_t)kScanBlock * kScanPer) {
        const int64_t i0 = base + (int64_t)t * kScanPer;
        int64_t v[kScanPer];
        if (i0 + kScanPer <= n) {
#pragma unroll
            for (int j = 0; j < kScanPer; ++j) v[j] = (int64_t)in[i0 + j];
        } else {
#pragma unroll
            for (int j = 0; j < kScanPer; ++j) v[j] = i0 + j < n ? (int64_t)in[i0 + j] : 0;
        }
        int64_t s = 0;
#pragma unroll
        for (int j = 0; j < kScanPer; ++j) s += v[j];
        // inclusive scan of the thread sums within the wave
        int64_t x = s;
#pragma unroll
        for (int off = 1; off < 64; off <<= 1) {
            const int64_t y = __shfl_up(x, off, 64);
            if (lane >= off) x += y;
        }
        if (lane == 63) wsum[w] = x;
        __syncthreads();
        int64_t before = 0, total = 0;  // sums of the waves before this one, of all waves
#pragma unroll
        for (int k = 0; k < kWaves; ++k) {
            const int64_t ws = wsum[k];
            before += k < w ? ws : 0;
            total += ws;
        }
        __syncthreads();  // wsum is rewritten by the next tile
        int64_t run = carry + before + x - s;
        if (i0 + kScanPer <= n) {
#pragma unroll
            for (int j = 0; j < kScanPer; ++j) {
                out[i0 + j] = run;
                run += v[j];
            }
        } else {
#pragma unroll
            for (int j = 0; j < kScanPer; ++j) {
                if (i0 + j < n) out[i0 + j] = run;
                run += v[j];
            }
        }
        carry += total;
    }
    if (t == 0) {
        out[n] = carry;
        if (total_out) *total_out = carry;  // the total once more (a copy the caller skips)
    }
}

static int scan_i64(const int64_t* in, int64_t* out, int64_t n, hipStream_t s,
                    int64_t* total_out = nullptr) {
    scan_exclusive_kernel<int64_t><<<1, kScanBlock, 0, s>>>(in, out, n, total_out);
    return (int)hipGetLastError();
}
static int scan_i32(const int* in, int64_t* out, int64_t n, hipStream_t s,
                    int64_t* total_out = nullptr) {
    scan_exclusive_kernel<int><<<1, kScanBlock, 0, s>>>(in, out, n, total_out);
    return (int)hipGetLastError();
}

// Workspace layout for a neighbor-list build of n atoms (all 256-B aligned):
//   bin_of int[n] | bin_count int[total] | bin_start i64[total+1] | order int[n]
//   | counts i64[n] | offsets i64[n+1]
struct NlLayout {
    size_t bin_of, bin_count, bin_start, order, counts, offsets, total_bytes;
};
static size_t align256(size_t x) { return (x + 255) & ~size_t(255); }
static NlLayout nl_layout(int64_t n, int total_bins) {
    NlLayout L;
    size_t o = 0;
    L.bin_of = o; o = align256(o + sizeof(int) * (size_t)n);
    L.bin_count = o; o = align256(o + sizeof(int) * (size_t)total_bins);
    L.bin_start = o; o = align256(o + sizeof(int64_t) * ((size_t)total_bins + 1));
    L.order = o; o = align256(o + sizeof(int) * (size_t)n);
    L.counts = o; o = align256(o + sizeof(int64_t) * (size_t)n);
    L.offsets = o; o = align256(o + sizeof(int64_t) * ((size_t)n + 1));
    L.total_bytes = o;
    return L;
}

}  // namespace bmhip

using namespace bmhip;

extern "C" int batteries_exclusive_scan_i64(const int64_t* in, int64_t* out, int64_t n,
                                            hipStream_t stream) {
    if (n < 0) return BM_ERR_ARG;
    return scan_i64(in, out, n, stream);
}

extern "C" size_t batteries_neighbor_list_workspace_bytes(int64_t N, const float* box,
                                                          float cutoff) {
    if (N < 0 || !box || !valid_box(box, cutoff)) return 0;
    const BinCfg c = make_bin_cfg(box, cutoff);
    return nl_layout(N, c.total).total_bytes;
}

extern "C" size_t batteries_neighbor_list_offsets_at(int64_t N, const float* box, float cutoff) {
    if (N < 0 || !box || !valid_box(box, cutoff)) return 0;
    const BinCfg c = make_bin_cfg(box, cutoff);
    return nl_layout(N, c.total).offsets;
}

extern "C" int batteries_neighbor_list_count(const float* positions, const float* box, int64_t N,
                                             float cutoff, int self_loops, void* workspace,
                                             size_t workspace_bytes, int64_t* d_num_edges,
                                             hipStream_t stream) {
    if (N < 0 || !box || !valid_box(box, cutoff)) return BM_ERR_ARG;
    const BinCfg c = make_bin_cfg(box, cutoff);
    const NlLayout L = nl_layout(N, c.total);
    if (!workspace || workspace_bytes < L.total_bytes) return BM_ERR_WORKSPACE;
    char* ws = static_cast<char*>(workspace);
    int* bin_of = reinterpret_cast<int*>(ws + L.bin_of);
    int* bin_count = reinterpret_cast<int*>(ws + L.bin_count);
    int64_t* bin_start = reinterpret_cast<int64_t*>(ws + L.bin_start);
    int* order = reinterpret_cast<int*>(ws + L.order);
    int64_t* counts = reinterpret_cast<int64_t*>(ws + L.counts);
    int64_t* offsets = reinterpret_cast<int64_t*>(ws + L.offsets);
    const int B = 256;
    int rc = BM_OK;
    if (N <= kBinSmallAtoms && c.total <= kBinSmallBins) {
        nl_bin_small_kernel<<<1, kBinSmallBlock, 0, stream>>>(positions, c, (int)N, bin_start,
                                                              order);
    } else {
        nl_zero_i32_kernel<<<(unsigned)ceil_div(c.total, B), B, 0, stream>>>(bin_count, c.total);
        if (N > 0)
            nl_assign_kernel<<<(unsigned)ceil_div(N, B), B, 0, stream>>>(positions, c, bin_of,
                                                                         bin_count, N);
        rc = scan_i32(bin_count, bin_start, c.total, stream);
        if (rc != BM_OK) return rc;
        nl_zero_i32_kernel<<<(unsigned)ceil_div(c.total, B), B, 0, stream>>>(bin_count, c.total);
        if (N > 0) {
            nl_place_kernel<<<(unsigned)ceil_div(N, B), B, 0, stream>>>(bin_of, bin_start,
                                                                        bin_count, order, N);
            nl_sort_bins_wave_kernel<<<(unsigned)c.total, 64, 0, stream>>>(bin_start, order,
                                                                           bin_of, c.total);
        }
    }
    if (N > 0) {
        nl_cell_kernel<false><<<(unsigned)c.total, 64 * kNlWaves, 0, stream>>>(
            positions, c, cutoff * cutoff, self_loops, bin_start, order, counts, nullptr, nullptr,
            nullptr, nullptr, ~0ull);
    }
    rc = scan_i64(counts, offsets, N, stream, d_num_edges);
    if (rc != BM_OK) return rc;
    return (int)hipGetLastError();
}

extern "C" int batteries_neighbor_list_write(const float* positions, const float* box, int64_t N,
                                             float cutoff, int self_loops, void* workspace,
                                             size_t workspace_bytes, int* edge_src, int* edge_dst,
                                             float* edge_vectors, int64_t* row_offsets,
                                             hipStream_t stream) {
    if (N < 0 || !box || !valid_box(box, cutoff)) return BM_ERR_ARG;
    const BinCfg c = make_bin_cfg(box, cutoff);
    const NlLayout L = nl_layout(N, c.total);
    if (!workspace || workspace_bytes < L.total_bytes) return BM_ERR_WORKSPACE;
    char* ws = static_cast<char*>(workspace);
    const int64_t* bin_start = reinterpret_cast<const int64_t*>(ws + L.bin_start);
    const int* order = reinterpret_cast<const int*>(ws + L.order);
    const int64_t* offsets = reinterpret_cast<const int64_t*>(ws + L.offsets);
    const int B = 256;
    if (N > 0) {
        nl_cell_kernel<true><<<(unsigned)c.total, 64 * kNlWaves, 0, stream>>>(
            positions, c, cutoff * cutoff, self_loops, bin_start, order, nullptr, offsets, edge_src,
            edge_dst, edge_vectors, ~0ull);
        nl_sort_rows_kernel<false><<<(unsigned)ceil_div(N, 4), 256, 0, stream>>>(
            offsets, edge_src, edge_dst, edge_vectors, N, nullptr, nullptr, nullptr, 0, ~0ull);
    }
    if (row_offsets) {
        hipError_t e = hipMemcpyAsync(row_offsets, offsets, sizeof(int64_t) * (size_t)(N + 1),
                                      hipMemcpyDeviceToDevice, stream);
        if (e != hipSuccess) return (int)e;
    }
    return (int)hipGetLastError();
}

// Spatial order from the neighbor list's cells: the cells in serpentine
// (boustrophedon) order, x fastest with the direction reversed on every other row,
// rows reversed on every other plane, so that consecutive cells are always
// adjacent; the atoms of a cell in ascending index (the binning's own order).
// One workgroup: each thread takes a run of consecutive path positions, their
// atom counts are scanned across the workgroup, then each thread writes its runs.
constexpr int kSerpBlock = 1024;

__global__ __launch_bounds__(kSerpBlock) void nl_serpentine_order_kernel(
    const int64_t* __restrict__ bin_start, const int* __restrict__ order, BinCfg c,
    int64_t* __restrict__ out, int64_t* __restrict__ offsets, int64_t n, uint64_t cap,
    int* __restrict__ overflow) {
    // capacity mode (after the passes that read the offsets): when the edges outgrew the
    // arrays, every row is emptied, so that no later kernel reads past them, and the flag
    // is raised; otherwise the flag is cleared
    if (overflow) {
        const bool over = (uint64_t)offsets[n] > cap;
        __syncthreads();  // every thread has read the total before any is cleared
        if (over)
            for (int64_t i = threadIdx.x; i <= n; i += kSerpBlock) offsets[i] = 0;
        if (threadIdx.x == 0) *overflow = over ? 1 : 0;
    }
    __shared__ int64_t sWave[kSerpBlock / 64];
    const int t = threadIdx.x, lane = t & 63, w = t >> 6;
    const int per = (c.total + kSerpBlock - 1) / kSerpBlock;
    const int p0 = min(t * per, c.total), p1 = min(p0 + per, c.total);
    int64_t sum = 0;
    for (int p = p0; p < p1; ++p) {
        const int k = serpentine_cell(p, c);
        sum += bin_start[k + 1] - bin_start[k];
    }
    // exclusive scan of the thread sums: within each wave by shuffles, then the waves
    int64_t incl = sum;
#pragma unroll
    for (int off = 1; off < 64; off <<= 1) {
        const int64_t v = __shfl_up(incl, off, 64);
        if (lane >= off) incl += v;
    }
    if (lane == 63) sWave[w] = incl;
    __syncthreads();
    int64_t base = 0;
    for (int i = 0; i < w; ++i) base += sWave[i];
    int64_t o = base + incl - sum;
    if (out)
        for (int p = p0; p < p1; ++p) {
            const int k = serpentine_cell(p, c);
            for (int64_t a = bin_start[k]; a < bin_start[k + 1]; ++a) out[o++] = order[a];
        }
}

// Phase 2 into int64 arrays: the message-passing layout (ref = 0) or the neighbor
// list's own orientation (ref = 1).
static int neighbor_write_i64(const float* positions, const float* box, int64_t N, float cutoff,
                              int self_loops, void* workspace, size_t workspace_bytes, int* tmp_j,
                              float* tmp_vec, int64_t* src, int64_t* dst, float* edge_vectors,
                              int64_t* row_offsets, int64_t* spatial_order, int ref,
                              int64_t capacity, int* overflow, hipStream_t stream) {
    if (N < 0 || !box || !valid_box(box, cutoff)) return BM_ERR_ARG;
    const uint64_t cap = capacity < 0 ? ~0ull : (uint64_t)capacity;
    const BinCfg c = make_bin_cfg(box, cutoff);
    const NlLayout L = nl_layout(N, c.total);
    if (!workspace || workspace_bytes < L.total_bytes) return BM_ERR_WORKSPACE;
    char* ws = static_cast<char*>(workspace);
    const int64_t* bin_start = reinterpret_cast<const int64_t*>(ws + L.bin_start);
    const int* order = reinterpret_cast<const int*>(ws + L.order);
    const int64_t* offsets = reinterpret_cast<const int64_t*>(ws + L.offsets);
    if (N > 0) {
        nl_cell_kernel<true><<<(unsigned)c.total, 64 * kNlWaves, 0, stream>>>(
            positions, c, cutoff * cutoff, self_loops, bin_start, order, nullptr, offsets, nullptr,
            tmp_j, tmp_vec, cap);
        nl_sort_rows_kernel<true><<<(unsigned)ceil_div(N, 4), 256, 0, stream>>>(
            offsets, nullptr, tmp_j, tmp_vec, N, src, dst, edge_vectors, ref, cap);
    }
    // the spatial order, and in capacity mode the overflow check (also for N = 0)
    if ((N > 0 && spatial_order) || overflow)
        nl_serpentine_order_kernel<<<1, kSerpBlock, 0, stream>>>(
            bin_start, order, c, spatial_order, const_cast<int64_t*>(offsets), N, cap, overflow);
    if (row_offsets) {
        hipError_t e = hipMemcpyAsync(row_offsets, offsets, sizeof(int64_t) * (size_t)(N + 1),
                                      hipMemcpyDeviceToDevice, stream);
        if (e != hipSuccess) return (int)e;
    }
    return (int)hipGetLastError();
}

extern "C" int batteries_neighbor_graph_write(const float* positions, const float* box, int64_t N,
                                              float cutoff, int self_loops, void* workspace,
                                              size_t workspace_bytes, int* tmp_j, float* tmp_vec,
                                              int64_t* src, int64_t* dst, float* edge_vectors,
                                              int64_t* row_offsets, int64_t* spatial_order,
                                              hipStream_t stream) {
    return neighbor_write_i64(positions, box, N, cutoff, self_loops, workspace, workspace_bytes,
                              tmp_j, tmp_vec, src, dst, edge_vectors, row_offsets, spatial_order,
                              0, -1, nullptr, stream);
}

extern "C" int batteries_neighbor_graph_write_capacity(
    const float* positions, const float* box, int64_t N, float cutoff, int self_loops,
    void* workspace, size_t workspace_bytes, int64_t capacity, int* tmp_j, float* tmp_vec,
    int64_t* src, int64_t* dst, float* edge_vectors, int64_t* row_offsets, int64_t* spatial_order,
    int* overflow, hipStream_t stream) {
    if (capacity < 0 || !overflow) return BM_ERR_ARG;
    return neighbor_write_i64(positions, box, N, cutoff, self_loops, workspace, workspace_bytes,
                              tmp_j, tmp_vec, src, dst, edge_vectors, row_offsets, spatial_order,
                              0, capacity, overflow, stream);
}

extern "C" int batteries_neighbor_list_write_i64(const float* positions, const float* box,
                                                 int64_t N, float cutoff, int self_loops,
                                                 void* workspace, size_t workspace_bytes,
                                                 int64_t num_edges, int* tmp_j, float* tmp_vec,
                                                 int64_t* edge_index, float* edge_vectors,
                                                 int64_t* row_offsets, hipStream_t stream) {
    if (num_edges < 0 || (num_edges > 0 && !edge_index)) return BM_ERR_ARG;
    return neighbor_write_i64(positions, box, N, cutoff, self_loops, workspace, workspace_bytes,
                              tmp_j, tmp_vec, edge_index, edge_index + num_edges, edge_vectors,
                              row_offsets, nullptr, 1, -1, nullptr, stream);
}

// ---------------------------------------------------------------------------
// Spatial (Morton) order of atoms: positions wrapped into the box, quantised to
// a grid of 2^b cells per axis, keyed by the 3b-bit Morton code of the cell;
// counting sort by key with ascending atom index inside a cell (deterministic).
// b is the largest value up to 5 with 8^b <= N (1 to 8 atoms per grid cell on
// average), so the scan over the cells stays about as long as the atom list.
// ---------------------------------------------------------------------------
constexpr int kMortonBits = 5;  // at most
constexpr int kMortonCells = 1 << (3 * kMortonBits);

static int morton_bits(int64_t N) {
    int b = 1;
    while (b < kMortonBits && ((int64_t)1 << (3 * (b + 1))) <= N) ++b;
    return b;
}

__device__ __forceinline__ int spread3(int v) {
    int r = 0;
#pragma unroll
    for (int b = 0; b < kMortonBits; ++b) r |= ((v >> b) & 1) << (3 * b);
    return r;
}

__global__ void morton_key_kernel(const float* __restrict__ pos, float bx, float by, float bz,
                                  int bits, int* __restrict__ key, int* __restrict__ count,
                                  int64_t n) {
    const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (i >= n) return;
    const float box[3] = {bx, by, bz};
    int q[3];
#pragma unroll
    for (int d = 0; d < 3; ++d) {
        const float p = pos[i * 3 + d];
        const float w = p - floorf(p / box[d]) * box[d];
        int v = (int)(w / box[d] * (float)(1 << bits));
        v = v < 0 ? 0 : (v > (1 << bits) - 1 ? (1 << bits) - 1 : v);
        q[d] = v;
    }
    const int k = spread3(q[0]) | (spread3(q[1]) << 1) | (spread3(q[2]) << 2);
    key[i] = k;
    atomicAdd(count + k, 1);
}

__global__ void morton_place_kernel(const int* __restrict__ key, const int64_t* __restrict__ start,
                                    int* __restrict__ cursor, int* __restrict__ tmp, int64_t n) {
    const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (i >= n) return;
    const int k = key[i];
    tmp[start[k] + atomicAdd(cursor + k, 1)] = (int)i;
}

__global__ void morton_finish_kernel(const int* __restrict__ tmp, int64_t* __restrict__ order,
                                     int64_t n) {
    const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (i < n) order[i] = tmp[i];
}

extern "C" size_t batteries_spatial_order_workspace_bytes(int64_t N) {
    if (N < 0) return 0;
    return align256(sizeof(int) * (size_t)N) * 2 + align256(sizeof(int) * kMortonCells) +
           align256(sizeof(int64_t) * (kMortonCells + 1));
}

extern "C" int batteries_spatial_order(const float* positions, const float* box, int64_t N,
                                       void* workspace, size_t workspace_bytes, int64_t* order,
                                       hipStream_t stream) {
    if (N < 0 || !box || !(box[0] > 0.f) || !(box[1] > 0.f) || !(box[2] > 0.f)) return BM_ERR_ARG;
    if (N == 0) return BM_OK;
    if (!workspace || workspace_bytes < batteries_spatial_order_workspace_bytes(N))
        return BM_ERR_WORKSPACE;
    char* ws = static_cast<char*>(workspace);
    int* key = reinterpret_cast<int*>(ws);
    int* tmp = reinterpret_cast<int*>(ws + align256(sizeof(int) * (size_t)N));
    int* count = reinterpret_cast<int*>(ws + 2 * align256(sizeof(int) * (size_t)N));
    int64_t* start = reinterpret_cast<int64_t*>(ws + 2 * align256(sizeof(int) * (size_t)N) +
                                                align256(sizeof(int) * kMortonCells));
    const int B = 256;
    const int bits = morton_bits(N);
    const int cells = 1 << (3 * bits);
    nl_zero_i32_kernel<<<(unsigned)ceil_div(cells, B), B, 0, stream>>>(count, cells);
    morton_key_kernel<<<(unsigned)ceil_div(N, B), B, 0, stream>>>(positions, box[0], box[1], box[2],
                                                                  bits, key, count, N);
    int rc = scan_i32(count, start, cells, stream);
    if (rc != BM_OK) return rc;
    nl_zero_i32_kernel<<<(unsigned)ceil_div(cells, B), B, 0, stream>>>(count, cells);
    morton_place_kernel<<<(unsigned)ceil_div(N, B), B, 0, stream>>>(key, start, count, tmp, N);
    nl_sort_bins_kernel<<<(unsigned)ceil_div(cells, B), B, 0, stream>>>(start, tmp, cells);
    morton_finish_kernel<<<(unsigned)ceil_div(N, B), B, 0, stream>>>(tmp, order, N);
    return (int)hipGetLastError();
}

// ---------------------------------------------------------------------------
// Reference-compatible C ABI (src/neighbor_list/neighbor_list.cu:456-478,
// include/neighbor_list.cuh:25-33): library-owned device buffers, freed by
// neighbor_list_free; cell [3,3] in device memory; one host sync for E.
// ---------------------------------------------------------------------------
// ---------------------------------------------------------------------------
// The neighbor list in three kernels and a scan for systems within the limits of
// nl_cells.h: binning, one workgroup per cell writing each atom's row already sorted
// by j into a slab, the exclusive scan of the counts, then the rows copied out.
// ---------------------------------------------------------------------------
extern "C" size_t batteries_neighbor_list_cells_workspace_bytes(int64_t N, const float* box,
                                                                float cutoff, int row_capacity) {
    if (N < 0 || !box || !valid_box(box, cutoff) || row_capacity < 0) return 0;
    const BinCfg c = make_bin_cfg(box, cutoff);
    if (!cells_supported(N, c)) return 0;
    return gb_layout(N, gb_row_cap(N, box, cutoff, row_capacity)).total;
}

extern "C" int batteries_neighbor_list_cells_count(const float* positions, const float* box,
                                                   int64_t N, float cutoff, int self_loops,
                                                   int row_capacity, void* workspace,
                                                   size_t workspace_bytes, int64_t* row_offsets,
                                                   int64_t* d_num_edges, hipStream_t stream) {
    if (N < 0 || !box || !valid_box(box, cutoff) || row_capacity < 0 || !row_offsets)
        return BM_ERR_ARG;
    const BinCfg c = make_bin_cfg(box, cutoff);
    if (!cells_supported(N, c)) return BM_ERR_ARG;
    const int rc = gb_row_cap(N, box, cutoff, row_capacity);
    const GbLayout L = gb_layout(N, rc);
    if (!workspace || workspace_bytes < L.total) return BM_ERR_WORKSPACE;
    char* ws = static_cast<char*>(workspace);
    int* pk = reinterpret_cast<int*>(ws + L.pk);
    int* cnt = reinterpret_cast<int*>(ws + L.cnt);
    float4* slab = reinterpret_cast<float4*>(ws + L.slab);
    const int n = (int)N;
    gb_bin_kernel<<<(unsigned)ceil_div(N, 256), 256, 0, stream>>>(positions, c, n, pk);
    gb_cell_kernel<<<(unsigned)c.total, kGbBlock, 0, stream>>>(positions, c, n, cutoff * cutoff,
                                                               self_loops, pk, rc, slab, cnt,
                                                               nullptr);
    const int r = scan_i32(cnt, row_offsets, N, stream, d_num_edges);
    if (r != BM_OK) return r;
    return (int)hipGetLastError();
}

template <typename TI>
static int cells_write(const float* positions, const float* box, int64_t N, float cutoff,
                       int self_loops, int row_capacity, void* workspace, size_t workspace_bytes,
                       const int64_t* row_offsets, TI* src, TI* dst, float* edge_vectors,
                       hipStream_t stream) {
    if (N < 0 || !box || !valid_box(box, cutoff) || row_capacity < 0 || !row_offsets)
        return BM_ERR_ARG;
    const BinCfg c = make_bin_cfg(box, cutoff);
    if (!cells_supported(N, c)) return BM_ERR_ARG;
    const int rc = gb_row_cap(N, box, cutoff, row_capacity);
    const GbLayout L = gb_layout(N, rc);
    if (!workspace || workspace_bytes < L.total) return BM_ERR_WORKSPACE;
    char* ws = static_cast<char*>(workspace);
    gb_rows_kernel<true, TI><<<(unsigned)ceil_div(N, 4), 256, 0, stream>>>(
        positions, c, (int)N, cutoff * cutoff, self_loops, reinterpret_cast<const int*>(ws + L.pk),
        rc, reinterpret_cast<const float4*>(ws + L.slab), reinterpret_cast<const int*>(ws + L.cnt),
        row_offsets, nullptr, nullptr, src, dst, edge_vectors, nullptr);
    return (int)hipGetLastError();
}

extern "C" int batteries_neighbor_list_cells_write_i64(
    const float* positions, const float* box, int64_t N, float cutoff, int self_loops,
    int row_capacity, void* workspace, size_t workspace_bytes, const int64_t* row_offsets,
    int64_t num_edges, int64_t* edge_index, float* edge_vectors, hipStream_t stream) {
    if (num_edges < 0 || (num_edges > 0 && (!edge_index || !edge_vectors))) return BM_ERR_ARG;
    if (num_edges == 0) return BM_OK;
    return cells_write<int64_t>(positions, box, N, cutoff, self_loops, row_capacity, workspace,
                                workspace_bytes, row_offsets, edge_index, edge_index + num_edges,
                                edge_vectors, stream);
}

extern "C" int neighbor_list_cuda(const float* positions, const float* cell, int64_t N,
                                  float cutoff, bool self_loops, NeighborListResult* result,
                                  hipStream_t stream) {
    if (!result) return BM_ERR_ARG;
    result->edge_index = nullptr;
    result->edge_vectors = nullptr;
    result->d_edge_index = nullptr;
    result->d_edge_vectors = nullptr;
    result->num_edges = 0;
    if (N == 0) return BM_OK;
    if (N < 0 || !positions || !cell) return BM_ERR_ARG;
    float h_cell[9];
    hipError_t e = hipMemcpy(h_cell, cell, sizeof(h_cell), hipMemcpyDeviceToHost);
    if (e != hipSuccess) return (int)e;
    const float box[3] = {h_cell[0], h_cell[4], h_cell[8]};
    if (!valid_box(box, cutoff)) return BM_ERR_ARG;
    // systems within the limits of nl_cells.h: three kernels, the scan, one host
    // synchronisation for E, the rows copied out
    const size_t cwsb = batteries_neighbor_list_cells_workspace_bytes(N, box, cutoff, 0);
    if (cwsb > 0) {
        void* cws = nullptr;
        int64_t* d_off = nullptr;
        e = hipMalloc(&cws, cwsb);
        if (e != hipSuccess) return (int)e;
        e = hipMalloc(&d_off, sizeof(int64_t) * (size_t)(N + 2));
        if (e != hipSuccess) {
            (void)hipFree(cws);
            return (int)e;
        }
        int rc = batteries_neighbor_list_cells_count(positions, box, N, cutoff, self_loops ? 1 : 0,
                                                     0, cws, cwsb, d_off, d_off + N + 1, stream);
        int64_t total = 0;
        if (rc == BM_OK) {
            e = hipMemcpyAsync(&total, d_off + N + 1, sizeof(int64_t), hipMemcpyDeviceToHost,
                               stream);
            if (e == hipSuccess) e = hipStreamSynchronize(stream);
            rc = (int)e;
        }
        if (rc == BM_OK && total > 0) {
            int* d_ei = nullptr;
            float* d_vec = nullptr;
            e = hipMalloc(&d_ei, sizeof(int) * 2 * (size_t)total);
            if (e == hipSuccess) e = hipMalloc(&d_vec, sizeof(float) * 3 * (size_t)total);
            if (e != hipSuccess) {
                if (d_ei) (void)hipFree(d_ei);
                rc = (int)e;
            } else {
                rc = cells_write<int>(positions, box, N, cutoff, self_loops ? 1 : 0, 0, cws, cwsb,
                                      d_off, d_ei, d_ei + total, d_vec, stream);
                if (rc == BM_OK) rc = (int)hipStreamSynchronize(stream);
                if (rc == BM_OK) {
                    result->d_edge_index = d_ei;
                    result->d_edge_vectors = d_vec;
                    result->edge_index = d_ei;
                    result->edge_vectors = d_vec;
                    result->num_edges = total;
                } else {
                    (void)hipFree(d_ei);
                    (void)hipFree(d_vec);
                }
            }
        }
        (void)hipFree(cws);
        (void)hipFree(d_off);
        return rc;
    }
    const size_t wsb = batteries_neighbor_list_workspace_bytes(N, box, cutoff);
    void* ws = nullptr;
    int64_t* d_total = nullptr;
    e = hipMalloc(&ws, wsb);
    if (e != hipSuccess) return (int)e;
    e = hipMalloc(&d_total, sizeof(int64_t));
    if (e != hipSuccess) {
        (void)hipFree(ws);
        return (int)e;
    }
    int rc = batteries_neighbor_list_count(positions, box, N, cutoff, self_loops ? 1 : 0, ws, wsb,
                                           d_total, stream);
    int64_t total = 0;
    if (rc == BM_OK) {
        e = hipMemcpyAsync(&total, d_total, sizeof(int64_t), hipMemcpyDeviceToHost, stream);
        if (e == hipSuccess) e = hipStreamSynchronize(stream);
        rc = (int)e;
    }
    if (rc == BM_OK && total > 0) {
        int* d_ei = nullptr;
        float* d_vec = nullptr;
        e = hipMalloc(&d_ei, sizeof(int) * 2 * (size_t)total);
        if (e == hipSuccess) e = hipMalloc(&d_vec, sizeof(float) * 3 * (size_t)total);
        if (e != hipSuccess) {
            if (d_ei) (void)hipFree(d_ei);
            rc = (int)e;
        } else {
            rc = batteries_neighbor_list_write(positions, box, N, cutoff, self_loops ? 1 : 0, ws, wsb,
                                               d_ei, d_ei + total, d_vec, nullptr, stream);
            if (rc == BM_OK) rc = (int)hipStreamSynchronize(stream);
            if (rc == BM_OK) {
                result->d_edge_index = d_ei;
                result->d_edge_vectors = d_vec;
                result->edge_index = d_ei;
                result->edge_vectors = d_vec;
                result->num_edges = total;
            } else {
                (void)hipFree(d_ei);
                (void)hipFree(d_vec);
            }
        }
    }
    (void)hipFree(ws);
    (void)hipFree(d_total);
    return rc;
}

extern "C" void neighbor_list_free(NeighborListResult* result) {
    if (!result) return;
    if (result->d_edge_index) (void)hipFree(result->d_edge_index);
    if (result->d_edge_vectors) (void)hipFree(result->d_edge_vectors);
    result->d_edge_index = nullptr;
    result->d_edge_vectors = nullptr;
    result->edge_index = nullptr;
    result->edge_vectors = nullptr;
    result->num_edges = 0;
}

extern "C" size_t neighbor_list_estimate_memory(int64_t N, float density, float cutoff) {
    // same estimate as reference neighbor_list.cu:442-451
    const float vol = (4.0f / 3.0f) * 3.14159f * cutoff * cutoff * cutoff;
    const int avg = (int)(density * vol) + 1;
    const size_t edge_memory = (size_t)N * avg * (2 * sizeof(int) + 3 * sizeof(float));
    const size_t temp_memory = (size_t)N * sizeof(int) * 4;
    return edge_memory + temp_memory;
}
