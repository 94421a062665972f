// Cell-list geometry shared by the neighbor-list and graph-build kernels: the bin
// layout, the binning of a position, the minimum-image vector, and the serpentine
// path through the cells.
//
// Same geometry as the reference (src/neighbor_list/neighbor_list.cu:18-90): box =
// cell diagonal, bins per axis = max(3, int(L / r_c)), bin = min(int(wrap(p) / b),
// bins - 1) with wrap(p) = p - floorf(p * (1/L)) * L, minimum image
// d -= rintf(d * (1/L)) * L.  The distance arithmetic is evaluated without FMA
// contraction in one fixed order, so the kept pairs are a function of the fp32
// inputs alone.
#pragma once

#include "common.h"

namespace bmhip {

struct BinCfg {
    int nb[3];
    float bin[3];
    float box[3];
    float inv[3];
    int total;
};

static inline BinCfg make_bin_cfg(const float box[3], float cutoff) {
    BinCfg c;
    for (int d = 0; d < 3; ++d) {
        c.box[d] = box[d];
        c.inv[d] = 1.0f / box[d];
        const int n = (int)(box[d] / cutoff);
        c.nb[d] = n > 3 ? n : 3;
        c.bin[d] = box[d] / (float)c.nb[d];
    }
    c.total = c.nb[0] * c.nb[1] * c.nb[2];
    return c;
}

// A box the cell list accepts: positive cutoff and sides, fewer than 2^30 cells.
static inline bool valid_box(const float box[3], float cutoff) {
    if (!(cutoff > 0.0f)) return false;
    for (int d = 0; d < 3; ++d)
        if (!(box[d] > 0.0f)) return false;
    const BinCfg c = make_bin_cfg(box, cutoff);
    return (int64_t)c.nb[0] * c.nb[1] * c.nb[2] < (int64_t)1 << 30;
}

#pragma clang fp contract(off)

__device__ __forceinline__ void bin_coords(float px, float py, float pz, const BinCfg& c,
                                           int* b) {
    const float p[3] = {px, py, pz};
#pragma unroll
    for (int d = 0; d < 3; ++d) {
        const float t = p[d] * c.inv[d];
        const float fl = floorf(t) * c.box[d];
        const float wpos = p[d] - fl;
        const int v = (int)(wpos / c.bin[d]);
        // upper clamp as the reference (neighbor_list.cu:48-50); the lower clamp only
        // guards non-finite input (a finite wrapped position never gives v < 0)
        const int hi = v < c.nb[d] - 1 ? v : c.nb[d] - 1;
        b[d] = hi > 0 ? hi : 0;
    }
}

__device__ __forceinline__ float min_image(const float* pi, const float* pj, const BinCfg& c,
                                           float* d) {
#pragma unroll
    for (int k = 0; k < 3; ++k) {
        const float t = pj[k] - pi[k];
        const float s = t * c.inv[k];
        const float r = rintf(s);
        const float m = r * c.box[k];
        d[k] = t - m;
    }
    const float xx = d[0] * d[0];
    const float yy = d[1] * d[1];
    const float zz = d[2] * d[2];
    const float s = xx + yy;
    return s + zz;
}

#pragma clang fp contract(on)

__host__ __device__ __forceinline__ int wrap_bin(int b, int n) { return (b + n) % n; }

// The serpentine (boustrophedon) path through the cells: x fastest with the
// direction reversed on every other row, rows reversed on every other plane, so
// that consecutive cells are always adjacent.  serpentine_cell(p) is the cell at
// path position p, serpentine_pos its inverse.
__host__ __device__ __forceinline__ int serpentine_cell(int p, const BinCfg& c) {
    const int nx = c.nb[0], ny = c.nb[1];
    const int row = p / nx, px = p - row * nx;
    const int bz = row / ny, py = row - bz * ny;
    const int by = (bz & 1) ? ny - 1 - py : py;
    const int bx = (row & 1) ? nx - 1 - px : px;
    return bx + by * nx + bz * nx * ny;
}

__host__ __device__ __forceinline__ int serpentine_pos(int bx, int by, int bz, const BinCfg& c) {
    const int nx = c.nb[0], ny = c.nb[1];
    const int row = bz * ny + ((bz & 1) ? ny - 1 - by : by);
    return row * nx + ((row & 1) ? nx - 1 - bx : bx);
}

}  // namespace bmhip
