/*
 * Neighbor-list oracle (TEST INFRASTRUCTURE ONLY), plain C, fp32.
 *
 * nl_cell_list restates the reference cell-list algorithm
 *   src/neighbor_list/neighbor_list.cu
 *     :261-284  box from the cell diagonal, 1/L, bins = max(3, int(L / r_c)),
 *               bin size L / bins, cutoff^2
 *     :30-36    periodic bin index
 *     :41-52    wrap into [0, L) with floorf(p * (1/L)) * L, bin = min(int(p / b), bins-1)
 *     :57-62    minimum image d -= rintf(d * (1/L)) * L
 *     :112-171  27-cell stencil, j != i unless self loops, keep d.d <= r_c^2
 *     :176-240  emit (src = i, dst = j, vec = d) grouped by i
 * with one fixed op order and no FMA contraction (build with -ffp-contract=off).
 * Inside a cell the reference places atoms in atomic order; this restatement
 * uses ascending atom index.  Edge order does not matter to the callers of this
 * file: the tests compare edge sets sorted by (i, j).
 *
 * nl_brute_force restates the brute force of reference
 * tests/test_neighbor_list.cu:30-68 with the kernel's minimum-image arithmetic
 * (multiply by 1/L rather than divide by L), over all pairs.
 */
#include <math.h>
#include <stdint.h>
#include <stdlib.h>
#include <string.h>

typedef struct {
    int nb[3];
    float bin[3];
    float box[3];
    float inv[3];
    int total;
} Cfg;

static void make_cfg(const float* cell, float cutoff, Cfg* c) {
    c->box[0] = cell[0];
    c->box[1] = cell[4];
    c->box[2] = cell[8];
    for (int d = 0; d < 3; ++d) {
        c->inv[d] = 1.0f / c->box[d];
        int n = (int)(c->box[d] / cutoff);
        c->nb[d] = n > 3 ? n : 3;
        c->bin[d] = c->box[d] / (float)c->nb[d];
    }
    c->total = c->nb[0] * c->nb[1] * c->nb[2];
}

static int wrap(int b, int n) { return (b + n) % n; }

static void bin_coords(const float* p, const Cfg* c, int* out) {
    for (int d = 0; d < 3; ++d) {
        float t = p[d] * c->inv[d];
        float w = p[d] - floorf(t) * c->box[d];
        int b = (int)(w / c->bin[d]);
        int hi = b < c->nb[d] - 1 ? b : c->nb[d] - 1;
        out[d] = hi > 0 ? hi : 0;  /* lower clamp: the kernel's guard for non-finite input */
    }
}

static float min_image_dist2(const float* pi, const float* pj, const Cfg* c, float* d) {
    for (int k = 0; k < 3; ++k) {
        float t = pj[k] - pi[k];
        float s = t * c->inv[k];
        float r = rintf(s);
        float m = r * c->box[k];
        d[k] = t - m;
    }
    float xx = d[0] * d[0];
    float yy = d[1] * d[1];
    float zz = d[2] * d[2];
    float s = xx + yy;
    return s + zz;
}

/* Returns the number of edges found; writes at most max_edges of them. */
int64_t nl_cell_list(const float* pos, const float* cell, int64_t n, float cutoff,
                     int self_loops, int64_t max_edges,
                     int32_t* src, int32_t* dst, float* vec) {
    Cfg c;
    make_cfg(cell, cutoff, &c);
    const float rc2 = cutoff * cutoff;
    int* bin_of = (int*)malloc(sizeof(int) * (size_t)(n > 0 ? n : 1));
    int* start = (int*)calloc((size_t)c.total + 1, sizeof(int));
    int* order = (int*)malloc(sizeof(int) * (size_t)(n > 0 ? n : 1));
    int* fill = (int*)calloc((size_t)c.total, sizeof(int));
    for (int64_t i = 0; i < n; ++i) {
        int b[3];
        bin_coords(pos + 3 * i, &c, b);
        bin_of[i] = b[0] + b[1] * c.nb[0] + b[2] * c.nb[0] * c.nb[1];
        start[bin_of[i] + 1]++;
    }
    for (int k = 0; k < c.total; ++k) start[k + 1] += start[k];
    for (int64_t i = 0; i < n; ++i) order[start[bin_of[i]] + fill[bin_of[i]]++] = (int)i;
    int64_t e = 0;
    for (int64_t i = 0; i < n; ++i) {
        int bi[3];
        bin_coords(pos + 3 * i, &c, bi);
        for (int dz = -1; dz <= 1; ++dz)
            for (int dy = -1; dy <= 1; ++dy)
                for (int dx = -1; dx <= 1; ++dx) {
                    int nb = wrap(bi[0] + dx, c.nb[0]) + wrap(bi[1] + dy, c.nb[1]) * c.nb[0]
                             + wrap(bi[2] + dz, c.nb[2]) * c.nb[0] * c.nb[1];
                    for (int k = start[nb]; k < start[nb + 1]; ++k) {
                        int j = order[k];
                        if (!self_loops && j == i) continue;
                        float d[3];
                        if (min_image_dist2(pos + 3 * i, pos + 3 * (int64_t)j, &c, d) <= rc2) {
                            if (e < max_edges) {
                                src[e] = (int32_t)i;
                                dst[e] = j;
                                memcpy(vec + 3 * e, d, sizeof(d));
                            }
                            ++e;
                        }
                    }
                }
    }
    free(bin_of);
    free(start);
    free(order);
    free(fill);
    return e;
}

int64_t nl_brute_force(const float* pos, const float* cell, int64_t n, float cutoff,
                       int self_loops, int64_t max_edges,
                       int32_t* src, int32_t* dst, float* vec) {
    Cfg c;
    make_cfg(cell, cutoff, &c);
    const float rc2 = cutoff * cutoff;
    int64_t e = 0;
    for (int64_t i = 0; i < n; ++i)
        for (int64_t j = 0; j < n; ++j) {
            if (!self_loops && i == j) continue;
            float d[3];
            if (min_image_dist2(pos + 3 * i, pos + 3 * j, &c, d) <= rc2) {
                if (e < max_edges) {
                    src[e] = (int32_t)i;
                    dst[e] = (int32_t)j;
                    memcpy(vec + 3 * e, d, sizeof(d));
                }
                ++e;
            }
        }
    return e;
}
