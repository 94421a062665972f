// Shared device helpers for the batmobile MI355X (gfx950) kernels.
//
// All Clebsch-Gordan and spherical-harmonic constants come from
// generated_tables.h and are folded into straight-line code at compile time
// (static_for over constexpr tables), so no kernel reads a coefficient from
// memory.
#pragma once

#include <hip/hip_runtime.h>

#include <algorithm>
#include <cstdint>
#include <utility>

#include "generated_tables.h"

namespace bmhip {

typedef float v4f __attribute__((ext_vector_type(4)));

// ---------------------------------------------------------------------------
// compile-time loop: f(std::integral_constant<int, i>) for i in [0, N)
// ---------------------------------------------------------------------------
template <typename F, int... I>
__device__ __forceinline__ void static_for_impl(F&& f, std::integer_sequence<int, I...>) {
    (f(std::integral_constant<int, I>{}), ...);
}
template <int N, typename F>
__device__ __forceinline__ void static_for(F&& f) {
    static_for_impl(f, std::make_integer_sequence<int, N>{});
}

__host__ __device__ constexpr int sh_dim(int l) { return (l + 1) * (l + 1); }

// ---------------------------------------------------------------------------
// v_mfma_f32_16x16x4f32: D (16x16) += A (16x4) * B (4x16), fp32 in and out.
// Lane l supplies A[l % 16][l / 16] and B[l / 16][l % 16] and holds
// D[4 (l / 16) + r][l % 16] in element r of the accumulator.
// mfma4 runs four of them, k-step s taking component s of both float4s.
// ---------------------------------------------------------------------------
__device__ __forceinline__ v4f mfma1(float a, float b, v4f acc) {
    return __builtin_amdgcn_mfma_f32_16x16x4f32(a, b, acc, 0, 0, 0);
}

// ---------------------------------------------------------------------------
// v_mfma_f32_4x4x1_16b_f32 with the A operand of one block broadcast to all 16
// blocks (CBSZ = 4, ABID = the source block): block b (lanes 4b .. 4b + 3)
// accumulates the 4x4 outer product D_b[i][j] += A[i] B_b[j], with A[i] read from
// lane 4 ABID + i and B_b[j] from lane 4b + j; lane 4b + j holds D_b[r][j] in
// element r of the accumulator.
// ---------------------------------------------------------------------------
template <int ABID>
__device__ __forceinline__ v4f mfma_4x4_bcast(float a, float b, v4f acc) {
    return __builtin_amdgcn_mfma_f32_4x4x1f32(a, b, acc, 4, ABID, 0);
}

// Raw buffer loads: 32-bit lane offset (VGPR) + uniform offset (SGPR) from a
// base address, reads past num_records bytes return 0.
constexpr int kBufferDword3 = 0x00020000;  // gfx9-family raw buffer descriptor word 3

__device__ __forceinline__ __amdgpu_buffer_rsrc_t buffer_rsrc(const float* p, uint32_t bytes) {
    return __builtin_amdgcn_make_buffer_rsrc(const_cast<float*>(p), (short)0, (int)bytes,
                                             kBufferDword3);
}
__device__ __forceinline__ float buffer_ld(__amdgpu_buffer_rsrc_t r, int voff, int soff) {
    return __int_as_float(__builtin_amdgcn_raw_buffer_load_b32(r, voff, soff, 0));
}
// 16 bytes at a 4-byte aligned offset (one buffer_load_dwordx4)
__device__ __forceinline__ float4 buffer_ld4(__amdgpu_buffer_rsrc_t r, int voff, int soff) {
    const auto v = __builtin_amdgcn_raw_buffer_load_b128(r, voff, soff, 0);
    return make_float4(__int_as_float(v[0]), __int_as_float(v[1]), __int_as_float(v[2]),
                       __int_as_float(v[3]));
}

// Index-mode buffer load (buffer_load_dwordx4 ... idxen offen): 16 bytes at
// base + vindex * stride + voffset + soffset, the stride taken from the
// descriptor (at most 16383 bytes on gfx9).  vindex and voffset are VGPRs, so a
// row index that is uniform across the wave needs no scalar register.
typedef int v4i_t __attribute__((ext_vector_type(4)));
__device__ v4i_t struct_buffer_load_b128(__amdgpu_buffer_rsrc_t rsrc, int vindex, int voffset,
                                         int soffset, int aux)
    __asm("llvm.amdgcn.struct.ptr.buffer.load.v4i32");
constexpr int kMaxBufferStride = 16383;

// Store of a lane's 16 bytes of an MFMA accumulator at base + lane_off (base
// uniform, in scalar registers), issued from the accumulator registers as
// inline assembly.  The compiler does not count the store in the vector-memory
// counter: on gfx9 that counter is shared by loads and stores, and a store it
// knew of would make it wait for every load in flight at the next use of one.
// Loads complete in order, so a store it does not know of can only lengthen a
// wait for a load, never end one early.  The nops cover the SGPR-write ->
// VMEM-read and the store-data -> VALU-write hazards, which the compiler does
// not check inside inline assembly.  Nothing in the same kernel may read what
// this writes.
__device__ __forceinline__ void store_row_acc(char* base, int lane_off, v4f acc) {
    asm volatile("s_nop 4\n\tglobal_store_dwordx4 %0, %1, %2\n\ts_nop 1" ::"v"(lane_off), "a"(acc),
                 "s"(base));
}

__device__ __forceinline__ v4f mfma4(const float4 a, const float4 b, v4f acc) {
    acc = mfma1(a.x, b.x, acc);
    acc = mfma1(a.y, b.y, acc);
    acc = mfma1(a.z, b.z, acc);
    acc = mfma1(a.w, b.w, acc);
    return acc;
}

// ---------------------------------------------------------------------------
// Real spherical harmonics (e3nn component normalisation, y polar axis) of a
// (not necessarily unit) vector, as the recurrence
//   Y_{l+1}[M] = sum c * Y_l[m] * r_j .
// Same polynomials as reference spherical_harmonics.cu:56-256.
// ---------------------------------------------------------------------------
template <int L>
__device__ __forceinline__ void sh_forward(float x, float y, float z, float* Y) {
    Y[0] = 1.0f;
    const float r[3] = {x, y, z};
    static_for<kSHTermStart[L]>([&](auto tt) {
        constexpr int t = decltype(tt)::value;
        constexpr SHTerm T = kSHTerms[t];
        constexpr int l = [] {
            int ll = 0;
            while (kSHTermStart[ll + 1] <= t) ++ll;
            return ll;
        }();
        constexpr bool first = (t == kSHTermStart[l]) || (kSHTerms[t > 0 ? t - 1 : 0].M != T.M);
        constexpr int out = sh_dim(l) + T.M;
        constexpr int in = l * l + T.m;
        if constexpr (first) {
            Y[out] = (T.c * Y[in]) * r[T.j];
        } else {
            Y[out] = fmaf(T.c * Y[in], r[T.j], Y[out]);
        }
    });
}

// Coefficient of x^a y^b z^c in component k of the expanded recurrence (0 if absent).
constexpr float sh_mono(int k, int a, int b, int c) {
    for (int i = 0; i < kSHMonoCount; ++i)
        if (kSHMono[i].k == k && kSHMono[i].a == a && kSHMono[i].b == b && kSHMono[i].c == c)
            return kSHMono[i].v;
    return 0.0f;
}
constexpr int sh_mono_terms(int k) {
    int n = 0;
    for (int i = 0; i < kSHMonoCount; ++i) n += kSHMono[i].k == k ? 1 : 0;
    return n;
}

// The same Y (L = 3) as sh_forward<3>, as closed-form polynomials over shared
// subexpressions (x^2, y^2, z^2, s = x^2 + z^2, d = z^2 - x^2): 33 operations
// against about 70 for the recurrence.  The coefficients are those of the
// expanded recurrence; the static_asserts check every term the factored form
// relies on (and that there are no others).
__device__ __forceinline__ void sh_forward_l3(float x, float y, float z, float* Y) {
    constexpr float c1 = sh_mono(1, 1, 0, 0);
    static_assert(c1 == sh_mono(2, 0, 1, 0) && c1 == sh_mono(3, 0, 0, 1), "l=1");
    constexpr float c4 = sh_mono(4, 1, 0, 1), c7 = sh_mono(7, 0, 1, 1);
    static_assert(c4 == sh_mono(5, 1, 1, 0), "xz and xy share a coefficient");
    constexpr float c6y = sh_mono(6, 0, 2, 0), c6s = sh_mono(6, 2, 0, 0);
    static_assert(c6s == sh_mono(6, 0, 0, 2), "Y6 = c6y y^2 + c6s (x^2 + z^2)");
    constexpr float c8 = sh_mono(8, 0, 0, 2);
    static_assert(-c8 == sh_mono(8, 2, 0, 0), "Y8 = c8 (z^2 - x^2)");
    constexpr float c9z = sh_mono(9, 1, 0, 2), c9x = sh_mono(9, 3, 0, 0);
    constexpr float c10 = sh_mono(10, 1, 1, 1);
    constexpr float c11y = sh_mono(11, 1, 2, 0), c11s = sh_mono(11, 3, 0, 0);
    static_assert(c11s == sh_mono(11, 1, 0, 2), "Y11 = x (c11y y^2 + c11s s)");
    static_assert(c11y == sh_mono(13, 0, 2, 1) && c11s == sh_mono(13, 0, 0, 3) &&
                      c11s == sh_mono(13, 2, 0, 1), "Y13 = z (c11y y^2 + c11s s)");
    constexpr float c12y = sh_mono(12, 0, 3, 0), c12s = sh_mono(12, 2, 1, 0);
    static_assert(c12s == sh_mono(12, 0, 1, 2), "Y12 = y (c12y y^2 + c12s s)");
    constexpr float c14 = sh_mono(14, 0, 1, 2);
    static_assert(-c14 == sh_mono(14, 2, 1, 0), "Y14 = c14 y (z^2 - x^2)");
    constexpr float c15z = sh_mono(15, 0, 0, 3), c15x = sh_mono(15, 2, 0, 1);
    static_assert(sh_mono(0, 0, 0, 0) == 1.0f && sh_mono_terms(0) == 1, "Y0");
    static_assert(sh_mono_terms(1) == 1 && sh_mono_terms(2) == 1 && sh_mono_terms(3) == 1 &&
                      sh_mono_terms(4) == 1 && sh_mono_terms(5) == 1 && sh_mono_terms(6) == 3 &&
                      sh_mono_terms(7) == 1 && sh_mono_terms(8) == 2 && sh_mono_terms(9) == 2 &&
                      sh_mono_terms(10) == 1 && sh_mono_terms(11) == 3 && sh_mono_terms(12) == 3 &&
                      sh_mono_terms(13) == 3 && sh_mono_terms(14) == 2 && sh_mono_terms(15) == 2,
                  "no other terms");
    const float xx = x * x, yy = y * y, zz = z * z;
    const float s = xx + zz, d = zz - xx;
    Y[0] = 1.0f;
    Y[1] = c1 * x;
    Y[2] = c1 * y;
    Y[3] = c1 * z;
    const float cx = c4 * x;
    Y[4] = cx * z;
    Y[5] = cx * y;
    Y[6] = fmaf(yy, c6y, c6s * s);
    Y[7] = (c7 * y) * z;
    Y[8] = c8 * d;
    Y[9] = x * fmaf(zz, c9z, c9x * xx);
    Y[10] = (Y[5] * z) * (c10 / c4);
    const float t = fmaf(yy, c11y, c11s * s);
    Y[11] = x * t;
    Y[12] = y * fmaf(yy, c12y, c12s * s);
    Y[13] = z * t;
    Y[14] = (c14 * y) * d;
    Y[15] = z * fmaf(zz, c15z, c15x * xx);
}

// Reverse-mode gradient of sh_forward: g (dL/dY, clobbered) -> dL/d(x,y,z).
template <int L>
__device__ __forceinline__ void sh_backward(float x, float y, float z, const float* Y, float* g,
                                            float& gx, float& gy, float& gz) {
    const float r[3] = {x, y, z};
    float gr[3] = {0.0f, 0.0f, 0.0f};
    constexpr int NT = kSHTermStart[L];
    static_for<NT>([&](auto tt) {
        constexpr int t = NT - 1 - decltype(tt)::value;  // reverse order
        constexpr SHTerm T = kSHTerms[t];
        constexpr int l = [] {
            int ll = 0;
            while (kSHTermStart[ll + 1] <= t) ++ll;
            return ll;
        }();
        constexpr int out = sh_dim(l) + T.M;
        constexpr int in = l * l + T.m;
        const float go = g[out] * T.c;
        gr[T.j] = fmaf(go, Y[in], gr[T.j]);
        if constexpr (in != 0) g[in] = fmaf(go, r[T.j], g[in]);
    });
    gx = gr[0];
    gy = gr[1];
    gz = gr[2];
}

// u = v / max(|v|, 1e-10): SphericalHarmonicsFunction's normalisation
// (reference python/batmobile/autograd.py:46-52).
__device__ __forceinline__ float normalize3(float& x, float& y, float& z) {
    const float r = fmaxf(sqrtf(x * x + y * y + z * z), 1e-10f);
    const float inv = 1.0f / r;
    x *= inv;
    y *= inv;
    z *= inv;
    return r;
}

// ---------------------------------------------------------------------------
// Simple tensor product pieces (34 paths, 611 entries, L<=3).
// ---------------------------------------------------------------------------

// out[o] = sum c * x[a] * y[b]
__device__ __forceinline__ void tp_simple(const float* x, const float* y, float* out) {
#pragma unroll
    for (int o = 0; o < 16; ++o) out[o] = 0.0f;
    static_for<kNumEntries>([&](auto kk) {
        constexpr CGEntry e = kCG[decltype(kk)::value];
        out[e.o] = fmaf(e.c * y[e.b], x[e.a], out[e.o]);
    });
}

// gx[a] = sum c * g[o] * y[b];  gy[b] = sum c * g[o] * x[a]
__device__ __forceinline__ void tp_simple_backward(const float* x, const float* y, const float* g,
                                                   float* gx, float* gy) {
#pragma unroll
    for (int i = 0; i < 16; ++i) {
        gx[i] = 0.0f;
        gy[i] = 0.0f;
    }
    static_for<kNumEntries>([&](auto kk) {
        constexpr CGEntry e = kCG[decltype(kk)::value];
        const float cg = e.c * g[e.o];
        gx[e.a] = fmaf(cg, y[e.b], gx[e.a]);
        gy[e.b] = fmaf(cg, x[e.a], gy[e.b]);
    });
}

// Edge operator M(y)[o][a] = sum_b c * y[b], so that tp_simple(x, y) = M x.
// Row o only (compile-time), written to m[0..15].
template <int O>
__device__ __forceinline__ void edge_operator_row(const float* y, float* m) {
#pragma unroll
    for (int a = 0; a < 16; ++a) m[a] = 0.0f;
    static_for<kNumEntries>([&](auto kk) {
        constexpr CGEntry e = kCG[decltype(kk)::value];
        if constexpr (e.o == O) m[e.a] = fmaf(e.c, y[e.b], m[e.a]);
    });
}

// Per-path products: t[q] = sum_{(a,b) in slot q} c * x[a] * cy  with y given.
// cyq is not precomputed here; used by the weighted kernels.
__device__ __forceinline__ void tp_per_path(const float* x, const float* y, float* t) {
#pragma unroll
    for (int q = 0; q < kNumSlots; ++q) t[q] = 0.0f;
    static_for<kNumEntries>([&](auto kk) {
        constexpr CGEntry e = kCG[decltype(kk)::value];
        t[e.q] = fmaf(e.c * y[e.b], x[e.a], t[e.q]);
    });
}

// Adjoint of tp_per_path: given h[q] = dL/dt[q],
//   gx[a] += sum c * h[q] * y[b];  gy[b] += sum c * h[q] * x[a]
__device__ __forceinline__ void tp_per_path_backward(const float* x, const float* y, const float* h,
                                                     float* gx, float* gy) {
    static_for<kNumEntries>([&](auto kk) {
        constexpr CGEntry e = kCG[decltype(kk)::value];
        const float ch = e.c * h[e.q];
        gx[e.a] = fmaf(ch, y[e.b], gx[e.a]);
        gy[e.b] = fmaf(ch, x[e.a], gy[e.b]);
    });
}

// ---------------------------------------------------------------------------
// Output groups of the weighted product: slot q (path, m_out) belongs to group
// kSlotOut[q] / 4, i.e. output components o in [4G, 4G + 4).  Per-path sums
// stored for the weighted scatter's mixing stage list the slots group by group,
// in slot order within a group (fwd_slot_pos).
// ---------------------------------------------------------------------------
constexpr int kFwdGroups = 4;
constexpr bool fwd_in_group(int q, int G) { return kSlotOut[q] / 4 == G; }
constexpr int fwd_group_size(int G) {
    int c = 0;
    for (int q = 0; q < kNumSlots; ++q) c += fwd_in_group(q, G) ? 1 : 0;
    return c;
}
constexpr int fwd_local(int q, int G) {
    int c = 0;
    for (int i = 0; i < q; ++i) c += fwd_in_group(i, G) ? 1 : 0;
    return c;
}
constexpr int fwd_group_base(int G) {
    int c = 0;
    for (int i = 0; i < G; ++i) c += fwd_group_size(i);
    return c;
}
constexpr int fwd_slot_pos(int q) {
    return fwd_group_base(kSlotOut[q] / 4) + fwd_local(q, kSlotOut[q] / 4);
}

// ---------------------------------------------------------------------------
// small helpers
// ---------------------------------------------------------------------------
__host__ __device__ inline int64_t ceil_div(int64_t a, int64_t b) { return (a + b - 1) / b; }

// A wave-uniform 64-bit value in scalar registers.
__device__ __forceinline__ int64_t uniform_i64(int64_t v) {
    const uint32_t lo = __builtin_amdgcn_readfirstlane((uint32_t)v);
    const uint32_t hi = __builtin_amdgcn_readfirstlane((uint32_t)((uint64_t)v >> 32));
    return (int64_t)(((uint64_t)hi << 32) | lo);
}

// Inclusive sum over the lanes of a wave: row_shr 1, 2, 4, 8 within each row of 16,
// then the rows' totals by row_bcast 15 and 31 (lanes with no source add 0).  Every
// lane of the wave must execute it.
__device__ __forceinline__ int wave_incl_scan(int x) {
    x += __builtin_amdgcn_update_dpp(0, x, 0x111, 0xf, 0xf, false);
    x += __builtin_amdgcn_update_dpp(0, x, 0x112, 0xf, 0xf, false);
    x += __builtin_amdgcn_update_dpp(0, x, 0x114, 0xf, 0xf, false);
    x += __builtin_amdgcn_update_dpp(0, x, 0x118, 0xf, 0xf, false);
    x += __builtin_amdgcn_update_dpp(0, x, 0x142, 0xa, 0xf, false);
    x += __builtin_amdgcn_update_dpp(0, x, 0x143, 0xc, 0xf, false);
    return x;
}

// OR of x over lanes 0..15, returned uniform: row_shr 1, 2, 4, 8 inside the first row
// of 16 lanes (lanes with no source take 0), then lane 15.  Every lane of the wave
// must execute it.
__device__ __forceinline__ uint32_t row0_or(uint32_t x) {
    int v = (int)x;
    v |= __builtin_amdgcn_update_dpp(0, v, 0x111, 0xf, 0xf, false);
    v |= __builtin_amdgcn_update_dpp(0, v, 0x112, 0xf, 0xf, false);
    v |= __builtin_amdgcn_update_dpp(0, v, 0x114, 0xf, 0xf, false);
    v |= __builtin_amdgcn_update_dpp(0, v, 0x118, 0xf, 0xf, false);
    return (uint32_t)__builtin_amdgcn_readlane(v, 15);
}

}  // namespace bmhip

// Status codes returned by the C ABI (0 = success).
#define BM_OK 0
#define BM_ERR_ARG -1
#define BM_ERR_WORKSPACE -2
