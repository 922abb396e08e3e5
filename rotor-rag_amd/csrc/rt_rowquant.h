// Device helpers that turn one token row into int8 activations in the qx layout:
// the per-token absmax quantiser, optionally fused with the operation producing the row
// (RMSNorm, relu^2(gate)*up, relu^2(gate)*up followed by RMSNorm).  Shared by the
// quantiser kernel (rt_quant.hip, destination global memory) and the decode GEMV
// prologue (rt_gemv.hip, destination LDS).  Any workgroup size that is a multiple of 64
// up to 1024 works.
//
// Quantiser: src/rotor/quantization.py:137-149 (bits = 8, symmetric) applied per row:
// s = max|v| / 127 (1 when the row is all zero), q = clip(rint(v / s), -128, 127), with
// IEEE fp32 division (HIP's default `/`; never built with fast-math) and round-half-even
// (rintf -> v_rndne_f32); max|v| is order independent.
// RMSNorm: src/rotor/transformer.py:24-36 (x / sqrt(mean(x^2) + eps) * w); the mean of
// squares is accumulated in f64 and rounded once to f32, so its value does not depend
// on the summation order.
#pragma once

#include "rt_internal.h"

// every product and sum below rounds on its own unless written as fmaf (this header is
// included before the sources' own pragmas)
#pragma clang fp contract(off)

namespace rt {

typedef __attribute__((address_space(3))) float lfloat;

struct RowSmem {   // reduction scratch in LDS (one slot per wave)
    float f[16];
    double d[16];
    int qs[16];    // the 4- / 8-element and attention prologues: each wave's sum of its quantised values
    lfloat* fac;   // kAttnNorm: [heads][S] combine factors (-1 = empty block), then [heads] denominators
};

// op over the n (<= 64) slots red[0 .. n): lane l reads slot l, one DPP reduction (no chain of
// dependent LDS reads); the total is returned to every lane.  0 is the identity of op.
template <typename T, typename Op>
__device__ __forceinline__ T slots_reduce(const T* red, int n, Op op) {
    const int lane = threadIdx.x & 63;
    return lane63(wave_reduce63(lane < n ? red[lane] : T(0), T(0), op));
}

// Workgroup reduction through one slot per wave.  Each slot array serves one reduction
// per row_quantize call (sums in RowSmem::d, maxima in RowSmem::f), so no barrier is
// needed before the slots are written.  Every use reduces values >= 0 (sums of squares,
// maxima of |v|), so 0 is the identity of op.
// `wave_live` (wave-uniform) false: the wave only contributes v (the identity) and
// skips the DPP steps.
template <typename T, typename Op>
__device__ __forceinline__ T block_reduce(T v, T* red, Op op, bool wave_live = true) {
    if (wave_live) v = wave_reduce63(v, T(0), op);
    const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63, nw = blockDim.x >> 6;
    if (lane == 63) red[wave] = v;
    __syncthreads();
    return slots_reduce(red, nw, op);
}

// byte p (0..15) of a permuted group holds element 4*(p%4) + p/4 of the group
__device__ __forceinline__ v4u pack_permuted(const int (&q)[16]) {
    v4u o;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        unsigned d = 0u;
#pragma unroll
        for (int b = 0; b < 4; ++b) d |= ((unsigned)q[4 * b + i] & 0xffu) << (8 * b);
        o[i] = d;
    }
    return o;
}

// 16 elements of group g (k = 16g .. 16g+15) of a row; zeros past K.  `vec`: the row is
// 16-byte aligned with K % 16 == 0; groups wholly inside the row are then read as four
// float4 (the padding groups of Kp > K are never read).
__device__ __forceinline__ void load_group(const float* __restrict__ xr, int g, int K, bool vec, float (&v)[16]) {
    if (vec && (g + 1) * 16 <= K) {
        const float4* p = reinterpret_cast<const float4*>(xr + g * 16);
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            const float4 t = p[i];
            v[4 * i + 0] = t.x;
            v[4 * i + 1] = t.y;
            v[4 * i + 2] = t.z;
            v[4 * i + 3] = t.w;
        }
    } else {
#pragma unroll
        for (int e = 0; e < 16; ++e) {
            const int k = g * 16 + e;
            v[e] = k < K ? xr[k] : 0.0f;
        }
    }
}

__device__ __forceinline__ bool has_norm(const QuantProb& P) {
    return P.mode == kRmsNorm || P.mode == kRelu2MulNorm || P.mode == kAttnNorm || P.mode == kRmsNormSsq;
}
__device__ __forceinline__ bool has_relu2(const QuantProb& P) { return P.mode == kRelu2Mul || P.mode == kRelu2MulNorm; }
__device__ __forceinline__ const float* norm_weight(const QuantProb& P) {
    return P.mode == kRelu2MulNorm ? P.aux2 : P.aux;
}

// Output element d of head h from decode-attention partials work[h][s][0..hd+2)
// (unnormalised sum, block max, block sum of exponentials):
// o = sum_s e^(m_s - m) o_s[d] / sum_s e^(m_s - m) z_s, m = max_s m_s, empty blocks skipped;
// both sums are fused multiply-adds over s in order (every combine of the partials, here,
// in attn_factors / the o_proj prologue and in the q/k/v launch, uses this order).
__device__ __forceinline__ float attn_combine_element(const float* __restrict__ work, int hd, int S, int h, int d) {
    const float* wh = work + (size_t)h * S * (hd + 2);
    float mx = -INFINITY;
    for (int i = 0; i < S; ++i) mx = fmaxf(mx, wh[(size_t)i * (hd + 2) + hd]);
    float num = 0.0f, den = 0.0f;
    for (int i = 0; i < S; ++i) {
        const float* pi = wh + (size_t)i * (hd + 2);
        const float m_i = pi[hd];
        if (m_i == -INFINITY) continue;
        const float f = expf(m_i - mx);
        num = fmaf(f, pi[d], num);
        den = fmaf(f, pi[hd + 1], den);
    }
    return num / den;
}

// The values of group g before any row-wide normalisation:
// kQuant/kRmsNorm: x; kRelu2Mul(Norm): relu(gate)^2 * up.
// kAttnNorm, per head h: the factor e^(m_s - m) of every partial block (-1 for an
// empty block) and the denominator sum_s e^(m_s - m) z_s, in the operation order of
// attn_combine_element.
__device__ __forceinline__ void attn_factors(const QuantProb& P, lfloat* fac) {
    const int hd = P.attn_hd, S = P.attn_S, H = P.K / hd;
    for (int h = threadIdx.x; h < H; h += blockDim.x) {
        const float* wh = P.x + (size_t)h * S * (hd + 2);
        float mx = -INFINITY;
        for (int i = 0; i < S; ++i) mx = fmaxf(mx, wh[(size_t)i * (hd + 2) + hd]);
        float den = 0.0f;
        for (int i = 0; i < S; ++i) {
            const float m_i = wh[(size_t)i * (hd + 2) + hd];
            if (m_i == -INFINITY) {
                fac[h * S + i] = -1.0f;
                continue;
            }
            const float f = expf(m_i - mx);
            fac[h * S + i] = f;
            den = fmaf(f, wh[(size_t)i * (hd + 2) + hd + 1], den);
        }
        fac[H * S + h] = den;
    }
}

__device__ __forceinline__ void source_group(const QuantProb& P, const float* xr, const float* ur, int g, bool vec,
                                             float (&v)[16], const lfloat* fac = nullptr) {
    if (P.mode == kAttnNorm) {  // 16 consecutive elements of one head (hd % 16 == 0)
        const int hd = P.attn_hd, S = P.attn_S, H = P.K / hd;
        const int k0 = g * 16, h = k0 / hd, d0 = k0 % hd;
        if (k0 >= P.K) {
#pragma unroll
            for (int e = 0; e < 16; ++e) v[e] = 0.0f;
            return;
        }
        float num[16];
#pragma unroll
        for (int e = 0; e < 16; ++e) num[e] = 0.0f;
        const float* wh = P.x + (size_t)h * S * (hd + 2) + d0;
        for (int i = 0; i < S; ++i) {
            const float f = fac[h * S + i];
            if (f < 0.0f) continue;
            const float4* p = reinterpret_cast<const float4*>(wh + (size_t)i * (hd + 2));
#pragma unroll
            for (int q4 = 0; q4 < 4; ++q4) {
                const float4 t = p[q4];
                num[4 * q4 + 0] = fmaf(f, t.x, num[4 * q4 + 0]);
                num[4 * q4 + 1] = fmaf(f, t.y, num[4 * q4 + 1]);
                num[4 * q4 + 2] = fmaf(f, t.z, num[4 * q4 + 2]);
                num[4 * q4 + 3] = fmaf(f, t.w, num[4 * q4 + 3]);
            }
        }
        const float den = fac[H * S + h];
#pragma unroll
        for (int e = 0; e < 16; ++e) v[e] = num[e] / den;
        return;
    }
    load_group(xr, g, P.K, vec, v);
    if (has_relu2(P)) {
        float u[16];
        load_group(ur, g, P.K, vec, u);
#pragma unroll
        for (int e = 0; e < 16; ++e) v[e] = v[e] > 0.0f ? (v[e] * v[e]) * u[e] : 0.0f;
    }
}

// h = (v / norm) * w for group g
__device__ __forceinline__ void rmsnorm_group(const QuantProb& P, float norm, int g, bool vec, float (&v)[16]) {
    float w[16];
    load_group(norm_weight(P), g, P.K, vec, w);
#pragma unroll
    for (int e = 0; e < 16; ++e) v[e] = (v[e] / norm) * w[e];
}

// Destination of one row's permuted 16-byte groups: group g at
// base[(g / 4) * chunk + (g % 4) * sub] (v4u units); rows: chunk 4, sub 1; blocked qx:
// chunk 64, sub 16.
struct QxRow {
    v4u* base;
    int chunk, sub;
    __device__ __forceinline__ v4u& operator[](int g) const { return base[(g >> 2) * chunk + (g & 3) * sub]; }
};

// q = clip(rint(v / s), -128, 127) for one group; permuted 16-byte store and, when
// requested, the natural-order bytes and the fp32 values.
__device__ __forceinline__ void emit_group(const float (&v)[16], float s, int g, int K, const QxRow& qrow, int8_t* qn,
                                           float* vo) {
    int q[16];
#pragma unroll
    for (int e = 0; e < 16; ++e) {
        float r = rintf(v[e] / s);
        r = fminf(fmaxf(r, -128.0f), 127.0f);
        q[e] = (int)r;
    }
    qrow[g] = pack_permuted(q);
    if (qn || vo) {
#pragma unroll
        for (int e = 0; e < 16; ++e) {
            const int k = g * 16 + e;
            if (k < K) {
                if (qn) qn[k] = (int8_t)q[e];
                if (vo) vo[k] = v[e];
            }
        }
    }
}

__device__ __forceinline__ float amax_group(const float (&v)[16], float m) {
#pragma unroll
    for (int e = 0; e < 16; ++e) m = fmaxf(m, fabsf(v[e]));
    return m;
}

__device__ __forceinline__ double sumsq_group(const float (&v)[16], double s) {
#pragma unroll
    for (int e = 0; e < 16; ++e) s += (double)v[e] * (double)v[e];
    return s;
}

// One group of 16 per thread (Kp/16 <= threads), modes other than kAttnNorm: the row's
// loads (x, up, norm weight) and, separately, the arithmetic, so a caller can issue its
// own loads in between.  Waves past the row's groups do no arithmetic (they would share
// the SIMDs with the live ones) and only take part in the barriers.
struct RowRegs {
    float v[16], u[16], w[16];
    bool live;  // wave-uniform: some lane of this wave owns a group
};

__device__ __forceinline__ bool row_vec(const QuantProb& P, const float* xr, const float* ur) {
    bool vec = (P.K & 15) == 0 && ((uintptr_t)xr & 15u) == 0 && P.mode != kAttnNorm;
    if (ur) vec = vec && ((uintptr_t)ur & 15u) == 0;
    if (has_norm(P)) vec = vec && ((uintptr_t)norm_weight(P) & 15u) == 0;
    return vec;
}

__device__ __forceinline__ void row_load1(const QuantProb& P, int m, RowRegs& r) {
    const int K = P.K, groups = P.Kp >> 4, g = threadIdx.x;
    const float* xr = P.x + (size_t)m * K;
    const float* ur = has_relu2(P) ? P.aux + (size_t)m * K : nullptr;
    const bool vec = row_vec(P, xr, ur);
    r.live = __builtin_amdgcn_readfirstlane(threadIdx.x & ~63) < groups;
#pragma unroll
    for (int e = 0; e < 16; ++e) r.v[e] = r.u[e] = r.w[e] = 0.0f;
    if (r.live) {
        load_group(xr, g, K, vec, r.v);  // zeros past K
        if (ur) load_group(ur, g, K, vec, r.u);
        if (has_norm(P)) load_group(norm_weight(P), g, K, vec, r.w);
    }
}

__device__ __forceinline__ float row_finish1(const QuantProb& P, RowRegs& r, const QxRow& qrow, int8_t* qn, float* vo,
                                             RowSmem* sm) {
    auto fmax_op = [](float x, float y) { return fmaxf(x, y); };
    auto dadd_op = [](double x, double y) { return x + y; };
    const int K = P.K, groups = P.Kp >> 4, g = threadIdx.x;
    float (&v)[16] = r.v;
    if (r.live && has_relu2(P)) {
#pragma unroll
        for (int e = 0; e < 16; ++e) v[e] = v[e] > 0.0f ? (v[e] * v[e]) * r.u[e] : 0.0f;
    }
    if (has_norm(P)) {
        const double ss = block_reduce(r.live ? sumsq_group(v, 0.0) : 0.0, sm->d, dadd_op, r.live);
        const float norm = sqrtf((float)(ss / (double)K) + P.eps);
        if (r.live) {
#pragma unroll
            for (int e = 0; e < 16; ++e) v[e] = (v[e] / norm) * r.w[e];
        }
    }
    const float amax = block_reduce(r.live ? amax_group(v, 0.0f) : 0.0f, sm->f, fmax_op, r.live);
    const float s = amax > 0.0f ? amax / 127.0f : 1.0f;
    if (g < groups) emit_group(v, s, g, K, qrow, qn, vo);
    return s;
}

// True when row_load1 / row_finish1 apply to P with T threads.
__device__ __forceinline__ bool row_fits1(const QuantProb& P, int T) {
    return P.mode != kAttnNorm && (P.Kp >> 4) <= T;
}

// E (4 or 8) consecutive elements per thread (K % 64 == 0, K / E <= threads): thread t
// owns elements k = E t .. E t + E - 1, read with E / 4 16-byte loads per operand.  In the
// permuted layout element k = 16 g + e of group g sits at byte 4 (e % 4) + e / 4, and
// scatter_q writes the thread's int8 values to the LDS row one byte each.  Few elements
// per thread spread the row's arithmetic over many waves.
typedef float v4f_a8 __attribute__((ext_vector_type(4), aligned(8)));
typedef float v2f_a8 __attribute__((ext_vector_type(2), aligned(8)));

// v[j] / d for fp32 elements and one fp32 divisor d > 0, computed as fl32(v fl64(1 / d)):
// the f64 product is within 2^-52 (relative) of v / d, and a quotient in the normal range
// lies at least 2^-49 (relative) from every rounding midpoint of fp32 (for a midpoint m in
// [2^e, 2^(e+1)), v - m d is a non-zero multiple of 2^(e + e_d - 47)), so the rounded product
// is the correctly rounded quotient, at a third of the IEEE division's instructions.  A
// subnormal quotient can sit exactly on a midpoint: when a non-zero element's product lands
// at or below 2^-126 the thread takes the IEEE division for all its elements.
template <int E>
__device__ __forceinline__ void divide_all(float (&v)[E], float d) {
    const double r = 1.0 / (double)d;
    float c[E];
    bool tiny = false;
#pragma unroll
    for (int j = 0; j < E; ++j) {
        c[j] = (float)((double)v[j] * r);
        tiny = tiny || (v[j] != 0.0f && fabsf(c[j]) <= 0x1p-126f);
    }
    if (tiny) {
#pragma unroll
        for (int j = 0; j < E; ++j) c[j] = v[j] / d;
    }
#pragma unroll
    for (int j = 0; j < E; ++j) v[j] = c[j];
}

// Writes rint(v[j] / sc), clamped to the int8 range, to the LDS row (one byte each) and
// returns their sum.  v / sc as in divide_all; a quotient at or below 2^-126 in magnitude,
// where the product may round differently, rounds to 0 either way.
template <int E>
__device__ __forceinline__ int scatter_q(const float (&v)[E], float sc, v4u* lq) {
    const double r = 1.0 / (double)sc;
    int q[E], s = 0;
#pragma unroll
    for (int j = 0; j < E; ++j) {
        const float f = rintf((float)((double)v[j] * r));
        q[j] = (int)fminf(fmaxf(f, -128.0f), 127.0f);
        s += q[j];
    }
    if constexpr (E == 16) {  // the thread's elements are one whole group: one 16-byte write
        lq[threadIdx.x] = pack_permuted(q);
    } else {
        unsigned char* lb = reinterpret_cast<unsigned char*>(lq);
        const int k0 = E * (int)threadIdx.x;
#pragma unroll
        for (int j = 0; j < E; ++j) {
            const int k = k0 + j, e = k & 15;
            lb[(k & ~15) + 4 * (e & 3) + (e >> 2)] = (unsigned char)q[j];
        }
    }
    return s;
}

// The wave's sum of its quantised values into its slot RowSmem::qs (read after the caller's
// barrier): a GEMV subtracts the row's total once instead of every wave summing its slice.
__device__ __forceinline__ void qsum_to_slot(int s, RowSmem* sm, bool live) {
    if (live) s = wave_reduce63(s, 0, [](int a, int b) { return a + b; });
    if ((threadIdx.x & 63) == 63) sm->qs[threadIdx.x >> 6] = s;
}

template <int E>
struct RowRegsE {
    float v[E], u[E], w[E];
    double ssq[4];  // kRmsNormSsq: partial sums of squares l, l + 64, .. of this lane
    bool live;      // wave-uniform: some lane of this wave owns elements
};

template <int E>
__device__ __forceinline__ void loadE(const float* p, float (&v)[E]) {
#pragma unroll
    for (int i = 0; i < E / 4; ++i) {
        const v4f_a8 t = *reinterpret_cast<const v4f_a8*>(p + 4 * i);
#pragma unroll
        for (int j = 0; j < 4; ++j) v[4 * i + j] = t[j];
    }
}

template <int E>
__device__ __forceinline__ void row_loadE(const QuantProb& P, RowRegsE<E>& r) {
    const int t = threadIdx.x, K = P.K;
    r.live = __builtin_amdgcn_readfirstlane(threadIdx.x & ~63) < K / E;
#pragma unroll
    for (int j = 0; j < E; ++j) r.v[j] = r.u[j] = r.w[j] = 0.0f;
    if (t < K / E) {
        loadE<E>(P.x + E * t, r.v);
        if (has_relu2(P)) loadE<E>(P.aux + E * t, r.u);
        if (has_norm(P)) loadE<E>(norm_weight(P) + E * t, r.w);
    }
#pragma unroll
    for (int i = 0; i < 4; ++i) r.ssq[i] = 0.0;
    if (P.mode == kRmsNormSsq && r.live) {  // K / 32 <= 256 partials (K <= 8192): up to four per lane
        const double* pp = reinterpret_cast<const double*>(P.aux2);
        const int lane = threadIdx.x & 63, n = K >> 5;
#pragma unroll
        for (int i = 0; i < 4; ++i)
            if (lane + 64 * i < n) r.ssq[i] = pp[lane + 64 * i];
    }
}

// Reduction over the waves that hold the row (the first nlive, `live`): they reduce their
// values into slots, every wave passes the barrier, the live waves reduce the nlive slots.
// Waves without elements spend nothing but the barrier.
template <typename T, typename Op>
__device__ __forceinline__ T live_reduce(T v, T* red, Op op, bool live, int nlive) {
    if (live) {
        v = wave_reduce63(v, T(0), op);
        if ((threadIdx.x & 63) == 63) red[threadIdx.x >> 6] = v;
    }
    __syncthreads();
    return live ? slots_reduce(red, nlive, op) : T(0);
}

// The row's RMSNorm / relu^2 and absmax quantisation into the LDS row.  Waves that own no
// element (not live) take part in the barriers only; the returned scale and the RowSmem::qs
// slots are those of the live waves (wave 0 always is one: K >= 64).
template <int E>
__device__ __forceinline__ float row_finishE(const QuantProb& P, RowRegsE<E>& r, v4u* lq, RowSmem* sm) {
    auto fmax_op = [](float x, float y) { return fmaxf(x, y); };
    auto dadd_op = [](double x, double y) { return x + y; };
    const int t = threadIdx.x, K = P.K, nlive = (K / E + 63) >> 6;
    const bool mine = t < K / E;
    float (&v)[E] = r.v;
    if (mine && has_relu2(P)) {
#pragma unroll
        for (int j = 0; j < E; ++j) v[j] = v[j] > 0.0f ? (v[j] * v[j]) * r.u[j] : 0.0f;
    }
    if (has_norm(P)) {
        double ss = 0.0;
        if (P.mode == kRmsNormSsq) {  // every live wave adds the given partials, in one order
            if (r.live) ss = lane63(wave_reduce63((r.ssq[0] + r.ssq[1]) + (r.ssq[2] + r.ssq[3]), 0.0, dadd_op));
        } else {
#pragma unroll
            for (int j = 0; j < E; ++j) ss += (double)v[j] * (double)v[j];
            ss = live_reduce(ss, sm->d, dadd_op, r.live, nlive);
        }
        if (r.live) {
            const float norm = sqrtf((float)(ss / (double)K) + P.eps);
            if (mine) {
                divide_all<E>(v, norm);
#pragma unroll
                for (int j = 0; j < E; ++j) v[j] = v[j] * r.w[j];
            }
        }
    }
    float amax = 0.0f;
#pragma unroll
    for (int j = 0; j < E; ++j) amax = fmaxf(amax, fabsf(v[j]));
    amax = live_reduce(amax, sm->f, fmax_op, r.live, nlive);
    float sc = 1.0f;
    if (r.live) {
        sc = amax > 0.0f ? amax / 127.0f : 1.0f;
        qsum_to_slot(mine ? scatter_q<E>(v, sc, lq) : 0, sm, true);
    }
    return sc;
}

// kAttnNorm for one token with K % 64 == 0 and at most kAttnSMax partial blocks, four
// consecutive elements k = 4 t .. 4 t + 3 per thread (one head h = k / hd, dims
// d = k % hd ..): attn_load1 issues every load the thread needs at once -- per block one
// 16-byte load of its four values and one 8-byte load of the block's (max, sum) -- and its
// four norm weights; attn_finish1 combines them in the operation order of
// attn_combine_element, then RMSNorm and quantisation as row_finish4.
constexpr int kAttnSMax = 10;  // Lmax <= 640 (longer contexts take the general path)
struct AttnRegs {
    float p[kAttnSMax][4], m[kAttnSMax], z[kAttnSMax], w[4];
    bool live;  // wave-uniform: some lane of this wave owns elements
};

__device__ __forceinline__ bool attn_fits1(const QuantProb& P, int T) {
    return P.mode == kAttnNorm && P.attn_S <= kAttnSMax && (P.K & 63) == 0 && P.K / 4 <= T &&
           P.attn_hd % 16 == 0;
}

__device__ __forceinline__ void attn_load1(const QuantProb& P, AttnRegs& r) {
    const int K = P.K, hd = P.attn_hd, S = P.attn_S;
    r.live = __builtin_amdgcn_readfirstlane(threadIdx.x & ~63) < K / 4;
    // Straight-line loads, no branch: threads past K / 4 re-read the last thread's
    // elements and blocks past S re-read block S - 1; the combine ignores both.
    // Raw buffer loads: one resource for the partials, the lane's offset in a VGPR and the
    // block stride in the scalar offset, so the 2 S loads need no per-load address registers.
    const int t = min((int)threadIdx.x, K / 4 - 1);
    const int k0 = 4 * t, h = k0 / hd, d = k0 % hd, row = (hd + 2) * 4;
    const __amdgpu_buffer_rsrc_t rs = __builtin_amdgcn_make_buffer_rsrc(
        (void*)P.x, 0, (unsigned)((K / hd) * S * row), kBufDword3);
    const int off = h * S * row;
#pragma unroll
    for (int s = 0; s < kAttnSMax; ++s) {
        const int so = min(s, S - 1) * row;
        const v4f_a8 pv = __builtin_bit_cast(v4f_a8, __builtin_amdgcn_raw_buffer_load_b128(rs, off + 4 * d, so, 0));
        const v2f_a8 mz = __builtin_bit_cast(v2f_a8, __builtin_amdgcn_raw_buffer_load_b64(rs, off + 4 * hd, so, 0));
#pragma unroll
        for (int j = 0; j < 4; ++j) r.p[s][j] = pv[j];
        r.m[s] = mz[0];
        r.z[s] = mz[1];
    }
    loadE<4>(P.aux + k0, r.w);
}

// The combine (attn_combine1, ends the AttnRegs' lifetime) and the RMSNorm +
// quantisation (attn_norm1) are separate so a caller can issue loads in between.
__device__ __forceinline__ void attn_combine1(const QuantProb& P, const AttnRegs& r, float (&v)[4]) {
    const int t = threadIdx.x, K = P.K, S = P.attn_S;
    const bool mine = t < K / 4;
#pragma unroll
    for (int j = 0; j < 4; ++j) v[j] = 0.0f;
    if (mine) {
        float mx = -INFINITY;
#pragma unroll
        for (int s = 0; s < kAttnSMax; ++s)
            if (s < S) mx = fmaxf(mx, r.m[s]);
        float num[4] = {0.0f, 0.0f, 0.0f, 0.0f}, den = 0.0f;
#pragma unroll
        for (int s = 0; s < kAttnSMax; ++s) {
            if (s >= S || r.m[s] == -INFINITY) continue;
            const float f = expf(r.m[s] - mx);
#pragma unroll
            for (int j = 0; j < 4; ++j) num[j] = fmaf(f, r.p[s][j], num[j]);
            den = fmaf(f, r.z[s], den);
        }
        divide_all<4>(num, den);  // den >= 1: the block holding the maximum adds f = 1 times its sum >= 1
#pragma unroll
        for (int j = 0; j < 4; ++j) v[j] = num[j];
    }
}

__device__ __forceinline__ float attn_norm1(const QuantProb& P, float (&v)[4], const float (&w)[4], bool live,
                                            v4u* lq, RowSmem* sm) {
    auto fmax_op = [](float x, float y) { return fmaxf(x, y); };
    auto dadd_op = [](double x, double y) { return x + y; };
    const int t = threadIdx.x, K = P.K;
    const bool mine = t < K / 4;
    double ss = 0.0;
#pragma unroll
    for (int j = 0; j < 4; ++j) ss += (double)v[j] * (double)v[j];
    ss = block_reduce(ss, sm->d, dadd_op, live);
    const float norm = sqrtf((float)(ss / (double)K) + P.eps);
    float amax = 0.0f;
    if (mine) {
        divide_all<4>(v, norm);
#pragma unroll
        for (int j = 0; j < 4; ++j) {
            v[j] = v[j] * w[j];
            amax = fmaxf(amax, fabsf(v[j]));
        }
    }
    amax = block_reduce(amax, sm->f, fmax_op, live);
    const float sc = amax > 0.0f ? amax / 127.0f : 1.0f;
    qsum_to_slot(mine ? scatter_q<4>(v, sc, lq) : 0, sm, live);
    return sc;
}

// Quantise token row m of P (all modes but kPermute) into qrow (Kp/16 permuted groups)
// and return its scale.  Rows of up to REG groups of 16 per thread stay in registers,
// longer rows are read again on every pass.  Every thread of the workgroup must call it
// (it synchronises).
template <int REG>
__device__ __forceinline__ float row_quantize(const QuantProb& P, int m, const QxRow& qrow, int8_t* qn, float* vo,
                                              RowSmem* sm) {
    const int K = P.K, groups = P.Kp >> 4, T = blockDim.x;
    const float* xr = P.x + (size_t)m * K;
    const float* ur = has_relu2(P) ? P.aux + (size_t)m * K : nullptr;
    const bool vec = row_vec(P, xr, ur);
    auto fmax_op = [](float x, float y) { return fmaxf(x, y); };
    auto dadd_op = [](double x, double y) { return x + y; };

    if (P.mode == kAttnNorm) {
        attn_factors(P, sm->fac);
        __syncthreads();
    }
    if (groups <= REG * T) {  // the row stays in registers
        float v[REG][16];
#pragma unroll
        for (int r = 0; r < REG; ++r) source_group(P, xr, ur, threadIdx.x + r * T, vec, v[r], sm->fac);
        if (has_norm(P)) {
            double ss = 0.0;
#pragma unroll
            for (int r = 0; r < REG; ++r) ss = sumsq_group(v[r], ss);
            ss = block_reduce(ss, sm->d, dadd_op);
            const float norm = sqrtf((float)(ss / (double)K) + P.eps);
#pragma unroll
            for (int r = 0; r < REG; ++r) rmsnorm_group(P, norm, threadIdx.x + r * T, vec, v[r]);
        }
        float amax = 0.0f;
#pragma unroll
        for (int r = 0; r < REG; ++r) amax = amax_group(v[r], amax);
        amax = block_reduce(amax, sm->f, fmax_op);
        const float s = amax > 0.0f ? amax / 127.0f : 1.0f;
#pragma unroll
        for (int r = 0; r < REG; ++r) {
            const int g = threadIdx.x + r * T;
            if (g < groups) emit_group(v[r], s, g, K, qrow, qn, vo);
        }
        return s;
    }
    // long rows: recompute the source values on every pass
    float norm = 1.0f;
    if (has_norm(P)) {
        double ss = 0.0;
        for (int g = threadIdx.x; g < groups; g += T) {
            float v[16];
            source_group(P, xr, ur, g, vec, v, sm->fac);
            ss = sumsq_group(v, ss);
        }
        ss = block_reduce(ss, sm->d, dadd_op);
        norm = sqrtf((float)(ss / (double)K) + P.eps);
    }
    float amax = 0.0f;
    for (int g = threadIdx.x; g < groups; g += T) {
        float v[16];
        source_group(P, xr, ur, g, vec, v, sm->fac);
        if (has_norm(P)) rmsnorm_group(P, norm, g, vec, v);
        amax = amax_group(v, amax);
    }
    amax = block_reduce(amax, sm->f, fmax_op);
    const float s = amax > 0.0f ? amax / 127.0f : 1.0f;
    for (int g = threadIdx.x; g < groups; g += T) {
        float v[16];
        source_group(P, xr, ur, g, vec, v, sm->fac);
        if (has_norm(P)) rmsnorm_group(P, norm, g, vec, v);
        emit_group(v, s, g, K, qrow, qn, vo);
    }
    return s;
}

}  // namespace rt
