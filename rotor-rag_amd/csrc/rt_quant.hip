// Per-token absmax int8 activation quantiser, optionally fused with the operation
// that produces the activations (RMSNorm, relu^2(gate)*up), and the int8 permute used
// by the int32 parity entry point.
//
// Quantiser: src/rotor/quantization.py:137-149 (bits = 8, symmetric) applied to every
// row: s = max|v| / 127 (1 when the row is all zero), q = clip(rint(v / s), -128, 127).
// Bit-exactness against NumPy needs IEEE fp32 division (HIP's default `/`, which is
// correctly rounded; this library is never built with fast-math) and round-half-even
// (rintf -> v_rndne_f32); max|v| is order independent.
// RMSNorm: src/rotor/transformer.py:24-36 (x / sqrt(mean(x^2) + eps) * w); the mean of
// squares is accumulated in f64 and rounded once to f32, so its value does not depend
// on the summation order (the reference's fp32 pairwise mean agrees to ~1 ulp).
// relu^2(gate) * up: the FFN activation of the benchmark configuration, optionally
// followed by the FFN sub-norm (BitNet's ffn_sub_norm, src/rotor/transformer.py:336-337).
//
// One 256-thread workgroup per token row.  Each thread holds groups of 16 elements in
// registers (rows up to 16384 elements; longer rows recompute from memory), reduces
// (wave shuffles + LDS), converts its groups and writes each as one 16-byte store in
// the permuted qx order (rt_internal.h).  Rows in [M, Mpad) are zero-filled.
#include "rt_internal.h"

namespace rt {

constexpr int kRegGroups = 4;  // rows of up to 4*256*16 = 16384 elements stay in registers

__device__ __forceinline__ QuantProb select_quant(const QuantArgs& a, int i) { return a.dev ? a.dev[i] : a.p; }

template <typename T, typename Op>
__device__ __forceinline__ T block_reduce_256(T v, T* red, Op op) {
#pragma unroll
    for (int off = 32; off >= 1; off >>= 1) v = op(v, __shfl_xor(v, off, 64));
    const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
    __syncthreads();  // `red` may still be read by a previous reduction
    if (lane == 0) red[wave] = v;
    __syncthreads();
    return op(op(red[0], red[1]), op(red[2], red[3]));
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

// The values to quantise for group g, before any row-wide normalisation:
// kQuant/kRmsNorm: x; kRelu2Mul: relu(gate)^2 * up.
__device__ __forceinline__ void source_group(const QuantProb& P, const float* xr, const float* ur, int g, bool vec,
                                             float (&v)[16]) {
    load_group(xr, g, P.K, vec, v);
    if (P.mode == kRelu2Mul || P.mode == kRelu2MulNorm) {
        float u[16];
        load_group(ur, g, P.K, vec, u);
#pragma unroll
        for (int e = 0; e < 16; ++e) v[e] = v[e] > 0.0f ? (v[e] * v[e]) * u[e] : 0.0f;
    }
}

__device__ __forceinline__ bool has_norm(const QuantProb& P) { return P.mode == kRmsNorm || P.mode == kRelu2MulNorm; }
__device__ __forceinline__ const float* norm_weight(const QuantProb& P) { return P.mode == kRmsNorm ? P.aux : P.aux2; }

// kRmsNorm / kRelu2MulNorm: h = (v / norm) * w for group g
__device__ __forceinline__ void rmsnorm_group(const QuantProb& P, float norm, int g, bool vec, float (&v)[16]) {
    float w[16];
    load_group(norm_weight(P), g, P.K, vec, w);
#pragma unroll
    for (int e = 0; e < 16; ++e) v[e] = (v[e] / norm) * w[e];
}

// q = clip(rint(v / s), -128, 127) for one group; permuted 16-byte store to qx and,
// when requested, the natural-order bytes and the fp32 values.
__device__ __forceinline__ void emit_group(const float (&v)[16], float s, int g, int K, v4u* qrow, int8_t* qn,
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

__global__ void __launch_bounds__(256) quant_kernel(QuantArgs a) {
    __shared__ float redf[4];
    __shared__ double redd[4];
    const QuantProb P = select_quant(a, blockIdx.y);
    const int m = blockIdx.x;
    const int K = P.K, Kp = P.Kp, groups = Kp >> 4;
    v4u* qrow = reinterpret_cast<v4u*>(P.qx + (size_t)m * Kp);
    if (m >= a.M) {  // padding token rows
        const v4u z = {0u, 0u, 0u, 0u};
        for (int g = threadIdx.x; g < groups; g += blockDim.x) qrow[g] = z;
        if (threadIdx.x == 0 && P.sx) P.sx[m] = 0.0f;
        return;
    }
    if (P.mode == kPermute) {  // int8 in natural order -> qx
        const int8_t* qr = P.q_in + (size_t)m * K;
        for (int g = threadIdx.x; g < groups; g += blockDim.x) {
            int q[16];
#pragma unroll
            for (int e = 0; e < 16; ++e) {
                const int k = g * 16 + e;
                q[e] = k < K ? (int)qr[k] : 0;
            }
            qrow[g] = pack_permuted(q);
        }
        if (threadIdx.x == 0 && P.sx) P.sx[m] = 1.0f;
        return;
    }
    const float* xr = P.x + (size_t)m * K;
    const float* ur = (P.mode == kRelu2Mul || P.mode == kRelu2MulNorm) ? P.aux + (size_t)m * K : nullptr;
    int8_t* qn = P.q_nat ? P.q_nat + (size_t)m * K : nullptr;
    float* vo = P.v_out ? P.v_out + (size_t)m * K : nullptr;
    bool vec = (K & 15) == 0 && ((uintptr_t)xr & 15u) == 0;
    if (ur) vec = vec && ((uintptr_t)ur & 15u) == 0;
    if (has_norm(P)) vec = vec && ((uintptr_t)norm_weight(P) & 15u) == 0;
    auto fmax_op = [](float x, float y) { return fmaxf(x, y); };
    auto dadd_op = [](double x, double y) { return x + y; };

    if (groups <= kRegGroups * 256) {  // the row stays in registers
        float v[kRegGroups][16];
#pragma unroll
        for (int r = 0; r < kRegGroups; ++r) source_group(P, xr, ur, threadIdx.x + r * 256, vec, v[r]);
        if (has_norm(P)) {
            double ss = 0.0;
#pragma unroll
            for (int r = 0; r < kRegGroups; ++r) ss = sumsq_group(v[r], ss);
            ss = block_reduce_256(ss, redd, dadd_op);
            const float norm = sqrtf((float)(ss / (double)K) + P.eps);
#pragma unroll
            for (int r = 0; r < kRegGroups; ++r) rmsnorm_group(P, norm, threadIdx.x + r * 256, vec, v[r]);
        }
        float amax = 0.0f;
#pragma unroll
        for (int r = 0; r < kRegGroups; ++r) amax = amax_group(v[r], amax);
        amax = block_reduce_256(amax, redf, fmax_op);
        const float s = amax > 0.0f ? amax / 127.0f : 1.0f;
#pragma unroll
        for (int r = 0; r < kRegGroups; ++r) {
            const int g = threadIdx.x + r * 256;
            if (g < groups) emit_group(v[r], s, g, K, qrow, qn, vo);
        }
        if (threadIdx.x == 0 && P.sx) P.sx[m] = s;
        return;
    }
    // long rows: recompute the source values on every pass
    float norm = 1.0f;
    if (has_norm(P)) {
        double ss = 0.0;
        for (int g = threadIdx.x; g < groups; g += blockDim.x) {
            float v[16];
            source_group(P, xr, ur, g, vec, v);
            ss = sumsq_group(v, ss);
        }
        ss = block_reduce_256(ss, redd, dadd_op);
        norm = sqrtf((float)(ss / (double)K) + P.eps);
    }
    float amax = 0.0f;
    for (int g = threadIdx.x; g < groups; g += blockDim.x) {
        float v[16];
        source_group(P, xr, ur, g, vec, v);
        if (has_norm(P)) rmsnorm_group(P, norm, g, vec, v);
        amax = amax_group(v, amax);
    }
    amax = block_reduce_256(amax, redf, fmax_op);
    const float s = amax > 0.0f ? amax / 127.0f : 1.0f;
    for (int g = threadIdx.x; g < groups; g += blockDim.x) {
        float v[16];
        source_group(P, xr, ur, g, vec, v);
        if (has_norm(P)) rmsnorm_group(P, norm, g, vec, v);
        emit_group(v, s, g, K, qrow, qn, vo);
    }
    if (threadIdx.x == 0 && P.sx) P.sx[m] = s;
}

__global__ void __launch_bounds__(256) unpermute_kernel(const int8_t* __restrict__ qx, int K, int Kp,
                                                        int8_t* __restrict__ q) {
    const int m = blockIdx.y;
    const int k = blockIdx.x * blockDim.x + threadIdx.x;
    if (k >= K) return;
    const int g = k >> 4, e = k & 15;  // element e of group g sits at byte 4*(e%4) + e/4
    q[(size_t)m * K + k] = qx[(size_t)m * Kp + g * 16 + 4 * (e & 3) + (e >> 2)];
}

hipError_t launch_unpermute(const int8_t* qx, int M, int K, int Kp, int8_t* q, hipStream_t s) {
    hipLaunchKernelGGL(unpermute_kernel, dim3((unsigned)((K + 255) / 256), (unsigned)M), dim3(256), 0, s, qx, K, Kp, q);
    return hipGetLastError();
}

hipError_t launch_quant(const QuantArgs& a, hipStream_t s) {
    if (a.U <= 0 || a.Mpad <= 0) return hipSuccess;
    hipLaunchKernelGGL(quant_kernel, dim3((unsigned)a.Mpad, (unsigned)a.U), dim3(256), 0, s, a);
    return hipGetLastError();
}

}  // namespace rt
