// Per-token absmax int8 activation quantiser (and the int8 permute used by the
// int32 parity entry point).
//
// Formula: src/rotor/quantization.py:137-149 (bits = 8, symmetric) applied to every
// row: s = max|x| / 127 (1 when the row is all zero), q = clip(rint(x / s), -128, 127).
// Bit-exactness against NumPy needs IEEE fp32 division (HIP's default `/`, which is
// correctly rounded; this library is never built with fast-math) and round-half-even
// (rintf -> v_rndne_f32); max|x| is order independent.
//
// One 256-thread workgroup per token row.  Each thread holds groups of 16 elements in
// registers (rows up to 16384 elements; longer rows take a second pass over x),
// reduces max|x| (wave shuffles + LDS), then converts its groups and writes each as
// one 16-byte store in the permuted qx order (rt_internal.h).  Rows in [M, Mpad)
// are zero-filled.
#include "rt_internal.h"

namespace rt {

__device__ __forceinline__ QuantProb select_quant(const QuantArgs& a, int i) { return a.dev ? a.dev[i] : a.p; }

__device__ __forceinline__ float block_max_256(float v, float* red) {
#pragma unroll
    for (int off = 32; off >= 1; off >>= 1) v = fmaxf(v, __shfl_xor(v, off, 64));
    const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
    if (lane == 0) red[wave] = v;
    __syncthreads();
    v = fmaxf(fmaxf(red[0], red[1]), fmaxf(red[2], red[3]));
    return v;
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

constexpr int kRegGroups = 4;  // rows of up to 4*256*16 = 16384 elements stay in registers

// 16 elements of group g (k = 16g .. 16g+15); zeros past K.  `vec`: the row is
// 16-byte aligned with K % 16 == 0; groups wholly inside the row are then read as
// four float4 (the padding groups of Kp > K are never read).
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

// q = clip(rint(x / s), -128, 127) for one group; permuted 16-byte store to qx and,
// when requested, the natural-order bytes to q_nat.
__device__ __forceinline__ void emit_group(const float (&v)[16], float s, int g, int K, v4u* qrow, int8_t* qn) {
    int q[16];
#pragma unroll
    for (int e = 0; e < 16; ++e) {
        float r = rintf(v[e] / s);
        r = fminf(fmaxf(r, -128.0f), 127.0f);
        q[e] = (int)r;
    }
    qrow[g] = pack_permuted(q);
    if (qn) {
#pragma unroll
        for (int e = 0; e < 16; ++e) {
            const int k = g * 16 + e;
            if (k < K) qn[k] = (int8_t)q[e];
        }
    }
}

__global__ void __launch_bounds__(256) quant_kernel(QuantArgs a) {
    __shared__ float red[4];
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
    if (P.q_in) {  // permute mode: int8 in natural order -> qx
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
    int8_t* qn = P.q_nat ? P.q_nat + (size_t)m * K : nullptr;
    const bool vec = (K & 15) == 0 && ((uintptr_t)xr & 15u) == 0;
    if (groups <= kRegGroups * 256) {
        // x stays in registers between the max-reduction and the conversion
        float v[kRegGroups][16];
        float amax = 0.0f;
#pragma unroll
        for (int r = 0; r < kRegGroups; ++r) {
            const int g = threadIdx.x + r * 256;
            load_group(xr, g, K, vec, v[r]);
#pragma unroll
            for (int e = 0; e < 16; ++e) amax = fmaxf(amax, fabsf(v[r][e]));
        }
        amax = block_max_256(amax, red);
        const float s = amax > 0.0f ? amax / 127.0f : 1.0f;
#pragma unroll
        for (int r = 0; r < kRegGroups; ++r) {
            const int g = threadIdx.x + r * 256;
            if (g < groups) emit_group(v[r], s, g, K, qrow, qn);
        }
        if (threadIdx.x == 0 && P.sx) P.sx[m] = s;
        return;
    }
    // long rows: two passes over x
    float amax = 0.0f;
    for (int g = threadIdx.x; g < groups; g += blockDim.x) {
        float v[16];
        load_group(xr, g, K, vec, v);
#pragma unroll
        for (int e = 0; e < 16; ++e) amax = fmaxf(amax, fabsf(v[e]));
    }
    amax = block_max_256(amax, red);
    const float s = amax > 0.0f ? amax / 127.0f : 1.0f;
    for (int g = threadIdx.x; g < groups; g += blockDim.x) {
        float v[16];
        load_group(xr, g, K, vec, v);
        emit_group(v, s, g, K, qrow, qn);
    }
    if (threadIdx.x == 0 && P.sx) P.sx[m] = s;
}

hipError_t launch_quant(const QuantArgs& a, hipStream_t s) {
    if (a.U <= 0 || a.Mpad <= 0) return hipSuccess;
    hipLaunchKernelGGL(quant_kernel, dim3((unsigned)a.Mpad, (unsigned)a.U), dim3(256), 0, s, a);
    return hipGetLastError();
}

}  // namespace rt
