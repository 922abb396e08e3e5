// Per-token absmax int8 activation quantiser, optionally fused with the operation
// that produces the activations (RMSNorm, relu^2(gate)*up, relu^2(gate)*up followed by
// the FFN sub-norm), and the int8 permute used by the int32 parity entry point.
// The row arithmetic lives in rt_rowquant.h (shared with the decode GEMV prologue).
//
// One 256-thread workgroup per token row; rows in [M, Mpad) are zero-filled.
#include "rt_rowquant.h"

// every fp32 operation rounds on its own, as the reference restatement computes them
#pragma clang fp contract(off)

namespace rt {

__device__ __forceinline__ QuantProb select_quant(const QuantArgs& a, int i) { return a.dev ? a.dev[i] : a.p; }

__global__ void __launch_bounds__(256) quant_kernel(QuantArgs a) {
    __shared__ RowSmem sm;
    const QuantProb P = select_quant(a, blockIdx.y);
    const int m = blockIdx.x;
    const int K = P.K, Kp = P.Kp, groups = Kp >> 4;
    v4u* const qx = reinterpret_cast<v4u*>(P.qx);
    const QxRow qrow = P.blocked ? QxRow{qx + (size_t)(m >> 4) * (Kp >> 6) * 64 + (m & 15), 64, 16}
                                 : QxRow{qx + (size_t)m * (Kp >> 4), 4, 1};
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
    int8_t* qn = P.q_nat ? P.q_nat + (size_t)m * K : nullptr;
    float* vo = P.v_out ? P.v_out + (size_t)m * K : nullptr;
    const float s = row_quantize<4>(P, m, qrow, qn, vo, &sm);
    if (threadIdx.x == 0 && P.sx) P.sx[m] = s;
}

__global__ void __launch_bounds__(256) unpermute_kernel(const int8_t* __restrict__ qx, int K, int Kp, int blocked,
                                                        int8_t* __restrict__ q) {
    const int m = blockIdx.y;
    const int k = blockIdx.x * blockDim.x + threadIdx.x;
    if (k >= K) return;
    const int g = k >> 4, e = k & 15;  // element e of group g sits at byte 4*(e%4) + e/4
    const size_t group = blocked ? ((size_t)(m >> 4) * (Kp >> 6) + (g >> 2)) * 1024 + ((m & 15) + 16 * (g & 3)) * 16
                                 : (size_t)m * Kp + g * 16;
    q[(size_t)m * K + k] = qx[group + 4 * (e & 3) + (e >> 2)];
}

hipError_t launch_unpermute(const int8_t* qx, int M, int K, int Kp, bool blocked, int8_t* q, hipStream_t s) {
    hipLaunchKernelGGL(unpermute_kernel, dim3((unsigned)((K + 255) / 256), (unsigned)M), dim3(256), 0, s, qx, K, Kp,
                       (int)blocked, q);
    return hipGetLastError();
}

hipError_t launch_quant(const QuantArgs& a, hipStream_t s) {
    if (a.U <= 0 || a.Mpad <= 0) return hipSuccess;
    hipLaunchKernelGGL(quant_kernel, dim3((unsigned)a.Mpad, (unsigned)a.U), dim3(256), 0, s, a);
    return hipGetLastError();
}

}  // namespace rt
