// Per-token absmax int8 activation quantiser, optionally fused with the operation
// that produces the activations (RMSNorm, relu^2(gate)*up, relu^2(gate)*up followed by
// the FFN sub-norm), and the int8 permute used by the int32 parity entry point.
// The row arithmetic lives in rt_rowquant.h (shared with the decode GEMV prologue).
//
// One 256-thread workgroup per token row; rows in [M, Mpad) are zero-filled.
#include <algorithm>

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

// Rows with K % 64 == 0 and no natural-order / value outputs: K / E threads per row, E
// (4 or 8) consecutive elements each (the decode prologue's row path), the int8 row
// assembled in LDS and copied out 16 bytes per thread.
template <int E>
__global__ void __launch_bounds__(1024) quant_rows_kernel(QuantArgs a) {
    extern __shared__ __attribute__((aligned(16))) v4u qrow_lds[];
    RowSmem* sm = reinterpret_cast<RowSmem*>(qrow_lds + 512);  // rows of up to 8192 bytes
    const QuantProb P = select_quant(a, blockIdx.y);
    const int m = blockIdx.x;
    const int Kp = P.Kp, groups = Kp >> 4;
    v4u* const qx = reinterpret_cast<v4u*>(P.qx);
    const QxRow qrow = P.blocked ? QxRow{qx + (size_t)(m >> 4) * (Kp >> 6) * 64 + (m & 15), 64, 16}
                                 : QxRow{qx + (size_t)m * (Kp >> 4), 4, 1};
    if (m >= a.M) {  // padding token rows
        const v4u z = {0u, 0u, 0u, 0u};
        for (int g = threadIdx.x; g < groups; g += blockDim.x) qrow[g] = z;
        if (threadIdx.x == 0 && P.sx) P.sx[m] = 0.0f;
        return;
    }
    QuantProb R = P;  // row m of the sources
    R.x = P.x + (size_t)m * P.K;
    if (has_relu2(P)) R.aux = P.aux + (size_t)m * P.K;
    RowRegsE<E> rr;
    row_loadE<E>(R, rr);
    const float s = row_finishE<E>(R, rr, qrow_lds, sm);
    __syncthreads();
    for (int g = threadIdx.x; g < groups; g += blockDim.x) qrow[g] = qrow_lds[g];
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

// The vectorised row path applies when every problem has K % 64 == 0, K <= 8192, 16-byte
// aligned sources, a row mode (no kPermute / kAttnNorm) and no extra outputs; the host
// checks the single problem it knows of (a.dev == nullptr) or the plan's summary.
static bool aligned16q(const void* p) { return ((uintptr_t)p & 15u) == 0; }

bool quant_rows_ok(const QuantProb& P) {
    return P.mode != kPermute && P.mode != kAttnNorm && !P.q_nat && !P.v_out && P.K % 64 == 0 && P.K <= 8192 &&
           aligned16q(P.x) && aligned16q(P.aux) && aligned16q(P.aux2);
}

hipError_t launch_quant(const QuantArgs& a, hipStream_t s, int maxK) {
    if (a.U <= 0 || a.Mpad <= 0) return hipSuccess;
    if (maxK > 0) {  // every problem passed quant_rows_ok; maxK: the largest K
        const dim3 grid((unsigned)a.Mpad, (unsigned)a.U);
        const size_t lds = 8192 + sizeof(RowSmem);
        // whole waves (the workgroup reductions take one slot per wave); 8 or 16 elements per
        // thread: fewer waves in the row's two reductions (512-token prefill 4.70 -> 4.59 ms
        // against 4 and 8)
        if (maxK <= 4096) {
            hipLaunchKernelGGL((quant_rows_kernel<8>), grid, dim3((unsigned)((maxK / 8 + 63) / 64 * 64)), lds, s, a);
        } else {
            hipLaunchKernelGGL((quant_rows_kernel<16>), grid, dim3((unsigned)((maxK / 16 + 63) / 64 * 64)), lds, s, a);
        }
        return hipGetLastError();
    }
    hipLaunchKernelGGL(quant_kernel, dim3((unsigned)a.Mpad, (unsigned)a.U), dim3(256), 0, s, a);
    return hipGetLastError();
}

}  // namespace rt
