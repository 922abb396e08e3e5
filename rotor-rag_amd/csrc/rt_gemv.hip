// Decode GEMV / skinny GEMM for the ternary linear, M = 1..8 tokens per workgroup,
// no MFMA.  Replaces the reference's thread-per-row OpenCL kernel
// (src/rotor/gpu_ternary.py:12-45, launched per token at src/rotor/transformer.py:134-143)
// and its CPU twin np.dot(x, W_i8.T) * scale (src/rotor/transformer.py:150).
//
// Mapping (lane-per-row, wave-per-row-tile):
//   * a workgroup owns one 64-row block of one problem and `nw` waves split its
//     K chunks; lane r of every wave accumulates row 64*rb + r, so no cross-lane
//     reduction is needed, only a cross-wave one through LDS when nw > 1;
//   * each chunk step is one coalesced 16-byte-per-lane (1 KiB per wave)
//     non-temporal load of rotor bytes;
//   * the activations of a chunk are the same for all 64 lanes, so they are read
//     with scalar loads into SGPRs and fed to v_dot4_i32_i8 as the scalar operand.
//
// Decoding the rotor code (value = bit0 - bit1, field f = 2*bit0 + bit1) costs
// 9 VALU ops per 16 weights: for a weight dword u
//     t0 = u & 0x03030303          -> fields of element 0 of each byte (values 0..3)
//     t1 = u & 0x0C0C0C0C          -> fields of element 1 (values 0,4,8,12)
//     h  = u >> 4, t2 = h & 0x03030303, t3 = h & 0x0C0C0C0C
// and one v_perm_b32 per t turns the four selector bytes into four int8 weights.
// v_perm_b32 byte select: 0..3 pick src1 bytes, 4..7 src0 bytes, 8 replicates bit 7
// of src1 byte 1, 12 gives 0x00.  With src1 = 0x0001FF00 and src0 = 0x00000001:
//     t0: sel 0,1,2,3  -> 00, FF, 01, 00  =  w  for f = 00, 01, 10, 11
//     t1: sel 0,4,8,12 -> 00, 01, FF, 00  = -w  for f = 00, 01, 10, 11
// so element positions 0/2 accumulate into accP and 1/3 into accN, acc = accP - accN.
#include "rt_internal.h"

namespace rt {

constexpr unsigned kLutLo = 0x0001FF00u;  // src1 of v_perm_b32
constexpr unsigned kLutHi = 0x00000001u;  // src0 of v_perm_b32

// Address-space views: weights are global memory; the activations are read-only for
// the whole launch, so the constant address space lets uniform reads become s_load.
typedef __attribute__((address_space(1))) const v4u gv4u;
typedef __attribute__((address_space(4))) const int cint;

__device__ __forceinline__ GemvProb select_prob(const GemvArgs& a, int wg) {
    if (a.dev) {  // binary search over wg_begin (uniform, scalar loads)
        int lo = 0, hi = a.G - 1;
        while (lo < hi) {
            const int mid = (lo + hi + 1) >> 1;
            if (a.dev[mid].wg_begin <= wg) lo = mid; else hi = mid - 1;
        }
        return a.dev[lo];
    }
    GemvProb p = a.p[0];
#pragma unroll
    for (int j = 1; j < kMaxInline; ++j)
        if (j < a.G && a.p[j].wg_begin <= wg) p = a.p[j];
    return p;
}

template <int MT>
__device__ __forceinline__ void chunk_step(const v4u v, cint* __restrict__ xc, const int ldx,
                                           int (&accP)[MT], int (&accN)[MT]) {
    int d[16];
#pragma unroll
    for (int j = 0; j < 4; ++j) {
        const unsigned u = v[j];
        const unsigned h = u >> 4;
        d[4 * j + 0] = (int)__builtin_amdgcn_perm(kLutHi, kLutLo, u & 0x03030303u);
        d[4 * j + 1] = (int)__builtin_amdgcn_perm(kLutHi, kLutLo, u & 0x0C0C0C0Cu);
        d[4 * j + 2] = (int)__builtin_amdgcn_perm(kLutHi, kLutLo, h & 0x03030303u);
        d[4 * j + 3] = (int)__builtin_amdgcn_perm(kLutHi, kLutLo, h & 0x0C0C0C0Cu);
    }
#pragma unroll
    for (int m = 0; m < MT; ++m) {
        cint* __restrict__ xm = xc + m * ldx;
#pragma unroll
        for (int j = 0; j < 4; ++j) {
            accP[m] = __builtin_amdgcn_sdot4(d[4 * j + 0], xm[4 * j + 0], accP[m], false);
            accN[m] = __builtin_amdgcn_sdot4(d[4 * j + 1], xm[4 * j + 1], accN[m], false);
            accP[m] = __builtin_amdgcn_sdot4(d[4 * j + 2], xm[4 * j + 2], accP[m], false);
            accN[m] = __builtin_amdgcn_sdot4(d[4 * j + 3], xm[4 * j + 3], accN[m], false);
        }
    }
}

template <int MT>
__device__ __forceinline__ void gemv_body(gv4u* __restrict__ wp, cint* __restrict__ xq, const int ldx,
                                          const int cb, const int ce, int (&accP)[MT], int (&accN)[MT]) {
    constexpr int U = 4;  // chunks in flight per wave per batch
    int c = cb;
    for (; c + U <= ce; c += U) {
        v4u v[U];
#pragma unroll
        for (int i = 0; i < U; ++i) v[i] = __builtin_nontemporal_load(wp + (size_t)(c + i) * kRowBlock);
#pragma unroll
        for (int i = 0; i < U; ++i) chunk_step<MT>(v[i], xq + (c + i) * 16, ldx, accP, accN);
    }
    for (; c < ce; ++c) {
        const v4u v = __builtin_nontemporal_load(wp + (size_t)c * kRowBlock);
        chunk_step<MT>(v, xq + c * 16, ldx, accP, accN);
    }
}

template <int MT>
__global__ void __launch_bounds__(1024) gemv_kernel(GemvArgs a) {
    extern __shared__ int red[];  // [nw][MT][64] when nw > 1
    const GemvProb P = select_prob(a, blockIdx.x);
    const int rb = blockIdx.x - P.wg_begin;
    const int m0 = blockIdx.y * MT;
    const int lane = threadIdx.x & 63, nw = blockDim.x >> 6;
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);  // wave-uniform
    const int C = P.C;
    const int cb = (wave * C) / nw, ce = ((wave + 1) * C) / nw;
    const int ldx = C * 16;  // dwords per qx row
    gv4u* wp = (gv4u*)(P.w + (size_t)rb * C * kRowBlock) + lane;
    cint* xq = (cint*)(reinterpret_cast<const int*>(P.qx) + (size_t)m0 * ldx);

    int accP[MT], accN[MT];
#pragma unroll
    for (int m = 0; m < MT; ++m) accP[m] = accN[m] = 0;
    gemv_body<MT>(wp, xq, ldx, cb, ce, accP, accN);

    const int M = a.M;
    auto emit = [&](int m, int r, int acc) {
        const int n = rb * kRowBlock + r, mg = m0 + m;
        if (n >= P.N || mg >= M) return;
        if (a.out_i32) {
            static_cast<int*>(P.out)[(size_t)mg * P.ldo + n] = acc;
        } else {
            const float sw = P.rs ? P.rs[n] : P.s_w;
            static_cast<float*>(P.out)[(size_t)mg * P.ldo + n] = ((float)acc * P.sx[mg]) * sw;
        }
    };
    if (nw == 1) {
#pragma unroll
        for (int m = 0; m < MT; ++m) emit(m, lane, accP[m] - accN[m]);
        return;
    }
#pragma unroll
    for (int m = 0; m < MT; ++m) red[(wave * MT + m) * kRowBlock + lane] = accP[m] - accN[m];
    __syncthreads();
    for (int idx = threadIdx.x; idx < MT * kRowBlock; idx += blockDim.x) {
        const int m = idx / kRowBlock, r = idx % kRowBlock;
        int s = 0;
        for (int w = 0; w < nw; ++w) s += red[(w * MT + m) * kRowBlock + r];
        emit(m, r, s);
    }
}

int gemv_waves(int total_wgs, int C) {
    // Aim for ~8 waves per CU on 256 CUs; every wave keeps >= 2 chunks.
    int nw = (2048 + total_wgs - 1) / total_wgs;
    if (nw > 16) nw = 16;
    if (nw > C / 2) nw = C / 2;
    if (nw < 1) nw = 1;
    return nw;
}

hipError_t launch_gemv(const GemvArgs& a, int total_wgs, int mt, int nw, hipStream_t s) {
    if (total_wgs <= 0 || a.M <= 0) return hipSuccess;
    const dim3 grid((unsigned)total_wgs, (unsigned)((a.M + mt - 1) / mt));
    const dim3 block((unsigned)(64 * nw));
    const size_t lds = nw > 1 ? (size_t)nw * mt * kRowBlock * sizeof(int) : 0;
    switch (mt) {
        case 1: hipLaunchKernelGGL(gemv_kernel<1>, grid, block, lds, s, a); break;
        case 2: hipLaunchKernelGGL(gemv_kernel<2>, grid, block, lds, s, a); break;
        case 4: hipLaunchKernelGGL(gemv_kernel<4>, grid, block, lds, s, a); break;
        case 8: hipLaunchKernelGGL(gemv_kernel<8>, grid, block, lds, s, a); break;
        default: return hipErrorInvalidValue;
    }
    return hipGetLastError();
}

}  // namespace rt
