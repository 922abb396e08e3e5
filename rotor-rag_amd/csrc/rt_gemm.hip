// Prefill / batched ternary GEMM on the int8 matrix cores (gfx950 MFMA):
// C[M,N] = A[M,K] x W[N,K]^T with A the per-token quantised activations (qx layout)
// and W the rotor weight tiles, int32 accumulation, fp32 rescale epilogue.
// Replaces, for M >= 16 tokens, the reference's per-token loop
// (src/rotor/transformer.py:134-143) and its CPU sgemm (src/rotor/transformer.py:150).
//
// Workgroup tile BM x 128 x (K step 64), 4 waves in a 2 x 2 arrangement, each wave
// (BM/2) x 64 of v_mfma_i32_16x16x64_i8.  Per K step:
//   * A: BM rows x 64 int8 of qx go global -> registers -> LDS;
//   * W: the two 64-row blocks of the tile are one coalesced 1 KiB chunk each; 128
//     threads decode one 16-byte chunk (64 weights) each to int8 and store them to LDS
//     in the same permuted k order as qx (so operand bytes pair up one to one);
//   * the next step's global loads are issued before this step's MFMAs.
// The MFMA consumes, per lane, 16 bytes of one A row and 16 bytes of one W row at the
// same k positions, so any consistent assignment of k to (lane group, byte) gives the
// exact sum; the result layout used is D[4*(lane/16) + i][lane % 16], i = 0..3.
#include "rt_internal.h"

namespace rt {

typedef int v4i __attribute__((ext_vector_type(4)));

constexpr unsigned kLut = 0x0001FF00u;  // v_perm_b32 src1: field 0,1,2,3 -> 00, FF, 01, 00
constexpr int kBN = 128;
constexpr int kLdsRow = 80;             // 64 bytes + 16 pad per LDS row (bank spread)

// 16 weight bytes (64 rotor codes) -> 64 int8 weights in qx order: dword j of the
// source gives output dwords 4j..4j+3 = elements {16j+4b+i : b=0..3}, i = 0..3.
__device__ __forceinline__ void decode_chunk(const v4u v, v4u (&o)[4]) {
#pragma unroll
    for (int j = 0; j < 4; ++j) {
        const unsigned u = v[j];
        o[j][0] = __builtin_amdgcn_perm(0u, kLut, u & 0x03030303u);
        o[j][1] = __builtin_amdgcn_perm(0u, kLut, (u >> 2) & 0x03030303u);
        o[j][2] = __builtin_amdgcn_perm(0u, kLut, (u >> 4) & 0x03030303u);
        o[j][3] = __builtin_amdgcn_perm(0u, kLut, (u >> 6) & 0x03030303u);
    }
}

template <int BM>
__global__ void __launch_bounds__(256) gemm_kernel(GemmArgs a) {
    constexpr int WM = BM / 2;          // rows per wave
    constexpr int FI = WM / 16;         // A fragments per wave
    constexpr int FJ = 4;               // W fragments per wave (64 columns)
    constexpr int AL = BM * 4 / 256;    // 16-byte A loads per thread per step
    __shared__ __attribute__((aligned(16))) int8_t As[BM * kLdsRow];
    __shared__ __attribute__((aligned(16))) int8_t Bs[kBN * kLdsRow];

    const int t = threadIdx.x, lane = t & 63;
    const int wave = __builtin_amdgcn_readfirstlane(t >> 6);
    const int wm = wave >> 1, wn = wave & 1;
    const int n0 = blockIdx.x * kBN, m0 = blockIdx.y * BM;
    const int C = a.C, Kp = C * 64, Nb = a.Np / kRowBlock;

    // global sources of this thread
    const v4u* a_src[AL];  // qx rows are 16-byte aligned (Kp is a multiple of 64)
#pragma unroll
    for (int i = 0; i < AL; ++i) {
        const int idx = t + i * 256, row = idx >> 2, seg = idx & 3;
        a_src[i] = reinterpret_cast<const v4u*>(a.qx) + ((size_t)(m0 + row) * Kp >> 4) + seg;
    }
    const int w_rb = n0 / kRowBlock + (t >> 6);  // threads 0..127: row block of the tile
    const bool w_ok = t < 128 && w_rb < Nb;
    const v4u* w_src = a.w + (size_t)w_rb * C * kRowBlock + (t & 63);

    v4u ra[AL], rw = {0u, 0u, 0u, 0u};
    auto gload = [&](int c) {
#pragma unroll
        for (int i = 0; i < AL; ++i) ra[i] = a_src[i][c * 4];
        if (w_ok) rw = __builtin_nontemporal_load(w_src + (size_t)c * kRowBlock);
    };

    v4i acc[FI][FJ];
#pragma unroll
    for (int i = 0; i < FI; ++i)
#pragma unroll
        for (int j = 0; j < FJ; ++j) acc[i][j] = v4i{0, 0, 0, 0};

    gload(0);
    for (int c = 0; c < C; ++c) {
        __syncthreads();  // previous step's fragments are consumed
#pragma unroll
        for (int i = 0; i < AL; ++i) {
            const int idx = t + i * 256, row = idx >> 2, seg = idx & 3;
            *reinterpret_cast<v4u*>(As + row * kLdsRow + seg * 16) = ra[i];
        }
        if (t < 128) {
            v4u o[4];
            decode_chunk(rw, o);
#pragma unroll
            for (int j = 0; j < 4; ++j) *reinterpret_cast<v4u*>(Bs + t * kLdsRow + j * 16) = o[j];
        }
        __syncthreads();
        if (c + 1 < C) gload(c + 1);  // in flight during the MFMAs

        const int kseg = (lane >> 4) * 16, r16 = lane & 15;
        v4i fa[FI], fb[FJ];
#pragma unroll
        for (int i = 0; i < FI; ++i)
            fa[i] = *reinterpret_cast<const v4i*>(As + (wm * WM + i * 16 + r16) * kLdsRow + kseg);
#pragma unroll
        for (int j = 0; j < FJ; ++j)
            fb[j] = *reinterpret_cast<const v4i*>(Bs + (wn * 64 + j * 16 + r16) * kLdsRow + kseg);
#pragma unroll
        for (int i = 0; i < FI; ++i)
#pragma unroll
            for (int j = 0; j < FJ; ++j)
                acc[i][j] = __builtin_amdgcn_mfma_i32_16x16x64_i8(fa[i], fb[j], acc[i][j], 0, 0, 0);
    }

    // epilogue: D[4*(lane/16) + r][lane % 16] of every 16x16 fragment
#pragma unroll
    for (int i = 0; i < FI; ++i)
#pragma unroll
        for (int j = 0; j < FJ; ++j)
#pragma unroll
            for (int r = 0; r < 4; ++r) {
                const int m = m0 + wm * WM + i * 16 + 4 * (lane >> 4) + r;
                const int n = n0 + wn * 64 + j * 16 + (lane & 15);
                if (m >= a.M || n >= a.N) continue;
                const int v = acc[i][j][r];
                if (a.out_i32) {
                    static_cast<int*>(a.out)[(size_t)m * a.ldo + n] = v;
                } else {
                    const float sw = a.rs ? a.rs[n] : a.s_w;
                    const size_t o = (size_t)m * a.ldo + n;
                    const float y = ((float)v * a.sx[m]) * sw;
                    static_cast<float*>(a.out)[o] = a.res ? a.res[o] + y : y;
                }
            }
}

hipError_t launch_gemm(const GemmArgs& a, hipStream_t s) {
    if (a.M <= 0 || a.N <= 0) return hipSuccess;
    const int bm = gemm_bm(a.M);
    const dim3 grid((unsigned)((a.N + kBN - 1) / kBN), (unsigned)((a.M + bm - 1) / bm));
    if (bm == 64) hipLaunchKernelGGL(gemm_kernel<64>, grid, dim3(256), 0, s, a);
    else hipLaunchKernelGGL(gemm_kernel<128>, grid, dim3(256), 0, s, a);
    return hipGetLastError();
}

}  // namespace rt
