// Weight relayout: rotor bytes [N][ceil(K/4)] <-> gfx950 weight tiles.
//
// Element j of a byte stays in bits (2j+1, 2j) (src/rotor/core.py:99-108); the 16-byte
// chunks move to the tile placement and each 2-bit rotor code (bit0, bit1) becomes the
// device code g = w + 1 (rt_internal.h: device_code / rotor_code).  This replaces the
// reference's per-weight Python packing loop (src/rotor/gpu_ternary.py:112-136) and its
// C conversion loop (native/c/rotor_core.c:202-260): one thread per 16-byte unit.
#include "rt_internal.h"

namespace rt {

// Bytes of row n, byte columns [b0, b0+16), in device code; codes of k >= K and rows
// n >= N are weight 0.
__device__ __forceinline__ v4u gather_row_bytes(const uint8_t* __restrict__ src, int N, int K, int n, int b0) {
    const int kb = (K + 3) >> 2;
    unsigned wd[4] = {0u, 0u, 0u, 0u};
    if (n < N) {
        const uint8_t* row = src + (size_t)n * kb;
#pragma unroll
        for (int i = 0; i < 16; ++i) {
            const int b = b0 + i;
            unsigned byte = 0u;
            if (b < kb) {
                byte = row[b];
                const int valid = K - 4 * b;  // elements of this byte that exist
                if (valid < 4) byte &= (1u << (2 * valid)) - 1u;
            }
            wd[i >> 2] |= byte << (8 * (i & 3));
        }
    }
    v4u v = {device_code(wd[0]), device_code(wd[1]), device_code(wd[2]), device_code(wd[3])};
    return v;
}

__global__ void __launch_bounds__(256) relayout_kernel(const uint8_t* __restrict__ src, int N, int K, int C,
                                                       long long units, v4u* __restrict__ tiles) {
    const long long u = (long long)blockIdx.x * blockDim.x + threadIdx.x;
    if (u >= units) return;
    const int r = (int)(u % kRowBlock);
    const long long t = u / kRowBlock;
    const int c = (int)(t % C);
    const int rb = (int)(t / C);
    tiles[u] = gather_row_bytes(src, N, K, rb * kRowBlock + r, c * 16);
}

__global__ void __launch_bounds__(256) unrelayout_kernel(const v4u* __restrict__ tiles, int N, int K, int C,
                                                         long long total_bytes, uint8_t* __restrict__ dst) {
    const long long i = (long long)blockIdx.x * blockDim.x + threadIdx.x;
    if (i >= total_bytes) return;
    const int kb = (K + 3) >> 2;
    const int n = (int)(i / kb), b = (int)(i % kb);
    const int rb = n / kRowBlock, r = n % kRowBlock, c = b / 16, j = b % 16;
    const v4u v = tiles[((size_t)rb * C + c) * kRowBlock + r];
    const unsigned wd = rotor_code(v[j >> 2]);
    dst[i] = (uint8_t)(wd >> (8 * (j & 3)));
}

hipError_t launch_relayout(const uint8_t* src, int N, int K, v4u* tiles, hipStream_t s) {
    const int C = round_up(K, kChunk) / kChunk;
    const long long units = (long long)round_up(N, kRowBlock) * C;
    const long long blocks = (units + 255) / 256;
    hipLaunchKernelGGL(relayout_kernel, dim3((unsigned)blocks), dim3(256), 0, s, src, N, K, C, units, tiles);
    return hipGetLastError();
}

hipError_t launch_unrelayout(const v4u* tiles, int N, int K, uint8_t* dst, hipStream_t s) {
    const int C = round_up(K, kChunk) / kChunk;
    const long long total = (long long)N * ((K + 3) / 4);
    const long long blocks = (total + 255) / 256;
    if (total == 0) return hipSuccess;
    hipLaunchKernelGGL(unrelayout_kernel, dim3((unsigned)blocks), dim3(256), 0, s, tiles, N, K, C, total, dst);
    return hipGetLastError();
}

}  // namespace rt
