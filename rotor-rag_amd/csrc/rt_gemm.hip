// Prefill / batched ternary GEMM on the int8 matrix cores (gfx950 MFMA):
// C[M,N] = A[M,K] x W[N,K]^T with A the per-token quantised activations (qx layout)
// and W the rotor weight tiles, int32 accumulation, fp32 rescale epilogue.
// Replaces, for M > 8 tokens, the reference's per-token loop
// (src/rotor/transformer.py:134-143) and its CPU sgemm (src/rotor/transformer.py:150).
//
// Workgroup: 4 waves (WAVES_M x WAVES_N), tile BM x BN, K step 64 (one weight chunk) =
// two k-slices of v_mfma_i32_32x32x32_i8 (this shape runs at full rate from one wave
// per SIMD, which the large tiles here need: 256 accumulator registers per lane).
//   * Operands reach LDS by direct global->LDS loads (global_load_lds_dwordx4) into a
//     ring of STAGES stages, STAGES steps ahead.  A barrier per step publishes the next
//     stage (each wave first waits for its own loads of it: s_waitcnt vmcnt) and retires
//     the stage just read, which the next loads then refill.
//   * A (blocked qx layout) is stored as 1 KiB 16-row x 64-k blocks in operand order
//     (lane l: row l % 16, bytes 16 (l / 16) .. +15): one load copies a block to LDS with
//     contiguous 16-byte lanes.  The MFMA lane l wants
//     row l % 32, bytes 32 h + 16 (l / 32) .. +15 of slice h: one ds_read_b128, every
//     group of 8 lanes reading 128 contiguous bytes (conflict-free).
//   * W stays 2-bit in LDS (a 64-row block's chunk is 1 KiB, copied as is; device code
//     g = w + 1, rt_internal.h).  The 16
//     weights an MFMA lane needs are one dword of its row's 16-byte unit: ds_read_b32
//     and four v_perm_b32 expand it to int8 in the qx order.
//   * Software pipeline per step c: MFMAs of slice 0; barrier; loads of step
//     c + STAGES; fragment reads of step c + 1; MFMAs of slice 1 (hiding the reads);
//     weight expansion of step c + 1.
//   * Tiles are ordered m-major and dealt to the 8 XCDs in contiguous ranges
//     (workgroup i runs on XCD i % 8), so the workgroups sharing an A row tile share an
//     L2.
// Both operands assign k to (lane group, byte) the same way, so the int32 sums are exact
// whatever that assignment is; the result layout of a 32x32 block is
// D[8 (k / 4) + 4 (lane / 32) + k % 4][lane % 32], k = 0..15.
#include <type_traits>

#include "rt_internal.h"

// the epilogue rounds ((float)acc * sx) * sw, then adds the residual, as separate IEEE ops
#pragma clang fp contract(off)

namespace rt {

typedef int v4i __attribute__((ext_vector_type(4)));
typedef int v16i __attribute__((ext_vector_type(16)));
typedef float v4f __attribute__((ext_vector_type(4)));
typedef __attribute__((address_space(3))) void lds_void;

constexpr unsigned kLut = 0x000100FFu;  // v_perm_b32 src1: device code 0,1,2,(3) -> FF, 00, 01, 00

// one dword of device code (16 weights, byte b holds elements 4b..4b+3 at bits 2i) -> 16
// int8 weights in the qx order of a 16-group: output byte 4i + b = element 4b + i
__device__ __forceinline__ v4i decode_dword(unsigned u) {
    v4i o;
    o[0] = (int)__builtin_amdgcn_perm(0u, kLut, u & 0x03030303u);
    o[1] = (int)__builtin_amdgcn_perm(0u, kLut, (u >> 2) & 0x03030303u);
    o[2] = (int)__builtin_amdgcn_perm(0u, kLut, (u >> 4) & 0x03030303u);
    o[3] = (int)__builtin_amdgcn_perm(0u, kLut, (u >> 6) & 0x03030303u);
    return o;
}

// 16 bytes per lane from global memory straight into LDS: lane l's bytes land at
// lds + 16 l (lds wave-uniform)
__device__ __forceinline__ void load_lds16(const void* g, void* lds) {
    __builtin_amdgcn_global_load_lds(g, (lds_void*)lds, 16, 0, 0);
}

// Wait until at most N of this wave's vector-memory loads are outstanding and all of
// its LDS reads have returned, then barrier.  The scheduler moves nothing across.
template <int N>
__device__ __forceinline__ void wait_barrier() {
    __builtin_amdgcn_sched_barrier(0);
    asm volatile("s_waitcnt vmcnt(%0) lgkmcnt(0)\n\ts_barrier" ::"n"(N) : "memory");
    __builtin_amdgcn_sched_barrier(0);
}

// Wait until at most N of this wave's vector-memory loads are outstanding (no barrier).
template <int N>
__device__ __forceinline__ void wait_vm() {
    __builtin_amdgcn_sched_barrier(0);
    asm volatile("s_waitcnt vmcnt(%0)" ::"n"(N) : "memory");
    __builtin_amdgcn_sched_barrier(0);
}

template <int BM, int BN, int WAVES_M, int STAGES>
struct GemmTile {
    static constexpr int WAVES_N = 4 / WAVES_M;
    static constexpr int WM = BM / WAVES_M, WN = BN / WAVES_N;
    static constexpr int FI = WM / 32, FJ = WN / 32;  // 32 x 32 blocks per wave
    static constexpr int LA = BM / 64;                // A loads (16-row blocks) per wave per step
    static constexpr int RB = BN / kRowBlock;         // weight row blocks per tile
    // W region: one 1 KiB slot per wave (waves past the tile's row blocks fill a spare
    // slot, so every wave issues the same loads per step)
    static constexpr int A_BYTES = BM * 64, STAGE_BYTES = A_BYTES + 4 * 1024;
    static constexpr int SX_OFF = STAGES * STAGE_BYTES;  // BM row scales after the ring
    static constexpr int LDS_BYTES = SX_OFF + BM * 4;
    static_assert(WAVES_M * WAVES_N == 4 && FI >= 1 && FJ >= 1 && LA >= 1 && RB >= 1 && RB <= 4, "tile shape");
    static_assert(STAGES >= 2, "ring depth");
};

// Writes a wave's FI x FJ blocks.  EPI 0: int32 accumulators; 1: fp32
// acc * sx[m] * s_w; 2: as 1 plus the residual.  Output (and residual) rows are raw
// buffers from the tile's first row m0 to row min(m0 + BM, M): rows past M fall outside
// the range and the hardware drops those stores; a column past N adds bit 31 to the
// offset (row and column terms stay below 2^31), which puts it outside as well.
// mrow: this lane's first row relative to m0 (includes 4 (lane / 32)); nb: first column.
template <int FI, int FJ, int EPI>
__device__ __forceinline__ void store_tile(const v16i (&acc)[FI][FJ], const GemmArgs& a, int m0, int rows, int mrow,
                                           int nb, const float* sx_lds, const float (&swv)[FJ]) {
    const unsigned range = (unsigned)rows * (unsigned)a.ldo * 4u;
    const __amdgpu_buffer_rsrc_t out =
        __builtin_amdgcn_make_buffer_rsrc(static_cast<char*>(a.out) + (size_t)m0 * a.ldo * 4, 0, range, kBufDword3);
    const __amdgpu_buffer_rsrc_t res = __builtin_amdgcn_make_buffer_rsrc(
        (void*)(a.res ? a.res + (size_t)m0 * a.ldo : nullptr), 0, EPI == 2 ? range : 0u, kBufDword3);
    int coff[FJ];
#pragma unroll
    for (int j = 0; j < FJ; ++j) {
        const int n = nb + j * 32;
        coff[j] = (int)((unsigned)n * 4u + ((unsigned)(n >= a.N) << 31));
    }
    const int row_bytes = a.ldo * 4;
#pragma unroll
    for (int i = 0; i < FI; ++i) {
        float sxv[16];
        if (EPI) {
#pragma unroll
            for (int q = 0; q < 4; ++q) {  // rows mrow + 32 i + 8 q + 0..3
                const v4f s4 = *reinterpret_cast<const v4f*>(sx_lds + mrow + i * 32 + q * 8);
#pragma unroll
                for (int r = 0; r < 4; ++r) sxv[q * 4 + r] = s4[r];
            }
        }
#pragma unroll
        for (int j = 0; j < FJ; ++j) {
            int off[16];
            float rv[16];
#pragma unroll
            for (int k = 0; k < 16; ++k) {
                off[k] = (mrow + i * 32 + 8 * (k >> 2) + (k & 3)) * row_bytes + coff[j];
                if (EPI == 2) rv[k] = __builtin_bit_cast(float, __builtin_amdgcn_raw_buffer_load_b32(res, off[k], 0, 0));
            }
#pragma unroll
            for (int k = 0; k < 16; ++k) {
                unsigned bits;
                if (EPI == 0) {
                    bits = (unsigned)acc[i][j][k];
                } else {
                    const float y = ((float)acc[i][j][k] * sxv[k]) * swv[j];
                    bits = __builtin_bit_cast(unsigned, EPI == 2 ? rv[k] + y : y);
                }
                __builtin_amdgcn_raw_buffer_store_b32(bits, out, off[k], 0, 0);
            }
        }
    }
}

// The gate/up pair's epilogue (GemmArgs::pair_a): the wave's column blocks 2 jp and 2 jp + 1
// are the gate and up rows of the same 32 outputs (their 64-column group starts at a multiple
// of 64), so lane l forms a = relu(g)^2 * u of output 32 (n / 64) + l % 32 for its 16 rows,
// g and u rounded as store_tile's fp32 epilogue rounds y, a in the order of the quantiser's
// relu^2 * up.  Rows and columns past the problem fall outside the buffer (as store_tile).
template <int FI, int FJ>
__device__ __forceinline__ void store_tile_pair(const v16i (&acc)[FI][FJ], const GemmArgs& a, int m0, int rows,
                                                int mrow, int nb, const float* sx_lds) {
    static_assert(FJ % 2 == 0, "gate and up blocks in pairs");
    const unsigned range = (unsigned)rows * (unsigned)a.ldo * 4u;
    const __amdgpu_buffer_rsrc_t out =
        __builtin_amdgcn_make_buffer_rsrc(a.pair_a + (size_t)m0 * a.ldo, 0, range, kBufDword3);
    int coff[FJ / 2];
#pragma unroll
    for (int jp = 0; jp < FJ / 2; ++jp) {
        const int n = nb + jp * 64, no = 32 * (n >> 6) + (n & 31);  // gate column, output column
        coff[jp] = (int)((unsigned)no * 4u + ((unsigned)(n >= a.N) << 31));
    }
    const int row_bytes = a.ldo * 4;
#pragma unroll
    for (int i = 0; i < FI; ++i) {
        float sxv[16];
#pragma unroll
        for (int q = 0; q < 4; ++q) {  // rows mrow + 32 i + 8 q + 0..3
            const v4f s4 = *reinterpret_cast<const v4f*>(sx_lds + mrow + i * 32 + q * 8);
#pragma unroll
            for (int r = 0; r < 4; ++r) sxv[q * 4 + r] = s4[r];
        }
#pragma unroll
        for (int jp = 0; jp < FJ / 2; ++jp)
#pragma unroll
            for (int k = 0; k < 16; ++k) {
                const int off = (mrow + i * 32 + 8 * (k >> 2) + (k & 3)) * row_bytes + coff[jp];
                const float g = ((float)acc[i][2 * jp][k] * sxv[k]) * a.pair_sg;
                const float u = ((float)acc[i][2 * jp + 1][k] * sxv[k]) * a.pair_su;
                const float av = g > 0.0f ? (g * g) * u : 0.0f;
                __builtin_amdgcn_raw_buffer_store_b32(__builtin_bit_cast(unsigned, av), out, off, 0, 0);
            }
    }
}

// One problem, or a group of them (dev != nullptr): unit b (a row block of the split-K
// kernel, a tile of the tile kernel) serves problem rb2p[b], whose units start at its
// wg_begin.
struct GemmGroupArgs {
    const GemmArgs* dev;
    const int* rb2p;
    GemmArgs one;
    // nb >= 0: descriptor i + 1 starts at unit bnd[i] (i < nb), so a unit finds its descriptor
    // by comparing with these arguments instead of loading rb2p [unit] first; nb < 0: rb2p
    int nb;
    int bnd[kGroupBounds];
};

// Problem of unit b, read through constant-address-space pointers so that it stays
// in scalar registers (see the GEMV's find_prob).
typedef __attribute__((address_space(4))) const GemmArgs cgemm;
typedef __attribute__((address_space(4))) const int cidx_g;
__device__ __forceinline__ GemmArgs find_gemm(const GemmGroupArgs& ga, int b) {
    // the bounds are read before the branch (the empty asm keeps them there), so their loads
    // go out with the first ones
    const int nb = ga.nb;
    int j = 0;
#pragma unroll
    for (int i = 0; i < kGroupBounds; ++i) j += i < nb && b >= ga.bnd[i] ? 1 : 0;
    asm volatile("" ::"s"(j), "s"(nb));
    if (!ga.dev) return ga.one;
    if (nb < 0) j = ((cidx_g*)ga.rb2p)[b];
    const cgemm* q = (cgemm*)ga.dev + j;
    return GemmArgs{q->w,  q->qx,       q->sx, q->rs, q->out, q->s_w, q->M,     q->N,   q->Np,
                    q->C,  q->ldo,      q->out_i32, q->res, q->wg_begin, q->c0, q->c1, q->kp, q->parts,
                    q->cnt, q->part_ws, q->pair_a, q->pair_sg, q->pair_su};
}

template <int BM, int BN, int WAVES_M, int STAGES>
__global__ void __launch_bounds__(256) gemm_kernel(GemmGroupArgs ga) {
    using T = GemmTile<BM, BN, WAVES_M, STAGES>;
    constexpr int FI = T::FI, FJ = T::FJ, LA = T::LA;
    extern __shared__ __attribute__((aligned(16))) v4u lds[];

    const int t = threadIdx.x, lane = t & 63, g = lane >> 5, r32 = lane & 31;
    const int wave = __builtin_amdgcn_readfirstlane(t >> 6);
    const int wm = wave / T::WAVES_N, wn = wave % T::WAVES_N;

    // tile of this workgroup: the tiles of all problems in one order (each problem's
    // m-major), dealt to the XCDs in contiguous ranges; then its problem and local tile
    const int tiles = (int)gridDim.x;
    const int tile = xcd_order((int)blockIdx.x, tiles);
    const GemmArgs a = find_gemm(ga, tile);
    const int C = a.C, Nb = a.Np / kRowBlock;
    const int nT = (a.N + BN - 1) / BN, lt = tile - a.wg_begin;
    const int m0 = (lt / nT) * BM, n0 = (lt % nT) * BN;
    char* const lds_b = reinterpret_cast<char*>(lds);
    float* const sx_lds = reinterpret_cast<float*>(lds_b + T::SX_OFF);

    // Activations hold gemm_bm(M) = 256-row padding (M > 128).  A 192-row tile can end past
    // it: its rows there re-read the last padded row (their outputs fall outside the
    // output buffer range and are dropped).
    constexpr bool kClamp = 256 % BM != 0;
    const int last_row = kClamp ? ((a.M + 255) & ~255) - 1 : 0;
    // row scales of the tile into LDS (sx holds the padded rows), published by the
    // barrier before the epilogue; column scales into registers
    if (!a.out_i32 && t < BM) sx_lds[t] = a.sx[kClamp ? min(m0 + t, last_row) : m0 + t];
    const int mrow = wm * T::WM + 4 * g, nb = n0 + wn * T::WN + r32;
    float swv[FJ];
#pragma unroll
    for (int j = 0; j < FJ; ++j) swv[j] = a.out_i32 ? 0.f : a.rs ? a.rs[min(nb + j * 32, a.N - 1)] : a.s_w;

    // this lane's global sources; the wave's LDS destinations
    const int8_t* a_src[LA];
#pragma unroll
    for (int k = 0; k < LA; ++k) {
        const int f = wave + 4 * k;  // 16-row block f
        const int blk = kClamp ? min((m0 >> 4) + f, last_row >> 4) : (m0 >> 4) + f;
        a_src[k] = a.qx + ((size_t)blk * C) * 1024 + lane * 16;  // blocked qx
    }
    // weight row block of this wave's slot: clamped to a valid block (a wave past the
    // tile's blocks, or past N, loads data nobody reads)
    const int w_rb = min(n0 / kRowBlock + min(wave, T::RB - 1), Nb - 1);
    const v4u* w_src = a.w + (size_t)w_rb * C * kRowBlock + lane;
    constexpr int kLoads = LA + 1;  // loads per wave per step

    auto issue = [&](int c) {
        char* st = lds_b + (c % STAGES) * T::STAGE_BYTES;
#pragma unroll
        for (int k = 0; k < LA; ++k) load_lds16(a_src[k] + (size_t)c * 1024, st + (wave + 4 * k) * 1024);
        load_lds16(w_src + (size_t)c * kRowBlock, st + T::A_BYTES + wave * 1024);
    };

    // per-lane LDS read offsets inside a stage (slice h adds 512 for A, 8 for W)
    const int a_rd = ((wm * T::WM + r32) >> 4) * 1024 + ((r32 & 15) + 16 * g) * 16;
    int w_rd[FJ];
#pragma unroll
    for (int j = 0; j < FJ; ++j) {
        const int n = wn * T::WN + j * 32 + r32;
        w_rd[j] = T::A_BYTES + (n >> 6) * 1024 + (n & 63) * 16 + g * 4;
    }

    // Fragments of two steps (current p, next 1 - p): A per slice and block row, W raw
    // and expanded.  Index [p][h * F + block].
    v4i fa[2][2 * FI], fb[2][2 * FJ];
    unsigned wraw[2][2 * FJ];
    // read item r of step c into set p: W pairs (both slices of block j) first, then A
    auto read_item = [&](int p, int c, int r) {
        const char* st = lds_b + (c % STAGES) * T::STAGE_BYTES;
        if (r < FJ) {
            wraw[p][r] = *reinterpret_cast<const unsigned*>(st + w_rd[r]);
            wraw[p][FJ + r] = *reinterpret_cast<const unsigned*>(st + w_rd[r] + 8);
        } else {
            const int h = (r - FJ) / FI, i = (r - FJ) % FI;
            fa[p][h * FI + i] = *reinterpret_cast<const v4i*>(st + a_rd + i * 2048 + h * 512);
        }
    };
    auto issue_item = [&](int c, int k) {  // load k of step c (A blocks, then W)
        char* st = lds_b + (c % STAGES) * T::STAGE_BYTES;
        if (k < LA) load_lds16(a_src[k] + (size_t)c * 1024, st + (wave + 4 * k) * 1024);
        else load_lds16(w_src + (size_t)c * kRowBlock, st + T::A_BYTES + wave * 1024);
    };

    v16i acc[FI][FJ];
#pragma unroll
    for (int i = 0; i < FI; ++i)
#pragma unroll
        for (int j = 0; j < FJ; ++j) acc[i][j] = v16i{};

    // prologue: fill the ring, publish step 0, read and expand it
    for (int c = 0; c < STAGES && c < C; ++c) issue(c);
    if (C >= STAGES) wait_barrier<(STAGES - 1) * kLoads>();
    else wait_barrier<0>();
#pragma unroll
    for (int r = 0; r < 2 * FI + FJ; ++r) read_item(0, 0, r);
#pragma unroll
    for (int u = 0; u < 2 * FJ; ++u) fb[0][u] = decode_dword(wraw[0][u]);

    // Step c (fragments in set p).  MODE 0 (steady): publish step c + 1 (every wave's
    // reads of step c returned, so step c's stage takes step c + STAGES), read step
    // c + 1, load step c + STAGES, expand step c + 1's weights.  MODE 1 (tail): the same
    // without loads.  MODE 2: last step, MFMAs only.
    // The wave issues in order and an MFMA holds the matrix core 32 cycles, so the
    // other work is dealt out evenly between the step's MFMAs: the LDS reads (weights
    // first), the loads, then the weight expansion one output dword at a time (2-3 VALU
    // ops of 4 cycles).  Fences pin the order; each body is one basic block.
    constexpr int kMfma = 2 * FI * FJ, kReads = 2 * FI + FJ, kQuarters = 8 * FJ;
    auto body = [&](auto P, auto MODE, int c) {
        constexpr int p = decltype(P)::value, mode = decltype(MODE)::value;
        constexpr int nRd = mode == 2 ? 0 : kReads, nLd = mode == 0 ? kLoads : 0, nDec = mode == 2 ? 0 : kQuarters;
        constexpr int nItems = nRd + nLd + nDec;
        if (mode == 0) wait_barrier<(STAGES - 2) * kLoads>();
        if (mode == 1) wait_barrier<0>();
        auto item = [&](int t) {
            if (t < nRd) {
                read_item(1 - p, c + 1, t);
            } else if (t < nRd + nLd) {
                issue_item(c + STAGES, t - nRd);
            } else {
                const int d = t - nRd - nLd, u = d >> 2, q = d & 3;  // dword u, output q
                fb[1 - p][u][q] = (int)__builtin_amdgcn_perm(0u, kLut, (wraw[1 - p][u] >> (2 * q)) & 0x03030303u);
            }
        };
#pragma unroll
        for (int m = 0; m < kMfma; ++m) {
            const int h = m / (FI * FJ), i = (m / FJ) % FI, j = m % FJ;
            acc[i][j] = __builtin_amdgcn_mfma_i32_32x32x32_i8(fa[p][h * FI + i], fb[p][h * FJ + j], acc[i][j], 0, 0, 0);
            // items [m * nItems / kMfma, (m + 1) * nItems / kMfma) follow MFMA m
#pragma unroll
            for (int t = m * nItems / kMfma; t < (m + 1) * nItems / kMfma; ++t) {
                __builtin_amdgcn_sched_barrier(0);
                item(t);
            }
            __builtin_amdgcn_sched_barrier(0);
        }
    };
    // steps [c0, c1) in MODE; the register set follows the step's parity
    auto run = [&](auto MODE, int c0, int c1) {
        int c = c0;
        if (c < c1 && (c & 1)) body(std::integral_constant<int, 1>{}, MODE, c++);
        for (; c + 1 < c1; c += 2) {
            body(std::integral_constant<int, 0>{}, MODE, c);
            body(std::integral_constant<int, 1>{}, MODE, c + 1);
        }
        if (c < c1) body(std::integral_constant<int, 0>{}, MODE, c);
    };
    const int steady_end = max(C - STAGES, 0);
    run(std::integral_constant<int, 0>{}, 0, steady_end);
    run(std::integral_constant<int, 1>{}, steady_end, C - 1);
    run(std::integral_constant<int, 2>{}, C - 1, C);

    // epilogue (this barrier publishes the row scales)
    wait_barrier<0>();
    const int rows = min(BM, a.M - m0);
    if (a.out_i32) {
        store_tile<FI, FJ, 0>(acc, a, m0, rows, mrow, nb, sx_lds, swv);
    } else if (FJ == 2 && a.pair_a) {
        // the host pairs only tiles whose waves hold one 64-column group (in the 256-column
        // tile, even holding pair_a through the main loop made it spill)
        if constexpr (FJ == 2) store_tile_pair<FI, FJ>(acc, a, m0, rows, mrow, nb, sx_lds);
    } else if (a.res) {
        store_tile<FI, FJ, 2>(acc, a, m0, rows, mrow, nb, sx_lds, swv);
    } else {
        store_tile<FI, FJ, 1>(acc, a, m0, rows, mrow, nb, sx_lds, swv);
    }
}

// ---- long K, one round over the CUs: 128 x 160 regions -------------------------------
// Writes a wave's FI x FJ blocks of 16 x 16 (v_mfma_i32_16x16x64_i8 layout: lane l holds
// column l % 16, rows 4 (l / 16) + r of element r) with store_tile's conventions.
// mrow: this lane's first row relative to m0 (includes 4 (lane / 16)); nb: its column.
template <int FI, int FJ, int EPI>
__device__ __forceinline__ void store_tile16(const v4i (&acc)[FI][FJ], const GemmArgs& a, int m0, int rows, int mrow,
                                             int nb, const float* sx, const float (&swv)[FJ]) {
    const unsigned range = (unsigned)rows * (unsigned)a.ldo * 4u;
    const __amdgpu_buffer_rsrc_t out =
        __builtin_amdgcn_make_buffer_rsrc(static_cast<char*>(a.out) + (size_t)m0 * a.ldo * 4, 0, range, kBufDword3);
    const __amdgpu_buffer_rsrc_t res = __builtin_amdgcn_make_buffer_rsrc(
        (void*)(a.res ? a.res + (size_t)m0 * a.ldo : nullptr), 0, EPI == 2 ? range : 0u, kBufDword3);
    int coff[FJ];
#pragma unroll
    for (int j = 0; j < FJ; ++j) {
        const int n = nb + j * 16;
        coff[j] = (int)((unsigned)n * 4u + ((unsigned)(n >= a.N) << 31));
    }
    const int row_bytes = a.ldo * 4;
#pragma unroll
    for (int i = 0; i < FI; ++i) {
        v4f sxv = {};
        if (EPI) sxv = *reinterpret_cast<const v4f*>(sx + mrow + i * 16);  // rows mrow + 16 i + 0..3
        int off[FJ][4];
        float rv[FJ][4];
#pragma unroll
        for (int j = 0; j < FJ; ++j)
#pragma unroll
            for (int r = 0; r < 4; ++r) {
                off[j][r] = (mrow + i * 16 + r) * row_bytes + coff[j];
                if (EPI == 2) rv[j][r] = __builtin_bit_cast(float, __builtin_amdgcn_raw_buffer_load_b32(res, off[j][r], 0, 0));
            }
#pragma unroll
        for (int j = 0; j < FJ; ++j)
#pragma unroll
            for (int r = 0; r < 4; ++r) {
                unsigned bits;
                if (EPI == 0) {
                    bits = (unsigned)acc[i][j][r];
                } else {
                    const float y = ((float)acc[i][j][r] * sxv[r]) * swv[j];
                    bits = __builtin_bit_cast(unsigned, EPI == 2 ? rv[j][r] + y : y);
                }
                __builtin_amdgcn_raw_buffer_store_b32(bits, out, off[j][r], 0, 0);
            }
    }
}

// Region 128 x 160 per workgroup: the 2048 x 2560 outputs of a 6912-deep problem make 256
// regions, one per CU (the tile kernel's 192 x 128 tiles make 220).  Eight waves, two per
// SIMD: four compute waves and four load waves.  A wave that issues a vector-memory load
// waits until the CU's load path accepts it (measured: ~64 B/clk per CU into registers,
// ~40 B/clk straight into LDS), so loads dealt out between the MFMAs add their time to the
// MFMA stream; here no compute wave issues one.
//   * Compute wave w = 2 kh + nh covers K half kh (chunks [kh C / 2, (kh + 1) C / 2), C
//     even) of the region's columns [80 nh, 80 nh + 80) and all 128 rows: 8 x 5 blocks of
//     v_mfma_i32_16x16x64_i8 (160 accumulator registers; this shape runs at full rate with
//     8 or more independent accumulators).  Its A operand is exactly a 1 KiB qx block as
//     loaded (lane l: row l % 16, bytes 16 (l / 16) ..), its B operand one dword of device
//     code per lane (column l % 16, dword l / 16 of the row's 16-byte unit) expanded by four
//     v_perm_b32, the expansion's dependent steps in different gaps between MFMAs.
//   * Each K half has an LDS ring of S stages (its chunk's 8 A blocks and both column
//     halves' 80 weight rows); load wave 4 + 2 kh + q fills A blocks [4 q, 4 q + 4) and the
//     weight rows of column half q, S - 1 chunks ahead, by buffer loads straight into LDS.
//   * One barrier per chunk step: load waves arrive once chunk c + 1 is in LDS (s_waitcnt
//     on their loads), compute waves once their reads of chunk c - 1's stage have returned,
//     so after barrier c chunk c + 1 may be read and chunk c - 1's stage refilled.
//   * A chunk runs as two row halves (fragments 0-3, then 4-7), each over the five column
//     blocks, so that every fragment and expanded B block is refilled for the next chunk
//     right after its last use and 12 or more MFMAs before its next one (the compute waves
//     stall on no LDS read).
// The K-half partners then sum their partial regions in LDS (exact int32) and each compute
// wave stores 64 rows through store_tile16.
constexpr int kRegM = 128, kRegN = 160, kRegS = 7;
constexpr int kRegWBytes = (kRegN / 2) * 16;                     // one column half's weight rows
constexpr int kRegStage = (kRegM / 16) * 1024 + 2 * kRegWBytes;  // A blocks + both halves' rows
constexpr int kRegThreads = 8 * 64;

template <int S>
__global__ void __launch_bounds__(kRegThreads) gemm_region_kernel(GemmGroupArgs ga) {
    constexpr int FI = kRegM / 16, FJ = kRegN / 32;  // per compute wave: 16 x 16 blocks
    constexpr int A_BYTES = FI * 1024, STAGE = kRegStage;
    constexpr int LOADS = FI / 2 + 2;                // loads per load wave and chunk
    constexpr int kMfma = FI * FJ;
    static_assert(FJ * 16 > 64 && FJ * 16 <= 128, "two weight loads per chunk");
    static_assert((S - 2) * LOADS <= 63, "vmcnt range");
    static_assert(2 * S * STAGE >= 4 * (FI / 2) * FJ * 1024, "the rings hold the partial halves");
    extern __shared__ __attribute__((aligned(16))) v4u lds[];
    char* const lds_b = reinterpret_cast<char*>(lds);
    const int t = threadIdx.x, lane = t & 63;
    const int wave = __builtin_amdgcn_readfirstlane(t >> 6);
    const bool loader = wave >= 4;
    const int kh = (wave >> 1) & 1, q = wave & 1;  // K half; column half (compute) or share (load)
    const int reg = xcd_order((int)blockIdx.x, (int)gridDim.x);
    const GemmArgs a = find_gemm(ga, reg);
    const int C = a.C, nR = (a.N + kRegN - 1) / kRegN, lr = reg - a.wg_begin;
    const int m0 = (lr / nR) * kRegM, n0 = (lr % nR) * kRegN + q * (kRegN / 2);
    const int cb = __builtin_amdgcn_readfirstlane(kh ? C >> 1 : 0);
    const int ce = __builtin_amdgcn_readfirstlane(kh ? C : C >> 1);
    char* const ring = lds_b + kh * (S * STAGE);
    auto stage = [&](int c) { return ring + ((c - cb) % S) * STAGE; };

    v4i acc[FI][FJ];
#pragma unroll
    for (int i = 0; i < FI; ++i)
#pragma unroll
        for (int j = 0; j < FJ; ++j) acc[i][j] = v4i{};

    if (loader) {
        // A: 16-row block f of chunk c at ((m0 / 16 + f) C + c) KiB + 16 l of the activations
        // (256-row padding); W: rows n0 + l (and n0 + 64 + l, l < 16), clamped to the padded
        // rows, chunk c at + c KiB
        const unsigned a_bytes = (unsigned)((a.M + 255) & ~255) * (unsigned)C * 64u;
        const __amdgpu_buffer_rsrc_t ar = __builtin_amdgcn_make_buffer_rsrc((void*)a.qx, 0, a_bytes, kBufDword3);
        const __amdgpu_buffer_rsrc_t wr =
            __builtin_amdgcn_make_buffer_rsrc((void*)a.w, 0, (unsigned)a.Np * (unsigned)C * 16u, kBufDword3);
        const int a_soff = ((m0 >> 4) + (FI / 2) * q) * C * 1024;
        auto w_row = [&](int n) {
            n = min(n, a.Np - 1);
            return ((n >> 6) * C * 64 + (n & 63)) * 16;
        };
        const int w_off0 = w_row(n0 + lane), w_off1 = w_row(n0 + 64 + (lane & 15));
        const bool w_second = lane < FJ * 16 - 64;
        typedef __attribute__((address_space(3))) void* lds_p;
        auto load_chunk = [&](int c) {
            char* st = stage(c);
#pragma unroll
            for (int k = 0; k < FI / 2; ++k)
                __builtin_amdgcn_raw_ptr_buffer_load_lds(ar, (lds_p)(st + ((FI / 2) * q + k) * 1024), 16, lane * 16,
                                                         a_soff + (k * C + c) * 1024, 0, 0);
            __builtin_amdgcn_raw_ptr_buffer_load_lds(wr, (lds_p)(st + A_BYTES + q * kRegWBytes), 16, w_off0, c * 1024,
                                                     0, 0);
            if (w_second)
                __builtin_amdgcn_raw_ptr_buffer_load_lds(wr, (lds_p)(st + A_BYTES + q * kRegWBytes + 1024), 16, w_off1,
                                                         c * 1024, 0, 0);
        };
        for (int k = 0; k < S - 1; ++k) load_chunk(cb + k);
        wait_vm<(S - 2) * LOADS>();
        __builtin_amdgcn_s_barrier();  // barrier cb - 1: chunk cb in LDS (no fence: the wait is explicit)
        for (int c = cb; c + 1 < ce; ++c) {
            // barrier c - 1 passed: chunk c - 1's stage is free
            if (c + S - 1 < ce) {
                load_chunk(c + S - 1);
                wait_vm<(S - 2) * LOADS>();
            } else {
                wait_vm<0>();
            }
            __builtin_amdgcn_s_barrier();  // barrier c: chunk c + 1 in LDS
        }
    } else {
        const int a_rd = lane * 16, w_rd = A_BYTES + q * kRegWBytes + (lane & 15) * 16 + 4 * (lane >> 4);
        constexpr int HF = FI / 2;  // A fragments per row half
        unsigned wraw[FJ];          // raw weight dwords (refilled for the next chunk)
        v4i fa[FI];                 // A fragments (refilled for the next chunk)
        v4i fb[FJ];                 // expanded B blocks (re-expanded for the next chunk)
        unsigned xt[2][3], xm[2][4];  // expansion temporaries of blocks j (set j % 2)
        auto read_a = [&](const char* st, int i) { fa[i] = *reinterpret_cast<const v4i*>(st + a_rd + i * 1024); };
        auto read_w = [&](const char* st, int j) { wraw[j] = *reinterpret_cast<const unsigned*>(st + w_rd + j * 256); };
        // step s (0..6) of expanding raw dword wraw[j] into fb[j]: shifts, masks, permutes
        auto expand_step = [&](int j, int s) {
            constexpr unsigned M = 0x03030303u;
            const int e = j & 1;
            if (s == 0) {
                xt[e][0] = wraw[j] >> 2;
                xt[e][1] = wraw[j] >> 4;
                xt[e][2] = wraw[j] >> 6;
            } else if (s == 1) {
                xm[e][0] = wraw[j] & M;
                xm[e][1] = xt[e][0] & M;
            } else if (s == 2) {
                xm[e][2] = xt[e][1] & M;
                xm[e][3] = xt[e][2] & M;
            } else if (s < 7) {
                fb[j][s - 3] = (int)__builtin_amdgcn_perm(0u, kLut, xm[e][s - 3]);
            }
        };
        // Chunk c (LAST: no next chunk), MFMA m = 20 h + 4 j + r: row half h, column block j,
        // A fragment i = 4 h + r.  Items after the MFMAs:
        //   * MFMAs 0-3: this chunk's fragments 4-7 (first used at MFMA 20);
        //   * MFMAs 0-6: the rest of the expansion of this chunk's blocks 3 and 4;
        //   * barrier c before MFMA kBar (this wave's reads have returned), then the next
        //     chunk's weight dwords (MFMAs kBar..kBar + 4) and fragments 0-3 (MFMAs 20-23,
        //     after their last use in this chunk), each 12 or more MFMAs before first use;
        //   * the next chunk's block j (j < 4) expanded at MFMAs 24 + 4 j .. (after its last
        //     use in this chunk at 23 + 4 j), block 3's last steps and block 4 carried over.
        constexpr int kBar = 12;
        auto body = [&](auto LAST, int c) {
            constexpr bool last = decltype(LAST)::value;
            const char* st = stage(c);
            const char* nst = stage(c + 1);
#pragma unroll
            for (int m = 0; m < kMfma; ++m) {
                const int h = m / 20, j = (m % 20) / 4, i = HF * h + m % 4;
                if (m == kBar && !last) {
                    __builtin_amdgcn_sched_barrier(0);
                    asm volatile("s_waitcnt lgkmcnt(0)\n\ts_barrier" ::: "memory");
                    __builtin_amdgcn_sched_barrier(0);
                }
                acc[i][j] = __builtin_amdgcn_mfma_i32_16x16x64_i8(fa[i], fb[j], acc[i][j], 0, 0, 0);
                __builtin_amdgcn_sched_barrier(0);
                if (m < HF) read_a(st, HF + m);
                if (!last) {
                    if (m >= kBar && m < kBar + FJ) read_w(nst, m - kBar);
                    if (m >= 20 && m < 20 + HF) read_a(nst, m - 20);
                }
                __builtin_amdgcn_sched_barrier(0);
                if (m < 3) expand_step(3, 4 + m);
                if (m < 7) expand_step(4, m);
                if (!last) {
#pragma unroll
                    for (int jj = 0; jj < 4; ++jj) {
                        const int k = m - (24 + 4 * jj);
                        if (k >= 0 && k < (jj < 3 ? 7 : 4)) expand_step(jj, k);
                    }
                }
                __builtin_amdgcn_sched_barrier(0);
            }
        };
        static_assert(FI == 8 && FJ == 5 && kMfma == 40, "chunk schedule");
        __builtin_amdgcn_s_barrier();  // barrier cb - 1: chunk cb in LDS
#pragma unroll
        for (int i = 0; i < HF; ++i) read_a(stage(cb), i);
#pragma unroll
        for (int j = 0; j < FJ; ++j) read_w(stage(cb), j);
        // blocks 0-2 expanded, block 3 up to step 3: what a previous chunk would have done
#pragma unroll
        for (int j = 0; j < 4; ++j)
#pragma unroll
            for (int s7 = 0; s7 < (j < 3 ? 7 : 4); ++s7) expand_step(j, s7);
        for (int c = cb; c + 1 < ce; ++c) body(std::false_type{}, c);
        body(std::true_type{}, ce - 1);
    }

    // K halves: compute wave (kh, nh) keeps row blocks [4 kh, 4 kh + 4) and hands the other
    // four to its partner (1 - kh, nh) through slot w of 20 KiB, lane-major (16 bytes per
    // lane and block); the load waves only pass the barriers
    constexpr int HB = FI / 2;
    __syncthreads();  // every wave is done with the rings
    if (!loader) {
        char* mine = lds_b + wave * (HB * FJ * 1024) + lane * 16;
#pragma unroll
        for (int i = 0; i < FI; ++i)
            if ((i >= HB) != (kh == 1))  // the partner's rows
#pragma unroll
                for (int j = 0; j < FJ; ++j) *reinterpret_cast<v4i*>(mine + ((i % HB) * FJ + j) * 1024) = acc[i][j];
    }
    __syncthreads();
    if (loader) return;
    {
        const char* theirs = lds_b + (wave ^ 2) * (HB * FJ * 1024) + lane * 16;
#pragma unroll
        for (int i = 0; i < FI; ++i)
            if ((i >= HB) == (kh == 1))  // this wave's rows
#pragma unroll
                for (int j = 0; j < FJ; ++j) acc[i][j] += *reinterpret_cast<const v4i*>(theirs + ((i % HB) * FJ + j) * 1024);
    }
    const int mrow = HB * 16 * kh + 4 * (lane >> 4), nb = n0 + (lane & 15);
    float swv[FJ];
#pragma unroll
    for (int j = 0; j < FJ; ++j) swv[j] = a.out_i32 ? 0.f : a.rs ? a.rs[min(nb + j * 16, a.N - 1)] : a.s_w;
    const int rows = min(kRegM, a.M - m0);
    const float* const sxp = a.out_i32 ? nullptr : a.sx + m0;
    // this wave's half of the accumulators (row blocks [4 kh, 4 kh + 4))
    auto store = [&](const v4i(&half)[HB][FJ]) {
        if (a.out_i32) store_tile16<HB, FJ, 0>(half, a, m0, rows, mrow, nb, sxp, swv);
        else if (a.res) store_tile16<HB, FJ, 2>(half, a, m0, rows, mrow, nb, sxp, swv);
        else store_tile16<HB, FJ, 1>(half, a, m0, rows, mrow, nb, sxp, swv);
    };
    if (kh) store(reinterpret_cast<const v4i(&)[HB][FJ]>(acc[HB]));
    else store(reinterpret_cast<const v4i(&)[HB][FJ]>(acc[0]));
}

// ---- M <= 64: K split over the waves ------------------------------------------------
// One workgroup per 64-column tile of the output and all (<= 64) rows, over the unit's
// chunks (a part of a long-K problem, GemmArgs::parts, or all C); compute wave w of NW
// covers an NW-th of them (a wave tile of 64 x 64 = 2 x 2 blocks of 32 x 32, fragment
// reads, weight expansion and result layout those of gemm_kernel) from a private LDS ring
// of S stages.  Load wave NW + w fills that ring by direct loads (4 A blocks + 1 weight
// chunk per step, S - 1 steps ahead): a wave that issues a load waits until the CU's load
// path accepts it, which in the compute waves' stream cost more than their MFMAs.  One
// barrier per step: load waves arrive once the next step is in LDS, compute waves after
// the step's MFMAs (their reads of it returned), so the stage just read may be refilled.
// Every wave runs the same number of steps (the larger share), a compute wave with one
// chunk fewer skipping its last.  The NW int32 partial tiles are then summed in LDS
// (exact) and all 2 NW waves apply the fp32 epilogue.  Two workgroups share a CU (80 KiB
// of LDS, at most 128 registers per wave).
template <int NW, int S>
__global__ void __launch_bounds__(2 * NW * 64, 4) gemm_splitk_kernel(GemmGroupArgs ga) {
    constexpr int STAGE = 4 * 1024 + 1024, LOADS = 5;  // A: 4 blocks of 16 rows; W: 1 chunk
    constexpr int NT = 2 * NW * 64;                    // threads
    extern __shared__ __attribute__((aligned(16))) v4u lds[];
    char* const lds_b = reinterpret_cast<char*>(lds);
    const int t = threadIdx.x, lane = t & 63, g = lane >> 5, r32 = lane & 31;
    const int wave = __builtin_amdgcn_readfirstlane(t >> 6);
    const bool loader = wave >= NW;
    const int cw = loader ? wave - NW : wave;  // the compute wave this wave is or feeds
    const GemmArgs a = find_gemm(ga, blockIdx.x);
    const int C = a.C, rb = (int)blockIdx.x - a.wg_begin, n0 = rb * kRowBlock;
    // the epilogue's scales (thread t: column n0 + t % 64, rows t / 64 + 2 NW j), requested now
    // so that the epilogue does not wait for them (a load wave's ring waits count them too:
    // they are older than its ring loads)
    constexpr int EPT = 64 * 64 / NT, RS = NT / 64;  // elements per thread; row stride
    const int n = n0 + lane, mb = t >> 6;
    float sw = 0.0f, sxv[EPT];
    if (!a.out_i32) {
        sw = a.rs ? a.rs[min(n, a.N - 1)] : a.s_w;
#pragma unroll
        for (int j = 0; j < EPT; ++j) sxv[j] = a.sx[mb + RS * j];  // sx holds the 64 padded rows
    }
    // this unit's chunks (one part of a split problem, or all), split over the compute waves
    const int k0 = a.c1 > 0 ? a.c0 : 0, len = (a.c1 > 0 ? a.c1 : C) - k0;
    const int cb = k0 + __builtin_amdgcn_readfirstlane((cw * len) / NW);
    const int cnt = k0 + __builtin_amdgcn_readfirstlane(((cw + 1) * len) / NW) - cb;
    const int steps = (len + NW - 1) / NW;
    char* const ring = lds_b + cw * S * STAGE;
    auto stg = [&](int s) { return ring + (s % S) * STAGE; };  // step s: chunk cb + s

    v16i acc[2][2];
#pragma unroll
    for (int i = 0; i < 2; ++i)
#pragma unroll
        for (int j = 0; j < 2; ++j) acc[i][j] = v16i{};
    if (loader) {
        const int8_t* a_src = a.qx + (size_t)lane * 16;  // block f of chunk c at (f C + c) KiB
        const v4u* w_src = a.w + (size_t)(n0 / kRowBlock) * C * kRowBlock + lane;
        auto issue = [&](int s) {
            char* st = stg(s);
            const int c = cb + s;
#pragma unroll
            for (int f = 0; f < 4; ++f) load_lds16(a_src + ((size_t)f * C + c) * 1024, st + f * 1024);
            load_lds16(w_src + (size_t)c * kRowBlock, st + 4096);
        };
        for (int s = 0; s < S - 1 && s < cnt; ++s) issue(s);
        if (cnt >= S - 1) wait_vm<(S - 2) * LOADS>();
        else wait_vm<0>();
        __builtin_amdgcn_s_barrier();  // barrier -1: step 0 in LDS (no fence: the wait is explicit)
        for (int s = 0; s + 1 < steps; ++s) {
            // barrier s - 1 passed: step s - 1's stage is free
            if (s + S - 1 < cnt) {
                issue(s + S - 1);
                wait_vm<(S - 2) * LOADS>();
            } else {
                wait_vm<0>();
            }
            __builtin_amdgcn_s_barrier();  // barrier s: step s + 1 in LDS
        }
    } else {
        // per-lane read offsets in a stage (as gemm_kernel with WM = WN = 64)
        const int a_rd = (r32 >> 4) * 1024 + ((r32 & 15) + 16 * g) * 16;
        const int w_rd = 4096 + r32 * 16 + g * 4;  // column block j adds 32 rows = 512 bytes
        __builtin_amdgcn_s_barrier();              // barrier -1: step 0 in LDS
        for (int s = 0; s < steps; ++s) {
            if (s < cnt) {
                const char* st = stg(s);
                v4i fa[2][2], fb[2][2];
#pragma unroll
                for (int h = 0; h < 2; ++h) {
#pragma unroll
                    for (int i = 0; i < 2; ++i) fa[h][i] = *reinterpret_cast<const v4i*>(st + a_rd + i * 2048 + h * 512);
#pragma unroll
                    for (int j = 0; j < 2; ++j)
                        fb[h][j] = decode_dword(*reinterpret_cast<const unsigned*>(st + w_rd + j * 512 + h * 8));
                }
#pragma unroll
                for (int h = 0; h < 2; ++h)
#pragma unroll
                    for (int i = 0; i < 2; ++i)
#pragma unroll
                        for (int j = 0; j < 2; ++j)
                            acc[i][j] = __builtin_amdgcn_mfma_i32_32x32x32_i8(fa[h][i], fb[h][j], acc[i][j], 0, 0, 0);
            }
            if (s + 1 < steps) {
                __builtin_amdgcn_sched_barrier(0);
                asm volatile("s_waitcnt lgkmcnt(0)\n\ts_barrier" ::: "memory");  // barrier s
                __builtin_amdgcn_sched_barrier(0);
            }
        }
    }

    // sum the NW partial tiles: compute wave w stores its 64 x 64 int32 tile over its ring
    __syncthreads();  // every wave is done with the rings
    if (!loader) {
        int* part = reinterpret_cast<int*>(ring);
#pragma unroll
        for (int i = 0; i < 2; ++i)
#pragma unroll
            for (int j = 0; j < 2; ++j)
#pragma unroll
                for (int k = 0; k < 16; ++k)
                    part[(i * 32 + 8 * (k >> 2) + 4 * g + (k & 3)) * 64 + j * 32 + r32] = acc[i][j][k];
    }
    __syncthreads();
    // thread t: column n, rows mb + RS j, j < EPT; output and residual as raw buffers over M
    // rows (rows past M fall outside; a column past N adds bit 31)
    int v[EPT];
#pragma unroll
    for (int j = 0; j < EPT; ++j) {
        const int e = t + j * NT;
        int acc_e = 0;
#pragma unroll
        for (int w = 0; w < NW; ++w) acc_e += reinterpret_cast<const int*>(lds_b + w * S * STAGE)[e];
        v[j] = acc_e;
    }
    if (a.parts > 1) {  // one part of a split problem: publish the tile; the last part adds them up
        // The tiles and the count are device-scope (coherent across the XCDs) stores and loads
        // rather than plain ones behind fences: a device-scope fence writes back and
        // invalidates the whole L2 of the XCD (the launch took 33 instead of 19 us).  Each
        // wave's tile stores have completed (s_waitcnt) before the barrier that precedes the
        // count, so the part that sees the final count reads complete tiles.  The flag lives in
        // the ring past wave 0's partial tile (a static LDS variable would push two
        // workgroups past a CU's 160 KiB).
        int& last = *reinterpret_cast<int*>(lds_b + S * STAGE - 4);
        const size_t tile = (size_t)(a.Np / kRowBlock) * 4096;  // one part's tiles
        int* mine = a.part_ws + a.kp * tile + (size_t)rb * 4096;
#pragma unroll
        for (int j = 0; j < EPT; ++j)
            __hip_atomic_store(mine + (mb + RS * j) * 64 + lane, v[j], __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
        __syncthreads();
        if (t == 0)
            last = __hip_atomic_fetch_add(a.cnt + rb, 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) == a.parts - 1;
        __syncthreads();
        if (!last) return;
        for (int p = 0; p < a.parts; ++p) {
            if (p == a.kp) continue;
            const int* other = a.part_ws + p * tile + (size_t)rb * 4096;
#pragma unroll
            for (int j = 0; j < EPT; ++j)
                v[j] += __hip_atomic_load(other + (mb + RS * j) * 64 + lane, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        }
        // every part of this row block has arrived: the count is ready for the next launch
        if (t == 0) __hip_atomic_store(a.cnt + rb, 0, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    }
    const unsigned range = (unsigned)a.M * (unsigned)a.ldo * 4u;
    const __amdgpu_buffer_rsrc_t out = __builtin_amdgcn_make_buffer_rsrc(a.out, 0, range, kBufDword3);
    const int coff = (int)((unsigned)n * 4u + ((unsigned)(n >= a.N) << 31));
    if (a.out_i32) {
#pragma unroll
        for (int j = 0; j < EPT; ++j)
            __builtin_amdgcn_raw_buffer_store_b32((unsigned)v[j], out, (mb + RS * j) * a.ldo * 4 + coff, 0, 0);
        return;
    }
    float rv[EPT];
    const __amdgpu_buffer_rsrc_t res =
        __builtin_amdgcn_make_buffer_rsrc((void*)a.res, 0, a.res ? range : 0u, kBufDword3);
    if (a.res) {
#pragma unroll
        for (int j = 0; j < EPT; ++j)
            rv[j] = __builtin_bit_cast(float, __builtin_amdgcn_raw_buffer_load_b32(res, (mb + RS * j) * a.ldo * 4 + coff, 0, 0));
    }
#pragma unroll
    for (int j = 0; j < EPT; ++j) {
        const float y = ((float)v[j] * sxv[j]) * sw;
        const float o = a.res ? rv[j] + y : y;
        __builtin_amdgcn_raw_buffer_store_b32(__builtin_bit_cast(unsigned, o), out, (mb + RS * j) * a.ldo * 4 + coff, 0, 0);
    }
}

// The kernels' dynamic LDS sizes above 64 KiB are allowed once per device, at context
// creation (gemm_prepare_device), so that no launch, e.g. the first one under a stream
// capture, makes a function-attribute call.
template <typename Kern>
static hipError_t allow_lds(Kern* k, int bytes) {
    return bytes > 65536 ? hipFuncSetAttribute(reinterpret_cast<const void*>(k),
                                               hipFuncAttributeMaxDynamicSharedMemorySize, bytes)
                         : hipSuccess;
}

template <int NW, int S>
constexpr int splitk_lds() { return NW * S * (5 * 1024); }

template <int NW, int S>
static hipError_t launch_splitk(const GemmGroupArgs& ga, int blocks, hipStream_t s) {
    constexpr int LDS = splitk_lds<NW, S>();
    static_assert(S * 5 * 1024 >= 64 * 64 * 4 + 4, "a wave's ring must hold its partial tile (and wave 0's the arrival flag)");
    hipLaunchKernelGGL((gemm_splitk_kernel<NW, S>), dim3((unsigned)blocks), dim3(2 * NW * 64), LDS, s, ga);
    return hipGetLastError();
}

// Four waves per workgroup: 80 KiB of LDS, so two workgroups share a CU and the 356 row
// blocks of a BitNet-2B layer's seven projections are all resident at once (21.2 -> 19.8 us
// against eight waves, 160 KiB, one workgroup per CU and 1.4 rounds).
constexpr int kSplitkWaves = 4;

static GemmGroupArgs group_args(const GemmArgs* dev, const int* u2p, const int* bnd, int nb) {
    GemmGroupArgs ga{dev, u2p, GemmArgs{}, -1, {}};
    if (bnd && nb >= 0 && nb <= kGroupBounds) {
        ga.nb = nb;
        for (int i = 0; i < nb; ++i) ga.bnd[i] = bnd[i];
    }
    return ga;
}

hipError_t launch_gemm_group(const GemmArgs* dev, const int* rb2p, const int* bnd, int nb, int total_rb,
                             hipStream_t s) {
    if (total_rb <= 0) return hipSuccess;
    return launch_splitk<kSplitkWaves, 4>(group_args(dev, rb2p, bnd, nb), total_rb, s);
}

template <int BM, int BN, int WAVES_M, int STAGES>
static hipError_t launch_tile(const GemmGroupArgs& ga, int tiles, hipStream_t s) {
    using T = GemmTile<BM, BN, WAVES_M, STAGES>;
    if (tiles <= 0) return hipSuccess;
    hipLaunchKernelGGL((gemm_kernel<BM, BN, WAVES_M, STAGES>), dim3((unsigned)tiles), dim3(256), T::LDS_BYTES, s, ga);
    return hipGetLastError();
}

template <int S>
static hipError_t launch_region(const GemmGroupArgs& ga, int regions, hipStream_t s) {
    constexpr int LDS = 2 * S * kRegStage;
    if (regions <= 0) return hipSuccess;
    hipLaunchKernelGGL((gemm_region_kernel<S>), dim3((unsigned)regions), dim3(kRegThreads), LDS, s, ga);
    return hipGetLastError();
}

template <int BM, int BN, int WAVES_M, int STAGES>
static hipError_t allow_tile_lds() {
    return allow_lds(&gemm_kernel<BM, BN, WAVES_M, STAGES>, GemmTile<BM, BN, WAVES_M, STAGES>::LDS_BYTES);
}

hipError_t gemm_prepare_device() {
    hipError_t e = allow_lds(&gemm_splitk_kernel<kSplitkWaves, 4>, splitk_lds<kSplitkWaves, 4>());
    if (e == hipSuccess) e = allow_lds(&gemm_region_kernel<kRegS>, 2 * kRegS * kRegStage);
    if (e == hipSuccess) e = allow_tile_lds<128, 128, 2, 4>();
    if (e == hipSuccess) e = allow_tile_lds<256, 128, 2, 4>();
    if (e == hipSuccess) e = allow_tile_lds<256, 256, 2, 4>();
    if (e == hipSuccess) e = allow_tile_lds<192, 128, 2, 4>();
    if (e == hipSuccess) e = allow_tile_lds<64, 128, 1, 8>();
    return e;
}

static hipError_t launch_tile_cfg(int cfg, const GemmGroupArgs& ga, int tiles, hipStream_t s) {
    switch (cfg) {
        case kRegion128x160: return launch_region<kRegS>(ga, tiles, s);
        case kTile128x128: return launch_tile<128, 128, 2, 4>(ga, tiles, s);
        case kTile256x128: return launch_tile<256, 128, 2, 4>(ga, tiles, s);
        case kTile256x256: return launch_tile<256, 256, 2, 4>(ga, tiles, s);
        case kTile192x128: return launch_tile<192, 128, 2, 4>(ga, tiles, s);
        // 64-row tiles do 4 MFMAs per wave per step: an 8-deep ring (64 KiB) keeps more
        // steps of loads in flight (512-token prefill 4.87 -> 4.83 ms)
        case kTile64x128: return launch_tile<64, 128, 1, 8>(ga, tiles, s);
        default: return hipErrorInvalidValue;
    }
}

int gemm_tile_cfg(int M, const int* N, const int* C, int G) {
    if (gemm_bm(M) == 128) return kTile128x128;
    // long K: 128 x 160 regions when they make one round over the CUs.  Every problem must
    // split into two equal K halves (the halves' waves meet at one barrier per chunk) and
    // keep the kernel's 32-bit buffer offsets: activations Mpad x Kp and weights Np x Kp / 4
    // bytes below 2^31.
    bool region_ok = true;
    long long regions = 0;
    const long long mpad = ((long long)M + 255) & ~255ll;
    for (int g = 0; g < G; ++g) {
        const long long np = ((long long)N[g] + kRowBlock - 1) / kRowBlock * kRowBlock;
        region_ok = region_ok && C[g] >= kRegMinC && C[g] % 2 == 0 && mpad * C[g] * 64 < (1ll << 31) &&
                    np * C[g] * 16 < (1ll << 31);
        regions += (long long)((M + kRegM - 1) / kRegM) * ((N[g] + kRegN - 1) / kRegN);
    }
    if (region_ok && regions >= kRegMinTiles && regions <= kRegMaxTiles) return kRegion128x160;
    const long long mt = (M + 255) / 256;
    const long long mt192 = (M + 191) / 192;
    long long t256 = 0, t128 = 0, t192 = 0;
    for (int g = 0; g < G; ++g) {
        t256 += mt * ((N[g] + 255) / 256);
        t128 += mt * ((N[g] + 127) / 128);
        t192 += mt192 * ((N[g] + 127) / 128);
    }
    if (t256 >= kGemmFillTiles) return kTile256x256;
    if (t192 >= kGemm192Min && t192 <= kGemm192Max) return kTile192x128;
    if (t128 >= kGemmHalfTiles) return kTile256x128;
    return 2 * t128 >= kGemmHalfTiles ? kTile128x128 : kTile64x128;
}

long long gemm_tile_count(int cfg, int M, int N) {
    const int bm = gemm_tile_bm(cfg), bn = gemm_tile_bn(cfg);
    return (long long)((M + bm - 1) / bm) * ((N + bn - 1) / bn);
}

hipError_t launch_gemm_tiles(const GemmArgs* dev, const int* tile2p, const int* bnd, int nb, int total_tiles, int cfg,
                             hipStream_t s) {
    return launch_tile_cfg(cfg, group_args(dev, tile2p, bnd, nb), total_tiles, s);
}

hipError_t launch_gemm(const GemmArgs& a, hipStream_t s) {
    if (a.M <= 0 || a.N <= 0) return hipSuccess;
    // byte offsets inside one tile's rows are 32-bit
    if (!gemm_ldo_ok(a.M, a.ldo)) return hipErrorInvalidValue;
    // gemm_bm(M) sized the activation padding; the row tile divides it or clamps its loads
    const int bm = gemm_bm(a.M);
    if (bm == 64) {
        GemmArgs one = a;
        one.wg_begin = 0;
        return launch_splitk<kSplitkWaves, 4>(GemmGroupArgs{nullptr, nullptr, one, -1, {}}, a.Np / kRowBlock, s);
    }
    const int cfg = gemm_tile_cfg(a.M, &a.N, &a.C, 1);
    GemmArgs one = a;
    one.wg_begin = 0;
    return launch_tile_cfg(cfg, GemmGroupArgs{nullptr, nullptr, one, -1, {}}, (int)gemm_tile_count(cfg, a.M, a.N), s);
}

}  // namespace rt
