// Decode GEMV / skinny GEMM for the ternary linear, M = 1..8 tokens per workgroup,
// no MFMA.  Replaces the reference's thread-per-row OpenCL kernel
// (src/rotor/gpu_ternary.py:12-45, launched per token at src/rotor/transformer.py:134-143)
// and its CPU twin np.dot(x, W_i8.T) * scale (src/rotor/transformer.py:150).
//
// Mapping (lane-per-row, wave-per-row-tile):
//   * a wave owns one 64-row block of one problem; lane r accumulates row 64*rb + r,
//     so no cross-lane reduction is needed;
//   * each chunk step is one coalesced 16-byte-per-lane (1 KiB per wave) non-temporal
//     buffer load of rotor bytes; loads run one batch of U chunks ahead of the math;
//   * the activations of a chunk are the same for all 64 lanes, so they are read
//     with scalar loads into SGPRs and fed to v_dot4_i32_i8 as the scalar operand.
// Two launch shapes share the body:
//   * ROWS   (many row blocks, e.g. plans): a workgroup of nw waves covers nw
//     consecutive row blocks, each wave the whole K range;
//   * KSPLIT (few row blocks, e.g. one 6912x2560 GEMV): a workgroup is one row block
//     and its nw waves split the K chunks, combined through LDS.
//
// Decoding costs 5 VALU ops per 16 weights.  The tiles hold the device code g = w + 1
// (rt_internal.h), and a 2-bit field masked in place is a non-negative int8 multiple
// of g.  For a weight dword u (four bytes of four fields each) and h = u >> 4:
//     u & 0x03030303, h & 0x03030303   -> g of elements 0 and 2 of each byte
//     u & 0x0C0C0C0C, h & 0x0C0C0C0C   -> 4 g of elements 1 and 3
// so v_dot4_i32_i8 against the matching activation dwords accumulates sum g x into
// accP and 4 sum g x into accQ, and, with g = w + 1,
//     sum w x = accP + accQ / 4 - sum x.
// sum x over the same k range (padding activations are 0) is the same for every lane:
// each wave computes it once from the activation row (slice_sums), or, where a prologue
// quantised the row, the prologue leaves the row's total and one wave subtracts it.
#include <algorithm>
#include <type_traits>

#include "rt_rowquant.h"
#include "rt_attn_decode.h"

// every fp32 operation rounds on its own, as the reference restatement computes them
#pragma clang fp contract(off)

namespace rt {

constexpr int kAuxNT = 2;                 // cache policy: non-temporal (streamed once)

// The activations are read-only for the whole launch, so the constant address space
// lets uniform reads become s_load; a prologue-quantised row is read from LDS.
typedef __attribute__((address_space(4))) const int cint;
typedef __attribute__((address_space(3))) const int lint;

// Problem of global row block rbg.  Small plans: the descriptors are kernel arguments and
// the problem is the last one whose wg_begin <= rbg (scalar compares and selects).  Larger
// plans: two dependent scalar loads (table, descriptor), both read through
// constant-address-space pointers: merged with a generic one, the descriptor would turn
// into per-lane flat loads and the buffer resource into a readfirstlane loop.
typedef __attribute__((address_space(4))) const GemvProb cprob;
typedef __attribute__((address_space(4))) const int cidx;
__device__ __forceinline__ GemvProb find_prob(const GemvArgs& a, int rbg) {
    if (a.ninl > 0) {  // every descriptor is loaded (independent loads), then selected
        GemvProb P = a.inl[0];
#pragma unroll
        for (int j = 1; j < kInlineProbs; ++j)
            if (j < a.ninl && rbg >= a.inl[j].wg_begin) P = a.inl[j];
        return P;
    }
    if (!a.dev) return a.p;
    const cprob* q = (cprob*)a.dev + ((cidx*)a.rb2p)[rbg];
    return GemvProb{q->w, q->qx, q->sx, q->rs, q->out, q->s_w, q->N, q->C, q->ldo, q->wg_begin, q->res, q->xs, q->K};
}

// floor(a / nw) from m = ceil(2^31 / nw), for 1 <= nw <= 16 and 0 <= a < 2^23 (a = wave * C
// with C <= 2^16: weights hold K <= 2^22): with m nw = 2^31 + e, 0 <= e < nw, the quotient is
// exact while a e < 2^31.  SALU multiplies only: a division by the kernel argument nw runs on
// the VALU, and chunk bounds left in VGPRs put the buffer resource in VGPRs (a readfirstlane
// loop around every weight load).  (An inline-asm readfirstlane is no way out: the compiler
// inserts no wait states before an asm statement that reads a VGPR its previous VALU
// instruction wrote, and the asm can read the stale value.)
__device__ __forceinline__ int div_nw(int a, unsigned m) {
    return (int)(((unsigned long long)(unsigned)a * m) >> 31);
}
static unsigned nw_reciprocal(int nw) { return (unsigned)(((1ull << 31) + (unsigned)nw - 1) / (unsigned)nw); }

// The weight stream of global row block rbg, before anything else: for inline problems from
// the leading table of the arguments (one scalar load, then selects: no branch, no second
// load); otherwise from the row-block table and the descriptor.
struct WStream {
    const v4u* w;
    int C, wg_begin;
    int j;  // inline problems: the problem's index
};
// ninl: a.ninl, passed separately where it is a preloaded kernel argument.
__device__ __forceinline__ WStream find_stream(const GemvArgs& a, int ninl, int rbg) {
    if (ninl > 0) {
        WStream s{a.inw[0].w, a.inw[0].C, a.inw[0].wg_begin, 0};
#pragma unroll
        for (int j = 1; j < kInlineProbs; ++j) {
            const bool t = j < ninl && rbg >= a.inw[j].wg_begin;
            s.w = t ? a.inw[j].w : s.w;
            s.C = t ? a.inw[j].C : s.C;
            s.wg_begin = t ? a.inw[j].wg_begin : s.wg_begin;
            s.j = t ? j : s.j;
        }
        return s;
    }
    const GemvProb P = find_prob(a, rbg);
    return WStream{P.w, P.C, P.wg_begin, 0};
}

// The plain absmax quantisation of problem P's own input row (has_pro == 2).
__device__ __forceinline__ QuantProb own_source(const GemvProb& P) {
    return QuantProb{P.xs, nullptr, nullptr, nullptr, nullptr, P.K, P.C * kChunk, kQuant, nullptr, 0.0f, nullptr,
                     nullptr, 0, 0, 0};
}

template <int MT, typename XP>
__device__ __forceinline__ void chunk_step(const v4u v, XP* __restrict__ xc, const int ldx,
                                           int (&accP)[MT], int (&accQ)[MT]) {
    int d[16];
#pragma unroll
    for (int j = 0; j < 4; ++j) {
        const unsigned u = v[j];
        const unsigned h = u >> 4;
        d[4 * j + 0] = (int)(u & 0x03030303u);
        d[4 * j + 1] = (int)(u & 0x0C0C0C0Cu);
        d[4 * j + 2] = (int)(h & 0x03030303u);
        d[4 * j + 3] = (int)(h & 0x0C0C0C0Cu);
    }
#pragma unroll
    for (int m = 0; m < MT; ++m) {
        XP* __restrict__ xm = xc + m * ldx;
#pragma unroll
        for (int j = 0; j < 4; ++j) {
            accP[m] = __builtin_amdgcn_sdot4(d[4 * j + 0], xm[4 * j + 0], accP[m], false);
            accQ[m] = __builtin_amdgcn_sdot4(d[4 * j + 1], xm[4 * j + 1], accQ[m], false);
            accP[m] = __builtin_amdgcn_sdot4(d[4 * j + 2], xm[4 * j + 2], accP[m], false);
            accQ[m] = __builtin_amdgcn_sdot4(d[4 * j + 3], xm[4 * j + 3], accQ[m], false);
        }
    }
}

// sum x over activation dwords [d0, d1) (multiples of 4) of each of the MT rows at xq
// (row stride ldx dwords): lane l takes the 16-byte units d0 / 4 + l + 64 i, all loads
// issued before the first v_dot4 (against 0x01010101), then the wave adds the lanes up.
template <int MT, typename XP>
__device__ __forceinline__ void slice_sums(XP* __restrict__ xq, const int ldx, const int d0, const int d1,
                                           int (&sx)[MT]) {
    constexpr int R = 4;  // units per lane per round: one round covers K <= 16384
    const int lane = threadIdx.x & 63, u0 = d0 >> 2, u1 = d1 >> 2;
#pragma unroll
    for (int m = 0; m < MT; ++m) {
        XP* __restrict__ xm = xq + m * ldx;
        int t = 0;
        for (int u = u0 + lane; u < u1 + lane; u += 64 * R) {
            v4u x[R];
#pragma unroll
            for (int r = 0; r < R; ++r) {
                const int ur = u + 64 * r;
                if (ur < u1) {
                    x[r][0] = xm[4 * ur + 0];
                    x[r][1] = xm[4 * ur + 1];
                    x[r][2] = xm[4 * ur + 2];
                    x[r][3] = xm[4 * ur + 3];
                } else {
                    x[r] = v4u{0u, 0u, 0u, 0u};
                }
            }
#pragma unroll
            for (int r = 0; r < R; ++r)
#pragma unroll
                for (int j = 0; j < 4; ++j) t = __builtin_amdgcn_sdot4((int)x[r][j], 0x01010101, t, false);
        }
        sx[m] = wave_sum(t);
    }
}

// sum w x of one row from the two accumulators and the slice's sum x
__device__ __forceinline__ int row_dot(int accP, int accQ, int sx) { return accP + (accQ >> 2) - sx; }

// Accumulate chunks [cb, ce) of one row block.  `rsrc` starts at the row block and
// ends at chunk ce (num_records = ce KiB).  The chunk offset goes into the VGPR offset,
// which the buffer unit range-checks (the SGPR offset is not checked), so the loads
// that run past the range come back as zeros without touching memory.  That keeps
// every load unconditional -- two batches of U chunks in flight -- while the math on
// chunks >= ce is skipped.  The first two batches (A: chunks cb.., B: cb + U..) are
// issued by gemv_preload, which a caller may run before other work (a prologue) to
// overlap the weight latency with it.
template <int U>
__device__ __forceinline__ v4u gemv_load(__amdgpu_buffer_rsrc_t rsrc, const int lane_off, int c) {
    return __builtin_bit_cast(v4u, __builtin_amdgcn_raw_buffer_load_b128(rsrc, lane_off + c * 1024, 0, kAuxNT));
}

template <int U>
__device__ __forceinline__ void gemv_preload(__amdgpu_buffer_rsrc_t rsrc, const int lane_off, const int cb,
                                             v4u (&A)[U], v4u (&B)[U], bool second = true) {
#pragma unroll
    for (int i = 0; i < U; ++i) A[i] = gemv_load<U>(rsrc, lane_off, cb + i);
    if (second) {
#pragma unroll
        for (int i = 0; i < U; ++i) B[i] = gemv_load<U>(rsrc, lane_off, cb + U + i);
    }
}

// SHORT: the wave walks a few chunks (the K-split decode launches): a batch that starts
// past ce is not issued (its loads would return zeros, but the wave still waits for them
// before reusing the registers and at the closing barrier: decode 1.074 -> 1.055 ms/token).
// Long streams (the rows kernel) issue every batch unconditionally (3 % faster there).
template <int MT, int U, typename XP, bool SHORT = false>
__device__ __forceinline__ void gemv_body(__amdgpu_buffer_rsrc_t rsrc, const int lane_off, XP* __restrict__ xq,
                                          const int ldx, const int cb, const int ce, int (&accP)[MT],
                                          int (&accQ)[MT], v4u (&A)[U], v4u (&B)[U]) {
    for (int c = cb; c < ce; c += 2 * U) {
#pragma unroll
        for (int i = 0; i < U; ++i)
            if (c + i < ce) chunk_step<MT, XP>(A[i], xq + (c + i) * 16, ldx, accP, accQ);
        if (!SHORT || c + 2 * U < ce) {
#pragma unroll
            for (int i = 0; i < U; ++i) A[i] = gemv_load<U>(rsrc, lane_off, c + 2 * U + i);
        }
#pragma unroll
        for (int i = 0; i < U; ++i)
            if (c + U + i < ce) chunk_step<MT, XP>(B[i], xq + (c + U + i) * 16, ldx, accP, accQ);
        if (!SHORT || c + 3 * U < ce) {
#pragma unroll
            for (int i = 0; i < U; ++i) B[i] = gemv_load<U>(rsrc, lane_off, c + 3 * U + i);
        }
    }
}

// The fp32 output of row r of row block rb for one token (M = 1, fp32 output), from the
// row's residual res_v and scale sw_v loaded beforehand: stored, and returned for the
// statistics epilogue (0 for rows past N, which are not stored).
__device__ __forceinline__ float emit1(const GemvProb& P, int rb, int r, int acc, float sx_pro, float res_v,
                                       float sw_v) {
    const int n = rb * kRowBlock + r;
    if (n >= P.N) return 0.0f;
    const float y = ((float)acc * sx_pro) * sw_v;
    const float o = P.res ? res_v + y : y;
    static_cast<float*>(P.out)[n] = o;
    return o;
}

// sx_pro: the token scale computed by a prologue (used instead of P.sx when >= 0)
__device__ __forceinline__ void emit(const GemvArgs& a, const GemvProb& P, int rb, int m0, int m, int r, int acc,
                                     float sx_pro = -1.0f) {
    const int n = rb * kRowBlock + r, mg = m0 + m;
    if (n >= P.N || mg >= a.M) return;
    if (a.out_i32) {
        static_cast<int*>(P.out)[(size_t)mg * P.ldo + n] = acc;
    } else {
        const float sw = P.rs ? P.rs[n] : P.s_w;
        const size_t o = (size_t)mg * P.ldo + n;
        const float sx = sx_pro >= 0.0f ? sx_pro : P.sx[mg];
        const float y = ((float)acc * sx) * sw;
        static_cast<float*>(P.out)[o] = P.res ? P.res[o] + y : y;
    }
}

// PRO 0: activations quantised beforehand (qx); PRO 1 (M = 1): the workgroup first
// quantises its problem's own fp32 row into LDS.  With PRO the host sizes workgroups so
// that nw divides every problem's row-block count: all waves of a workgroup are live and
// serve one problem (the prologue synchronises the workgroup).
template <int MT, int PRO>
__global__ void __launch_bounds__(1024) gemv_rows_kernel(GemvArgs a) {
    constexpr int U = MT == 1 ? 4 : 2;
    extern __shared__ __attribute__((aligned(16))) v4u lds_row[];
    const int lane = threadIdx.x & 63, nw = blockDim.x >> 6;
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);  // wave-uniform
    // Workgroups of one problem run on one XCD, so its activation row is fetched into one
    // L2 rather than up to eight (metric plan 6.29 -> 6.46 TB/s)
    const int rbg = xcd_order((int)blockIdx.x, (int)gridDim.x) * nw + wave;  // global row block
    if (PRO == 0 && rbg >= a.total_rb) return;
    const GemvProb P = find_prob(a, rbg);
    const int rb = rbg - P.wg_begin;
    const int m0 = blockIdx.y * MT;
    const int C = P.C, ldx = C * 16;
    const __amdgpu_buffer_rsrc_t rsrc =
        __builtin_amdgcn_make_buffer_rsrc((void*)(P.w + (size_t)rb * C * kRowBlock), 0, C * 1024, kBufDword3);
    int accP[MT], accQ[MT], sx[MT];
#pragma unroll
    for (int m = 0; m < MT; ++m) accP[m] = accQ[m] = 0;
    v4u A[U], B[U];
    if constexpr (PRO != 0) {
        static_assert(MT == 1, "the prologue quantises one token");
        // Several workgroups share a CU, most of them streaming: the waves of one in its
        // prologue issue first until the row is in LDS (metric plan 6.17 -> 6.28 TB/s).  Both
        // weight batches go out before the prologue (the loop holds both; same registers):
        // metric +0.7 % over eight alternating pairs against the second batch after it.
        __builtin_amdgcn_s_setprio(2);
        const QuantProb Q = own_source(P);
        RowRegs rr;
        const bool early = row_fits1(Q, blockDim.x);
        if (early) row_load1(Q, 0, rr);
        gemv_preload<U>(rsrc, lane * 16, 0, A, B, true);
        RowSmem* sm = reinterpret_cast<RowSmem*>(lds_row + (Q.Kp >> 4));
        const QxRow qrow{lds_row, 4, 1};
        const float s_pro = early ? row_finish1(Q, rr, qrow, nullptr, nullptr, sm)
                                  : row_quantize<1>(Q, 0, qrow, nullptr, nullptr, sm);
        __syncthreads();
        __builtin_amdgcn_s_setprio(0);
        slice_sums<MT, lint>((lint*)lds_row, ldx, 0, ldx, sx);
        gemv_body<MT, U, lint>(rsrc, lane * 16, (lint*)lds_row, ldx, 0, C, accP, accQ, A, B);
        emit(a, P, rb, 0, 0, lane, row_dot(accP[0], accQ[0], sx[0]), s_pro);
    } else {
        cint* xq = (cint*)(reinterpret_cast<const int*>(P.qx) + (size_t)m0 * ldx);
        // the activation loads for sum x go out before the weights, so waiting for them
        // does not wait for the weight batches
        slice_sums<MT, cint>(xq, ldx, 0, ldx, sx);
        gemv_preload<U>(rsrc, lane * 16, 0, A, B);
        gemv_body<MT, U, cint>(rsrc, lane * 16, xq, ldx, 0, C, accP, accQ, A, B);
#pragma unroll
        for (int m = 0; m < MT; ++m) emit(a, P, rb, m0, m, lane, row_dot(accP[m], accQ[m], sx[m]));
    }
}

// The attention prologue holds 4 (kAttnSMax + 1) + 2 kAttnSMax values per thread in
// registers; its kernel runs at most 10 waves per workgroup, which leaves 168 VGPRs per
// lane (at 16 waves the budget is 128 and the partials would spill to scratch).
constexpr int kAttnMaxThreads = 640;

// LDS of the KSPLIT kernel: [nw][MT][64] int partial sums, then (prologue) the
// quantised input row (Kp bytes) and the reduction scratch of the prologue.
// PRO: 0 no prologue; 1 prologue quantising a row source (plain, RMSNorm, relu²·up,
// relu²·up + sub-norm), 16 elements per thread; 3 / 4 the same with 4 / 8 consecutive
// elements per thread (K % 64 == 0, K / 4 or K / 8 <= threads, 16-byte aligned sources);
// 2 prologue combining decode-attention partials (kAttnNorm).
// PAIR (PRO 3, gate/up of the decode FFN): the matrix interleaves gate and up in 32-row
// groups (row 64 j + r: gate row 32 j + r for r < 32, up row 32 j + r - 32 otherwise), so a
// workgroup's row block holds both inputs of 32 outputs: it writes the FFN activation
// a = relu(g)^2 * u of those 32 (g and u rounded as emit rounds y) and their f64 sum of
// squares, the two inputs of the down projection's sub-norm.
// Tail = AttnTail (M = 1, fp32 outputs): the attention partials of the token run in the
// same launch (qkv_attn_block): the GEMV's outputs are also stored as epoch-tagged
// device-coherent words, which the attention workgroups poll.
struct NoTail {};
template <int HD>
__device__ __forceinline__ void qkv_attn_block(const AttnTail& at, int total_rb);
// The launch's epoch (AttnTail): *done / natt + 1, the same for every workgroup of a launch.
__device__ __forceinline__ unsigned attn_epoch(const AttnTail& at) {
    return __hip_atomic_load(at.done, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) / at.natt + 1u;
}
template <int MT, int PRO, bool PAIR = false, typename Tail = NoTail>
__global__ void __launch_bounds__(PRO == 2 ? kAttnMaxThreads : 1024)
    gemv_ksplit_kernel(const float* pro_x, const float* pro_aux, const float* pro_aux2, int pro_K, int pro_mode,
                       float pro_eps, unsigned shape, unsigned nw_m, const v4u* w1, GemvArgs a, Tail at) {
    constexpr bool SIG = std::is_same<Tail, AttnTail>::value;
    if constexpr (SIG) {
        // the GEMV's workgroup count rides in the shape word (a launch of inline problems
        // has no C1), so the GEMV workgroups start without a kernel-argument load
        static_assert(MT == 1 && !PAIR, "attention partials follow the one-token qkv GEMV");
        const int total_rb = (int)(shape >> 8);
        if ((int)blockIdx.x >= total_rb) {
            qkv_attn_block<128>(at, total_rb);
            return;
        }
    }
    // The prologue source's fields, the launch shape word (waves per workgroup nw in bits
    // 0-4, inline problem count in bits 5-7, the chunks per row C1 of a one-problem launch
    // from bit 8), nw_m = ceil(2^31 / nw) and the weight tiles w1 of a one-problem launch
    // (null otherwise) lead the argument list as scalars: the kernel-argument preload
    // (-amdgpu-kernarg-preload-count; 14 dwords fit, these are 13) has them in SGPRs when
    // the waves start, so the row's loads and the first weight loads go out before any
    // kernel-argument load returns (blockDim would be one more load).
    const int ninl = (int)((shape >> 5) & 7u), C1 = (int)(shape >> 8);
    QuantProb pro = a.pro;
    pro.x = pro_x;
    pro.aux = pro_aux;
    pro.aux2 = pro_aux2;
    pro.K = pro_K;
    pro.mode = pro_mode;
    pro.eps = pro_eps;
    constexpr int U = MT == 1 ? 4 : 2;
    extern __shared__ __attribute__((aligned(16))) int red[];
    const int lane = threadIdx.x & 63, nw = (int)(shape & 31u);
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int m0 = blockIdx.y * MT;
    // With a prologue whose row fits one group per thread, the row's loads go out first
    // (they do not depend on the problem); then the problem, the weight resource and the
    // first weight batches, which stream in during the prologue's arithmetic.
    constexpr bool VEC = PRO == 3 || PRO == 4 || PRO == 6;  // the E-element prologues
    constexpr int E = PRO == 4 ? 8 : PRO == 6 ? 16 : 4;      // elements per thread of PRO 3 / 4 / 6
    using Regs = typename std::conditional<PRO == 2, AttnRegs,
                                           typename std::conditional<VEC, RowRegsE<E>, RowRegs>::type>::type;
    Regs rr;
    bool early = false;
    if constexpr (PRO == 1) {
        early = row_fits1(pro, blockDim.x);
        if (early) row_load1(pro, 0, rr);
    } else if constexpr (VEC) {
        early = true;  // the host launches PRO 3 / 4 / 6 only where K % 64 == 0 and K / E <= threads
        row_loadE<E>(pro, rr);
    } else if constexpr (PRO == 2) {
        early = attn_fits1(pro, blockDim.x);
        if (early) attn_load1(pro, rr);
    }
    static_assert(!PAIR || (VEC && MT == 1), "the pair epilogue follows an E-element prologue");
    const WStream ws = w1 ? WStream{w1, C1, 0, 0} : find_stream(a, ninl, blockIdx.x);
    const int rb = blockIdx.x - ws.wg_begin;
    const int C = ws.C, ldx = C * 16;
    // the wave's chunks [cb, ce): wave-uniform, in SGPRs (the buffer resource must not be
    // per-lane)
    const int cb = div_nw(wave * C, nw_m);
    const int ce = div_nw((wave + 1) * C, nw_m);
    const __amdgpu_buffer_rsrc_t rsrc =
        __builtin_amdgcn_make_buffer_rsrc((void*)(ws.w + (size_t)rb * C * kRowBlock), 0, ce * 1024, kBufDword3);
    v4u A[U], B[U];
    int accP[MT], accQ[MT], sx[MT];
#pragma unroll
    for (int m = 0; m < MT; ++m) accP[m] = accQ[m] = 0;
    // The rest of the descriptor (epilogue): for inline problems the one at the index the
    // stream lookup chose; otherwise the table lookup.
    const int pj = __builtin_amdgcn_readfirstlane(ws.j);
    GemvProb P;
    if (ninl > 0) {
        P = a.inl[0];
#pragma unroll
        for (int j = 1; j < kInlineProbs; ++j)
            if (pj == j) P = a.inl[j];
    } else {
        P = find_prob(a, blockIdx.x);
    }
    // sum x of the wave's slice: without a prologue its activation loads go out before
    // the weights (waiting for them then does not wait for the weight batches)
    cint* xq = (cint*)(reinterpret_cast<const int*>(P.qx) + (size_t)m0 * ldx);
    if constexpr (PRO == 0) slice_sums<MT, cint>(xq, ldx, cb * 16, ce * 16, sx);
    // With a prologue only the first batch is in flight during it (register budget); the
    // attention prologue holds its partials in registers first and issues it after their
    // combine.
    if (PRO != 2 || !early) gemv_preload<U>(rsrc, lane * 16, cb, A, B, PRO == 0 && cb + U < ce);
    // one token with a prologue: the residual and scale of wave 0's rows (the epilogue's),
    // requested now so that the epilogue does not wait for them
    float res_v = 0.0f, sw_v = P.s_w;
    if constexpr (MT == 1 && PRO != 0 && !PAIR) {
        const int n = rb * kRowBlock + lane;
        if (wave == 0 && n < P.N) {
            if (P.res) res_v = P.res[n];
            if (P.rs) sw_v = P.rs[n];
        }
    }
    // the tagged copy of the outputs: its address and the launch's epoch are read now, while
    // the prologue's row is in flight, and kept in SGPRs (read in the epilogue, the kernel
    // argument and the epoch would cost two memory latencies there)
    unsigned long long* tagged = nullptr;
    unsigned long long tag = 0;
    if constexpr (SIG) {
        tagged = at.tagged + (size_t)blockIdx.x * kRowBlock;
        tag = (unsigned long long)attn_epoch(at) << 32;
        asm volatile("" ::"s"(tagged), "s"(tag));
    }
    float sx_pro = -1.0f;
    if constexpr (PRO != 0) {
        v4u* lq = reinterpret_cast<v4u*>(red + nw * MT * kRowBlock);
        RowSmem* sm = reinterpret_cast<RowSmem*>(lq + (pro.Kp >> 4));
        sm->fac = (lfloat*)(sm + 1);  // kAttnNorm factors follow
        const QxRow qrow{lq, 4, 1};
        if (!early) sx_pro = row_quantize<1>(pro, 0, qrow, nullptr, nullptr, sm);
        else if constexpr (PRO == 1) sx_pro = row_finish1(pro, rr, qrow, nullptr, nullptr, sm);
        else if constexpr (VEC) sx_pro = row_finishE<E>(pro, rr, lq, sm);
        else {
            float v[4];
            attn_combine1(pro, rr, v);
            const float w[4] = {rr.w[0], rr.w[1], rr.w[2], rr.w[3]};
            gemv_preload<U>(rsrc, lane * 16, cb, A, B, false);
            sx_pro = attn_norm1(pro, v, w, rr.live, lq, sm);
        }
        if (cb + U < ce) {
#pragma unroll
            for (int i = 0; i < U; ++i) B[i] = gemv_load<U>(rsrc, lane * 16, cb + U + i);
        }
        __syncthreads();
        if (VEC || (PRO == 2 && early)) {
            // the prologue left each (live) wave's sum of quantised values in RowSmem::qs:
            // wave 0 subtracts the row's total, the other waves nothing (the epilogue adds
            // the waves)
            const int nq = VEC ? (pro.K / E + 63) >> 6 : nw;
            sx[0] = wave == 0 ? slots_reduce(sm->qs, nq, [](int x, int y) { return x + y; }) : 0;
        } else {
            slice_sums<MT, lint>((lint*)lq, ldx, cb * 16, ce * 16, sx);
        }
        gemv_body<MT, U, lint, true>(rsrc, lane * 16, (lint*)lq, ldx, cb, ce, accP, accQ, A, B);
    } else {
        gemv_body<MT, U, cint, true>(rsrc, lane * 16, xq, ldx, cb, ce, accP, accQ, A, B);
    }
#pragma unroll
    for (int m = 0; m < MT; ++m) red[(wave * MT + m) * kRowBlock + lane] = row_dot(accP[m], accQ[m], sx[m]);
    __syncthreads();
    if constexpr (PAIR) {
        if (threadIdx.x < kRowBlock) {  // wave 0; lanes 32.. only pad the reduction
            const int r = threadIdx.x & 31, nu = rb * kRowBlock + 32 + r, i = rb * 32 + r;
            int sg = 0, su = 0;
            for (int w = 0; w < nw; ++w) {
                sg += red[w * kRowBlock + r];
                su += red[w * kRowBlock + 32 + r];
            }
            float av = 0.0f;
            const bool valid = threadIdx.x < 32 && nu < P.N;
            if (valid) {
                const float g = ((float)sg * sx_pro) * a.pair_sg;
                const float u = ((float)su * sx_pro) * a.pair_su;
                av = g > 0.0f ? (g * g) * u : 0.0f;
                a.pair_a[i] = av;
                if (a.pair_g) a.pair_g[i] = g;
                if (a.pair_u) a.pair_u[i] = u;
            }
            const double ss = wave_reduce63((double)av * (double)av, 0.0, [](double x, double y) { return x + y; });
            if (threadIdx.x == kRowBlock - 1) a.pair_ssq[rb] = ss;
        }
        return;
    }
    if (MT == 1 && PRO != 0 && !a.out_i32) {  // one token, fp32 outputs
        if (threadIdx.x < kRowBlock) {
            const int r = threadIdx.x;
            int s = 0;
            for (int w = 0; w < nw; ++w) s += red[w * kRowBlock + r];
            const float o = emit1(P, rb, r, s, sx_pro, res_v, sw_v);
            if constexpr (SIG) {
                // rows past N are not read (every problem of a joint launch has N % 64 == 0)
                __hip_atomic_store(tagged + r, tag | __float_as_uint(o), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
            }
            if (a.out_ssq) {  // the next plan's RMSNORM_SSQ input (rows past N add 0)
                const double ss = half_reduce31((double)o * (double)o, 0.0, [](double x, double y) { return x + y; });
                const int grp = (rb * kRowBlock + r) >> 5;  // groups wholly past N have no entry
                if ((r & 31) == 31 && grp * 32 < P.N) a.out_ssq[grp] = ss;
            }
        }
        return;
    }
    for (int idx = threadIdx.x; idx < MT * kRowBlock; idx += blockDim.x) {
        const int m = idx / kRowBlock, r = idx % kRowBlock;
        int s = 0;
        for (int w = 0; w < nw; ++w) s += red[(w * MT + m) * kRowBlock + r];
        emit(a, P, rb, m0, m, r, s, sx_pro);
    }
}

// Decode qkv GEMV (E-element RMSNorm prologue) with the attention partials of the token in
// the same launch: workgroups [0, total_rb) are the GEMV's row blocks (q, k, v problems),
// the following Hkv * P workgroups (P = S Gq / hpw) the attention of (KV head kh, key block
// s, query heads hp hpw .. hp hpw + hpw - 1 of the group), kh slowest, then hp, each of hpw
// 256-thread tiles (blockDim = 256 Gq: the waves past hpw tiles end at once).  Splitting a
// group's heads over workgroups spreads the tiles' arithmetic over more CUs.  An attention
// workgroup issues its key block's loads and reads the position and the epoch; when its
// block holds a key, its first (hpw + 2) hd threads (one per q value of its heads and k, v
// value of its KV group) poll the GEMV's tagged outputs (bounded) until each carries the
// epoch and leave the values in LDS, and the tiles of rt_attn_decode.h run on them.
// Forward progress: the attention workgroups wait only for GEMV workgroups, which come
// first in the grid and never wait.
// With rt_plan_attention_combine (at.out set) the P attention workgroups of KV group kh
// share the group's combine: peer r = hp S + s takes the chunks of 32 outputs r, r + P, ..
// (< Gq HD / 32), one output per thread (chunk i on threads [32 i, 32 i + 32): the host
// allows the combine where they fit the workgroup's live threads).  A thread reads its output's partial value and the
// (m, z) of every block of its head from the tagged copies, polling (bounded) until every
// word carries the launch's epoch, combines them in the operation order of
// attn_combine_element and writes the output and, per chunk, the f64 sum of the squares of
// its 32 outputs (for an RMSNORM_SSQ prologue).  A workgroup waits only for its peers'
// partials, which every peer stores before any wait of its own; the host allows the combine
// only when the device holds the whole grid at once.
template <int HD>
__device__ __forceinline__ void attn_peer_combine(const AttnTail& at, int kh, int r, unsigned ep) {
    const int S = at.S, NC = at.Gq * HD / 32, P = S * (at.Gq / at.hpw);  // P: workgroups of a KV group
    const int t = (int)threadIdx.x;
    if (r + 2 * (t >> 6) * P >= NC) return;  // waves past the workgroup's chunks (no barrier follows)
    const int c = r + (t >> 5) * P;
    const bool act = c < NC;  // lanes of a chunk past the group re-read the last one's words
    const int e = min(c, NC - 1) * 32 + (t & 31);
    const int hg = e / HD, d = e % HD, h = kh * at.Gq + hg;
    const unsigned long long* ph = at.ptag + (size_t)h * S * (HD + 2);
    auto ld = [](const unsigned long long* q) {
        return __hip_atomic_load(q, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    };
    float m[kAttnSMax], z[kAttnSMax], p[kAttnSMax];
    for (unsigned it = 0;; ++it) {
        bool ok = true;
#pragma unroll
        for (int sb = 0; sb < kAttnSMax; ++sb) {  // blocks past S re-read block S - 1
            const unsigned long long* q = ph + (size_t)min(sb, S - 1) * (HD + 2);
            const unsigned long long wv = ld(q + d), wm = ld(q + HD), wz = ld(q + HD + 1);
            ok &= (unsigned)(wv >> 32) == ep && (unsigned)(wm >> 32) == ep && (unsigned)(wz >> 32) == ep;
            p[sb] = __uint_as_float((unsigned)wv);
            m[sb] = __uint_as_float((unsigned)wm);
            z[sb] = __uint_as_float((unsigned)wz);
        }
        if (__all(ok)) break;
        if (it >= kAttnSpinLimit) {  // never expected: counted, and the launch goes on
            if (t == 0) __hip_atomic_fetch_add(at.err, 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
            break;
        }
        __builtin_amdgcn_s_sleep(1);
    }
    float mx = -INFINITY;
#pragma unroll
    for (int sb = 0; sb < kAttnSMax; ++sb)
        if (sb < S) mx = fmaxf(mx, m[sb]);
    // the factors expf(m_sb - mx) are the same for the 32 outputs of a chunk (one head): lane
    // sb of the chunk computes block sb's, and every lane takes them from there
    const int cl = t & 31, cbase = t & 32;
    float mj = m[0];
#pragma unroll
    for (int sb = 1; sb < kAttnSMax; ++sb) mj = cl == sb ? m[sb] : mj;
    const float fj = expf(mj - mx);
    float f[kAttnSMax];
#pragma unroll
    for (int sb = 0; sb < kAttnSMax; ++sb) f[sb] = __shfl(fj, cbase + sb, 64);
    float num = 0.0f, den = 0.0f;
#pragma unroll
    for (int sb = 0; sb < kAttnSMax; ++sb) {
        if (sb >= S || m[sb] == -INFINITY) continue;
        num = fmaf(f[sb], p[sb], num);
        den = fmaf(f[sb], z[sb], den);
    }
    const float o = num / den;
    const int k = h * HD + d;
    if (act) at.out[k] = o;
    // lanes 0..31 and 32..63 of the wave: 32 consecutive outputs each
    const double ss = half_reduce31((double)o * (double)o, 0.0, [](double x, double y) { return x + y; });
    if (act && (t & 31) == 31) at.ssq[k >> 5] = ss;
}

template <int HD>
__device__ __forceinline__ void qkv_attn_block(const AttnTail& at, int total_rb) {
    extern __shared__ __attribute__((aligned(16))) int red[];
    // attention workgroup i: KV group kh, peer r = hp S + s in the group (key block s, query
    // heads [hp hpw, hp hpw + hpw) of the group), one 256-thread tile per head; the waves past
    // them end here, before any barrier
    const int i = (int)blockIdx.x - total_rb, P = at.S * (at.Gq / at.hpw);
    const int kh = i / P, r = i - kh * P, hp = r / at.S, s = r - hp * at.S;
    const int sub = (int)(threadIdx.x >> 8), t = (int)(threadIdx.x & 255);
    if (sub >= at.hpw) return;
    const int h0 = kh * at.Gq + hp * at.hpw, h = h0 + sub;
    const AttnLdsPtr<HD> sm = (AttnLdsPtr<HD>)red;
    typedef __attribute__((address_space(3))) float lfl;
    lfl* const qkv = (lfl*)(sm + at.hpw);  // the heads' q (hpw HD), the group's k (HD), v (HD)
    const int j0 = s * kAttnBlock;
    const int nin = (at.hpw + 2) * HD;
    AttnKV<HD> kv;
    attn_kv_load<HD>(at.Kc, at.Vc, kh, j0, at.Lmax, t, kv);
    const unsigned ep = attn_epoch(at);
    const int pos = *at.pos;
    float* wp = at.work + ((size_t)h * at.S + s) * (HD + 2);
    // with the combine in this launch the partials are also stored as tagged words
    unsigned long long* wt = at.out ? at.ptag + ((size_t)h * at.S + s) * (HD + 2) : nullptr;
    const unsigned long long tag = (unsigned long long)ep << 32;
    const bool live = pos >= j0;
    if (live) {
        float c, sn;
        attn_rope_load<HD>(at.rope, pos, t, c, sn);
        const int e = (int)threadIdx.x;
        if (e < nin) {  // waves whose lanes all hold a value of the heads or the group (nin % 64 == 0)
            const int g = e < at.hpw * HD ? h0 * HD + e
                                          : at.qrows + (e < (at.hpw + 1) * HD ? 0 : at.nkv) + kh * HD +
                                                (e - at.hpw * HD) % HD;
            unsigned it = 0;
            unsigned long long w;
            while (true) {
                w = __hip_atomic_load(at.tagged + g, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
                if (__all((unsigned)(w >> 32) == ep)) break;
                if (++it > kAttnSpinLimit) {  // never expected: counted, and the launch goes on
                    if ((threadIdx.x & 63) == 0) __hip_atomic_fetch_add(at.err, 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
                    break;
                }
                __builtin_amdgcn_s_sleep(1);
            }
            qkv[e] = __uint_as_float((unsigned)w);
        }
        __syncthreads();
        // one writer of the new key and value per KV group: the group's last head
        attn_tile<HD, true, true>(qkv + sub * HD, qkv + at.hpw * HD, qkv + (at.hpw + 1) * HD, c, sn, at.Kc, at.Vc,
                                  kh, h == kh * at.Gq + at.Gq - 1, at.Lmax, pos, j0, at.scale, wp, wt, tag, t,
                                  sm + sub, kv);
    } else {
        attn_tile_empty<HD, true>(wp, wt, tag, t);
    }
    if (at.out) attn_peer_combine<HD>(at, kh, r, ep);
    // this workgroup is past its reads of the launch's tagged words: count it (the epoch of
    // the next launch follows from the count; no result to wait for)
    if (threadIdx.x == 0) (void)__builtin_amdgcn_atomic_inc32(at.done, at.wrap, __ATOMIC_RELAXED, "agent");
}

GemvShape gemv_shape_fused(int total_rb, int min_C) {
    // the prologue needs one row block per workgroup (KSPLIT), whatever the size
    int nw = (2048 + total_rb - 1) / total_rb;
    if (nw > 16) nw = 16;
    if (nw > min_C / 2) nw = min_C / 2;
    if (nw < 1) nw = 1;
    return GemvShape{true, nw};
}

GemvShape gemv_shape(int total_rb, int m_blocks, int min_C) {
    // Enough waves to fill 256 CUs x 8 waves; split K only when rows alone cannot.
    const long long waves_rows = (long long)total_rb * m_blocks;
    GemvShape s;
    if (waves_rows >= 1024 || min_C < 4) {
        s.ksplit = false;
        s.nw = 4;
        return s;
    }
    int nw = (int)((2048 + waves_rows - 1) / waves_rows);
    if (nw > 16) nw = 16;
    if (nw > min_C / 2) nw = min_C / 2;
    s.ksplit = nw > 1;
    s.nw = s.ksplit ? nw : 4;
    return s;
}

static bool aligned16(const void* p) { return ((uintptr_t)p & 15u) == 0; }

int vec_elements(int K, int threads) {
    // the smallest E whose live waves stay within kVecLiveWaves (per-element work is the same
    // for every E; each live wave adds the prologue's per-wave work: reductions, norm, scale),
    // else the E with the fewest live waves
    if (K <= 0 || K % 64) return 0;
    for (int E : {4, 8, 16})
        if (K / E <= threads && (K / E + 63) / 64 <= kVecLiveWaves) return E;
    return K / 16 <= threads ? 16 : 0;
}

// One KSPLIT launch of nw waves per workgroup; the leading scalar arguments are the
// prologue source's fields (zeros without a prologue), the shape word (nw <= 16, the inline
// problem count and the chunks per row of a one-problem launch, C <= 2^16), nw's reciprocal
// and the weight tiles of a one-problem launch (null otherwise).
static_assert(kInlineProbs <= 7, "the inline problem count takes 3 bits of the shape word");
template <int MT, int PRO, bool PAIR = false>
static void launch_ksplit(dim3 grid, int nw, size_t lds, hipStream_t s, const GemvArgs& a) {
    const QuantProb& P = a.pro;
    const bool one = a.ninl == 1;
    const unsigned shape = (unsigned)nw | ((unsigned)a.ninl << 5) | (one ? (unsigned)a.inl[0].C << 8 : 0u);
    hipLaunchKernelGGL((gemv_ksplit_kernel<MT, PRO, PAIR>), grid, dim3((unsigned)(64 * nw)), lds, s, P.x, P.aux, P.aux2,
                       P.K, P.mode, P.eps, shape, nw_reciprocal(nw), one ? a.inl[0].w : nullptr, a, NoTail{});
}

hipError_t launch_gemv(const GemvArgs& args, int mt, GemvShape shape, hipStream_t s) {
    if (args.total_rb <= 0 || args.M <= 0) return hipSuccess;
    // the leading weight-stream table: the inline problems, or the one problem of a
    // single-problem launch as an inline problem
    GemvArgs a = args;
    if (a.ninl == 0 && !a.dev) {
        a.ninl = 1;
        a.inl[0] = a.p;
    }
    for (int j = 0; j < kInlineProbs; ++j)
        a.inw[j] = j < a.ninl ? GemvWeights{a.inl[j].w, a.inl[j].C, a.inl[j].wg_begin} : GemvWeights{nullptr, 0, 0};
    const unsigned mblocks = (unsigned)((a.M + mt - 1) / mt);
    const dim3 block((unsigned)(64 * shape.nw));
    if (a.has_pro == 2) {  // single token, each problem's own row quantised in the prologue: ROWS
        if (mt != 1 || a.M != 1 || shape.ksplit || a.total_rb % shape.nw) return hipErrorInvalidValue;
        const dim3 grid((unsigned)(a.total_rb / shape.nw), 1);
        const size_t lds = (size_t)a.pro.Kp + sizeof(RowSmem);  // pro.Kp: the largest Kp of the problems
        hipLaunchKernelGGL((gemv_rows_kernel<1, 1>), grid, block, lds, s, a);
    } else if (a.has_pro && a.pair_a) {  // gate/up pair: an E-element prologue
        const QuantProb& P = a.pro;
        const int E = vec_elements(P.K, 64 * shape.nw);
        if (mt != 1 || a.M != 1 || !shape.ksplit || P.K % 64 || !aligned16(P.x) || !aligned16(P.aux) ||
            !aligned16(P.aux2) || E == 0)
            return hipErrorInvalidValue;
        const dim3 grid((unsigned)a.total_rb, 1);
        const size_t lds = (size_t)shape.nw * kRowBlock * sizeof(int) + (size_t)P.Kp + sizeof(RowSmem);
        if (E == 4) launch_ksplit<1, 3, true>(grid, shape.nw, lds, s, a);
        else if (E == 8) launch_ksplit<1, 4, true>(grid, shape.nw, lds, s, a);
        else launch_ksplit<1, 6, true>(grid, shape.nw, lds, s, a);
    } else if (a.has_pro) {  // single token, prologue-quantised input: KSPLIT shape only
        if (mt != 1 || a.M != 1 || !shape.ksplit) return hipErrorInvalidValue;
        const dim3 grid((unsigned)a.total_rb, 1);
        const QuantProb& P = a.pro;
        const int nw = a.pro.mode == kAttnNorm ? std::min(shape.nw, kAttnMaxThreads / 64) : shape.nw;
        size_t lds = (size_t)nw * kRowBlock * sizeof(int) + (size_t)a.pro.Kp + sizeof(RowSmem);
        const bool vec = P.K % 64 == 0 && aligned16(P.x) && aligned16(P.aux) && aligned16(P.aux2);
        if (a.pro.mode == kAttnNorm) {
            lds += (size_t)(a.pro.K / a.pro.attn_hd) * (a.pro.attn_S + 1) * sizeof(float);
            launch_ksplit<1, 2>(grid, nw, lds, s, a);
        } else if (const int E = vec ? vec_elements(P.K, (int)block.x) : 0) {
            if (E == 4) launch_ksplit<1, 3>(grid, nw, lds, s, a);
            else if (E == 8) launch_ksplit<1, 4>(grid, nw, lds, s, a);
            else launch_ksplit<1, 6>(grid, nw, lds, s, a);
        } else {
            launch_ksplit<1, 1>(grid, nw, lds, s, a);
        }
    } else if (shape.ksplit) {
        const dim3 grid((unsigned)a.total_rb, mblocks);
        const size_t lds = (size_t)shape.nw * mt * kRowBlock * sizeof(int);
        switch (mt) {
            case 1: launch_ksplit<1, 0>(grid, shape.nw, lds, s, a); break;
            case 2: launch_ksplit<2, 0>(grid, shape.nw, lds, s, a); break;
            case 4: launch_ksplit<4, 0>(grid, shape.nw, lds, s, a); break;
            case 8: launch_ksplit<8, 0>(grid, shape.nw, lds, s, a); break;
            default: return hipErrorInvalidValue;
        }
    } else {
        const dim3 grid((unsigned)((a.total_rb + shape.nw - 1) / shape.nw), mblocks);
        switch (mt) {
            case 1: hipLaunchKernelGGL((gemv_rows_kernel<1, 0>), grid, block, 0, s, a); break;
            case 2: hipLaunchKernelGGL((gemv_rows_kernel<2, 0>), grid, block, 0, s, a); break;
            case 4: hipLaunchKernelGGL((gemv_rows_kernel<4, 0>), grid, block, 0, s, a); break;
            case 8: hipLaunchKernelGGL((gemv_rows_kernel<8, 0>), grid, block, 0, s, a); break;
            default: return hipErrorInvalidValue;
        }
    }
    return hipGetLastError();
}

template <int PRO>
static void launch_qkv_attn(dim3 grid, int nw, size_t lds, hipStream_t s, const GemvArgs& a, const AttnTail& at) {
    const QuantProb& P = a.pro;
    const unsigned shape = (unsigned)nw | ((unsigned)a.ninl << 5) | ((unsigned)a.total_rb << 8);
    hipLaunchKernelGGL((gemv_ksplit_kernel<1, PRO, false, AttnTail>), grid, dim3((unsigned)(64 * nw)), lds, s, P.x,
                       P.aux, P.aux2, P.K, P.mode, P.eps, shape, nw_reciprocal(nw), static_cast<const v4u*>(nullptr),
                       a, at);
}

hipError_t launch_gemv_attn(const GemvArgs& args, const AttnTail& at, int Hkv, int hd, GemvShape shape,
                            hipStream_t s) {
    GemvArgs a = args;
    for (int j = 0; j < kInlineProbs; ++j)
        a.inw[j] = j < a.ninl ? GemvWeights{a.inl[j].w, a.inl[j].C, a.inl[j].wg_begin} : GemvWeights{nullptr, 0, 0};
    const QuantProb& P = a.pro;
    const int nw = shape.nw;
    // the shapes the kernel assumes: three inline problems over one RMSNorm-quantised row,
    // one row block per workgroup, a 256-thread tile per query head of a KV group, groups of
    // whole row blocks; an attention workgroup's live threads (256 hpw) hold its poll's
    // (hpw + 2) hd values, so hpw >= 2 at hd = 128
    const bool vec = P.K % 64 == 0 && aligned16(P.x) && aligned16(P.aux) && aligned16(P.aux2);
    const int E = vec ? vec_elements(P.K, 64 * nw) : 0;
    if (a.has_pro != 1 || a.M != 1 || a.out_i32 || a.pair_a || a.ninl != 3 || !shape.ksplit ||
        E == 0 || P.mode == kAttnNorm || hd != 128 || 64 * nw != 256 * at.Gq ||
        at.qrows != at.Gq * Hkv * hd || at.nkv != Hkv * hd || a.inl[0].N != at.qrows || a.inl[1].N != at.nkv ||
        a.inl[2].N != at.nkv || a.inl[1].wg_begin * kRowBlock != at.qrows ||
        a.inl[2].wg_begin * kRowBlock != at.qrows + at.nkv || at.S <= 0 || at.S != attn_splits(at.Lmax) ||
        at.hpw < 2 || at.Gq % at.hpw || at.natt != (unsigned)(Hkv * at.S * (at.Gq / at.hpw)))
        return hipErrorInvalidValue;
    const dim3 grid((unsigned)(a.total_rb + (int)at.natt), 1);
    const size_t lds = std::max((size_t)nw * kRowBlock * sizeof(int) + (size_t)P.Kp + sizeof(RowSmem),
                                (size_t)at.Gq * sizeof(AttnTileLds<128>) + (size_t)(at.Gq + 2) * hd * sizeof(float));
    if (E == 4) launch_qkv_attn<3>(grid, nw, lds, s, a, at);
    else if (E == 8) launch_qkv_attn<4>(grid, nw, lds, s, a, at);
    else launch_qkv_attn<6>(grid, nw, lds, s, a, at);
    return hipGetLastError();
}

hipError_t gemv_attn_capacity(int K, int Kp, int nw, int Gq, int* workgroups) {
    *workgroups = 0;
    const int E = K % 64 == 0 ? vec_elements(K, 64 * nw) : 0;
    if (E == 0) return hipErrorInvalidValue;
    const size_t lds = std::max((size_t)nw * kRowBlock * sizeof(int) + (size_t)Kp + sizeof(RowSmem),
                                (size_t)Gq * sizeof(AttnTileLds<128>) + (size_t)(Gq + 2) * 128 * sizeof(float));
    const void* k = E == 4   ? reinterpret_cast<const void*>(&gemv_ksplit_kernel<1, 3, false, AttnTail>)
                    : E == 8 ? reinterpret_cast<const void*>(&gemv_ksplit_kernel<1, 4, false, AttnTail>)
                             : reinterpret_cast<const void*>(&gemv_ksplit_kernel<1, 6, false, AttnTail>);
    int per_cu = 0, dev = 0, cus = 0;
    hipError_t e = hipOccupancyMaxActiveBlocksPerMultiprocessor(&per_cu, k, 64 * nw, lds);
    if (e == hipSuccess) e = hipGetDevice(&dev);
    if (e == hipSuccess) e = hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev);
    if (e == hipSuccess) *workgroups = per_cu * cus;
    return e;
}


}  // namespace rt
