// Internal declarations shared by the HIP translation units of librotor_hip.so.
//
// Device layouts (all chosen for gfx950; the host-facing format is the rotor
// byte matrix [N][ceil(K/4)] described in include/rotor_hip.h):
//
//  * Weight tiles.  Kp = K rounded up to 64, C = Kp/64 "chunks" of 64 weights
//    (16 bytes) per row, Np = N rounded up to 64, Nb = Np/64 row blocks.  The
//    16-byte unit (rb, c, r) holds bytes [16c, 16c+16) of row 64*rb + r and
//    lives at unit index (rb*C + c)*64 + r.  A wave that owns row block rb and reads
//    chunk c therefore issues one fully coalesced 1 KiB load (lane r <- row r), and
//    the whole row block is one contiguous C KiB stream.
//    The element positions of the rotor bytes are kept (element j of a byte in bits
//    2j+1..2j), the 2-bit code is not: the device stores g = w + 1 (00 = -1, 01 = 0,
//    10 = +1), so that a field masked in place, read as an int8, is g or 4 g and one
//    v_dot4 gives sum g x = sum w x + sum x; the GEMV subtracts sum x (see
//    device_code).  Padding weights (k >= K, rows >= N) are 01 (= 0).
//
//  * Quantised activations "qx".  Per token, Kp int8 values; inside every group of
//    16 consecutive k the bytes are stored in the order
//        x0 x4 x8 x12 | x1 x5 x9 x13 | x2 x6 x10 x14 | x3 x7 x11 x15
//    so that dword i of a group holds element i of each of the 4 weight bytes of the
//    matching weight dword: the decoded weight dword for field position i of a weight
//    dword pairs with activation dword i in one v_dot4_i32_i8.  Padding is 0.
//    Rows are padded with zeros to a multiple of the GEMV's tokens per workgroup.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include <string>

namespace rt {

typedef unsigned v4u __attribute__((ext_vector_type(4)));

constexpr int kRowBlock = 64;   // rows per weight tile (one per lane)
constexpr int kChunk = 64;      // weights per 16-byte chunk
// Zeroed bytes allocated after every weight tile buffer.  The GEMV issues its next
// loads before it knows whether the range has ended; those loads are range-checked
// by the buffer unit (and return zeros), and this slack keeps them inside the
// allocation even so.
constexpr size_t kTileSlack = 16384;

inline int round_up(int a, int b) { return (a + b - 1) / b * b; }

// MI355X: 8 XCDs, each with its own L2; workgroups are dealt to them round-robin by
// blockIdx.  xcd_order maps blockIdx.x to a workgroup index such that each XCD runs one
// contiguous range of indices (a bijection on [0, gridDim.x)).
constexpr int kXcds = 8;
__device__ __forceinline__ int xcd_order(int L, int n) {
    const int xcd = L % kXcds, base = n / kXcds, rem = n % kXcds;
    return xcd * base + min(xcd, rem) + L / kXcds;
}

// Rotor code (per 2-bit field: high bit = bit0, low bit = bit1, w = bit0 - bit1;
// src/rotor/core.py:99-108) <-> device code g = w + 1, 16 fields per dword at once.
// Rotor 00 -> 01, 10 -> 10, 01 -> 00 and the reserved 11 (w = 0) -> 01; back, 01 -> 00,
// so a reserved 11 returns as the canonical 00.
__host__ __device__ inline unsigned device_code(unsigned r) {
    const unsigned b0 = (r >> 1) & 0x55555555u, b1 = r & 0x55555555u;
    const unsigned hi = b0 & ~b1, lo = ~(b0 ^ b1) & 0x55555555u;
    return (hi << 1) | lo;
}
__host__ __device__ inline unsigned rotor_code(unsigned g) {
    const unsigned hi = (g >> 1) & 0x55555555u, lo = g & 0x55555555u;
    return (hi << 1) | (~hi & ~lo & 0x55555555u);
}

// ---- one quantisation problem (-> qx, sx) -----------------------------------------
// The value quantised for element k of a row depends on `mode`:
//   kQuant    v = x[k]
//   kPermute  q = q_in[k] taken as is (no quantisation, s = 1)
//   kRmsNorm  v = (x[k] / sqrt(mean_k x^2 + eps)) * norm_w[k], mean accumulated in f64
//   kRelu2Mul v = x[k] > 0 ? (x[k] * x[k]) * u[k] : 0        (x = gate, u = up)
//   kRelu2MulNorm  v = RMSNorm(relu2mul(x, u)) * norm_w       (norm_w = aux2)
//   kAttnNorm v = RMSNorm(combined decode-attention partials x) * norm_w (aux),
//             partials [K/hd heads][S][hd + 2]  (one token only)
//   kRmsNormSsq  as kRmsNorm, with sum_k x^2 also given as K/32 f64 partial sums in aux2
//             (cast; the `ssq` output of a gate/up pair plan): the 4- and 8-element
//             prologues add those up instead of reducing x over the workgroup; every
//             other path ignores them and reduces x itself
enum QuantMode { kQuant = 0, kPermute = 1, kRmsNorm = 2, kRelu2Mul = 3, kRelu2MulNorm = 4, kAttnNorm = 5,
                 kRmsNormSsq = 6 };

struct QuantProb {
    const float* x;      // fp32 [M][K] (gate in kRelu2Mul)
    const int8_t* q_in;  // int8 [M][K] (kPermute)
    int8_t* qx;          // [Mpad][Kp]
    float* sx;           // [Mpad]
    int8_t* q_nat;       // optional natural-order q [M][K]
    int K, Kp;
    int mode;
    const float* aux;    // norm_w [K] (kRmsNorm) or up [M][K] (kRelu2Mul)
    float eps;
    float* v_out;        // optional fp32 [M][K]: the values that were quantised
    const float* aux2;   // norm_w [K] (kRelu2MulNorm)
    int attn_S, attn_hd; // kAttnNorm: partial blocks per head, head dimension
    int blocked;         // qx layout: 0 rows, 1 blocked (see qx_blocked)
};

// ---- one GEMV problem (a ternary matrix applied to M tokens) -------------------
struct GemvProb {
    const v4u* w;        // weight tiles
    const int8_t* qx;    // quantised activations [Mpad][Kp] (layout above)
    const float* sx;     // [Mpad] per-token scales (unused for int32 output)
    const float* rs;     // [N] per-row scales or nullptr (then s_w)
    void* out;           // float y[M][ldo] or int32 acc[M][ldo]
    float s_w;
    int N, C, ldo;
    int wg_begin;        // first global row block of this problem (prefix sum over problems)
    const float* res;    // optional fp32 [M][ldo] added to y (may alias out)
    const float* xs;     // has_pro == 2: the problem's own fp32 input row [K] (quantised in the prologue)
    int K;               // has_pro == 2: its length
};

// Plans of up to this many problems carry their descriptors in the kernel arguments
// (GemvArgs::inl): the workgroup finds its problem by comparing its row block with the
// problems' wg_begin, with no dependent loads from a descriptor table.
constexpr int kInlineProbs = 4;

// What a GEMV workgroup needs before it can issue its first weight loads: its problem's
// weight tiles, chunks per row and first global row block.
struct GemvWeights {
    const v4u* w;
    int C, wg_begin;
};

struct GemvArgs {
    // the weight streams of the inline problems and their count lead the arguments, so one
    // scalar load brings in all a workgroup needs to start streaming its weights
    GemvWeights inw[kInlineProbs];
    int ninl;             // > 0: the G = ninl problems are inl[] (dev and rb2p unused)
    const GemvProb* dev;  // device descriptor array [G] (plans) or nullptr -> p
    const int* rb2p;      // [total_rb] problem index of every global row block (plans)
    int G, M, out_i32;
    int total_rb;         // row blocks over all problems
    GemvProb p;           // the problem of a single-problem launch
    int has_pro;          // M = 1: every workgroup quantises its input row into LDS first:
                          // 1 the shared row `pro` (KSPLIT), 2 its problem's xs (ROWS, plain absmax)
    QuantProb pro;        // has_pro == 1: source row of the prologue (mode, x, aux, aux2, eps, K, Kp)
    GemvProb inl[kInlineProbs];
    // gate/up pair (KSPLIT, has_pro == 1, one problem whose rows interleave gate and up in
    // groups of 32): row block j writes, instead of y, pair_a[32 j + r] = relu(g)^2 * u of
    // its rows r and 32 + r, pair_ssq[j] = sum over those 32 of (double) a^2, and g, u to
    // pair_g, pair_u when they are not null
    float* pair_a;
    double* pair_ssq;
    float* pair_g;
    float* pair_u;
    float pair_sg, pair_su;  // the gate and up scales
    // one-token plans with a prologue and fp32 outputs: out_ssq[j] = sum over outputs
    // 32 j .. 32 j + 31 of (double) y^2 (rt_plan_set_output_ssq), when not null
    double* out_ssq;
};

// Attention partials in the qkv GEMV's launch (gemv_ksplit_kernel with an AttnTail): the
// GEMV workgroups also store every output y of the q, k and v problems (concatenated, row
// n of the launch at index n) as tagged[n] = epoch << 32 | bits(y), a 64-bit
// device-coherent store; the natt = Hkv * S * Gq / hpw attention workgroups (hpw query heads
// of a KV group and one key block each) poll their heads' q and the group's k and v words
// until every one carries the epoch (bounded; err counts the waits that gave up,
// never expected).  Each attention workgroup adds one to *done when it has finished, without
// waiting for the result, and a launch's epoch is *done / natt + 1, read by every workgroup
// at its start: the count grows by natt per launch and reaches the next multiple only when
// every attention workgroup of the launch has finished, after every workgroup read it (the
// GEMV workgroups before storing the outputs all attention workgroups wait for), so the
// epoch is the same throughout a launch and the next launch's tags differ.  The count wraps
// to 0 after wrap (a wrapping increment), wrap + 1 being the largest multiple of natt below
// 2^32, so every launch starts on a multiple of natt; epochs repeat only after
// (wrap + 1) / natt launches, long after any word of theirs was overwritten.
constexpr unsigned kAttnSpinLimit = 1u << 18;
struct AttnTail {
    unsigned long long* tagged;  // [H hd + 2 Hkv hd]
    unsigned* done;              // [1]
    int* err;                    // [1]
    unsigned natt;               // Hkv S Gq / hpw: the attention workgroups of a launch
    unsigned wrap;               // natt floor((2^32 - 1) / natt) - 1
    float* Kc;                   // [Hkv][hd][Lmax]
    float* Vc;                   // [Hkv][Lmax][hd]
    const float* rope;
    const int* pos;
    float* work;                 // partials [H][S][hd + 2]
    int Gq, Lmax, S, nkv;        // nkv = Hkv hd: where k starts after q (H hd), v after k
    int hpw;                     // query heads per attention workgroup (Gq / hpw of them per key block)
    int qrows;                   // H hd
    float scale;
    // rt_plan_attention_combine (out != nullptr, S <= kAttnSMax): the attention workgroups
    // also store their partials as tagged words ptag [H][S][hd + 2] (epoch << 32 | bits),
    // and the S Gq / hpw workgroups of KV group kh share its combine: each polls the partials
    // of its share of the group's outputs, combines them into out [H hd] and writes per 32 outputs
    // the f64 sum of their squares into ssq [H hd / 32]
    float* out;
    double* ssq;
    unsigned long long* ptag;
};

struct GemvShape {
    bool ksplit;  // true: one row block per workgroup, waves split K
    int nw;       // waves per workgroup
};

struct QuantArgs {
    const QuantProb* dev;  // device descriptor array [U] or nullptr -> p
    int U, M, Mpad;
    QuantProb p;
};

// ---- one GEMM problem (int8 MFMA path, M > kGemvMaxM) ---------------------------
struct GemmArgs {
    const v4u* w;        // weight tiles (Np rows, C chunks)
    const int8_t* qx;    // [Mpad][Kp], Mpad a multiple of gemm_bm(M)
    const float* sx;     // [Mpad]
    const float* rs;     // [N] per-row scales or nullptr (then s_w)
    void* out;           // float y[M][ldo] or int32 acc[M][ldo]
    float s_w;
    int M, N, Np, C, ldo, out_i32;
    const float* res;    // optional fp32 [M][ldo] added to y (may alias out)
    int wg_begin;        // grouped launches: first global row block of this problem
    // Split-K launches (M <= 64) may cut a long-K problem into `parts` descriptors, part kp
    // covering chunks [c0, c1) (c1 == 0: all C, unsplit).  Each part's workgroup stores its
    // int32 64 x 64 tile in part_ws [parts][row blocks][64][64] and counts its arrival in
    // cnt [row blocks]; the last part of a row block sums the tiles, applies the epilogue
    // and resets the count to 0 for the next launch.
    int c0, c1, kp, parts;
    int* cnt;
    int* part_ws;
    // gate/up pair (tile GEMM, rt_plan_create_act_gate_up): the matrix interleaves gate and up
    // in groups of 32 rows (row 64 j + r: gate row 32 j + r for r < 32, up row 32 j + r - 32),
    // and the epilogue writes, instead of out, pair_a [M][ldo = N / 2] = relu(g)^2 * u with
    // g = ((float)acc * sx) * pair_sg and u likewise with pair_su
    float* pair_a;
    float pair_sg, pair_su;
};

constexpr int kBufDword3 = 0x00020000;  // buffer resource word 3 for gfx9 raw buffers

// Grouped GEMM launches of at most kGroupBounds + 1 descriptors pass the first unit of each
// descriptor after the first in their arguments (a unit then finds its descriptor without
// a table load)
constexpr int kGroupBounds = 15;

// Wave64 reductions on the DPP network: row_shr 1, 2, 4, 8 leave each 16-lane row's
// total in its lane 15, row_bcast 15 and 31 carry the row totals into lane 63, which
// ends up holding op over all 64 lanes (the other lanes hold partial results).  A lane
// whose DPP source does not exist takes `id`, op's identity.  Six dependent VALU steps,
// where a butterfly of __shfl_xor is six LDS round trips.
template <int CTRL, int ROWS>
__device__ __forceinline__ unsigned dpp_u32(unsigned v, unsigned id) {
    return (unsigned)__builtin_amdgcn_update_dpp((int)id, (int)v, CTRL, ROWS, 0xf, false);
}
template <int CTRL, int ROWS, typename T>
__device__ __forceinline__ T dpp_step(T v, T id) {
    if constexpr (sizeof(T) == 8) {
        const unsigned long long b = __builtin_bit_cast(unsigned long long, v),
                                 i = __builtin_bit_cast(unsigned long long, id);
        const unsigned lo = dpp_u32<CTRL, ROWS>((unsigned)b, (unsigned)i);
        const unsigned hi = dpp_u32<CTRL, ROWS>((unsigned)(b >> 32), (unsigned)(i >> 32));
        return __builtin_bit_cast(T, ((unsigned long long)hi << 32) | lo);
    } else {
        return __builtin_bit_cast(T, dpp_u32<CTRL, ROWS>(__builtin_bit_cast(unsigned, v),
                                                         __builtin_bit_cast(unsigned, id)));
    }
}
template <typename T, typename Op>
__device__ __forceinline__ T wave_reduce63(T v, T id, Op op) {
    v = op(v, dpp_step<0x111, 0xf>(v, id));  // row_shr:1
    v = op(v, dpp_step<0x112, 0xf>(v, id));  // row_shr:2
    v = op(v, dpp_step<0x114, 0xf>(v, id));  // row_shr:4
    v = op(v, dpp_step<0x118, 0xf>(v, id));  // row_shr:8
    v = op(v, dpp_step<0x142, 0xa>(v, id));  // row_bcast:15 into rows 1, 3
    v = op(v, dpp_step<0x143, 0xc>(v, id));  // row_bcast:31 into rows 2, 3
    return v;
}
// The first five steps of wave_reduce63 (up to row_bcast 15): lane 31 holds op over
// lanes 0..31 and lane 63 op over lanes 32..63.
template <typename T, typename Op>
__device__ __forceinline__ T half_reduce31(T v, T id, Op op) {
    v = op(v, dpp_step<0x111, 0xf>(v, id));  // row_shr:1
    v = op(v, dpp_step<0x112, 0xf>(v, id));  // row_shr:2
    v = op(v, dpp_step<0x114, 0xf>(v, id));  // row_shr:4
    v = op(v, dpp_step<0x118, 0xf>(v, id));  // row_shr:8
    v = op(v, dpp_step<0x142, 0xa>(v, id));  // row_bcast:15 into rows 1, 3
    return v;
}
// value of v in lane `lane` (wave-uniform), returned to every lane (through an SGPR)
template <typename T>
__device__ __forceinline__ T read_lane(T v, int lane) {
    if constexpr (sizeof(T) == 8) {
        const unsigned long long b = __builtin_bit_cast(unsigned long long, v);
        const unsigned lo = (unsigned)__builtin_amdgcn_readlane((int)(unsigned)b, lane);
        const unsigned hi = (unsigned)__builtin_amdgcn_readlane((int)(unsigned)(b >> 32), lane);
        return __builtin_bit_cast(T, ((unsigned long long)hi << 32) | lo);
    } else {
        return __builtin_bit_cast(T, __builtin_amdgcn_readlane(__builtin_bit_cast(int, v), lane));
    }
}
// the lane-63 total, returned to every lane (through an SGPR)
template <typename T>
__device__ __forceinline__ T lane63(T v) {
    return read_lane(v, 63);
}
__device__ __forceinline__ int wave_sum(int v) {
    return lane63(wave_reduce63(v, 0, [](int a, int b) { return a + b; }));
}
constexpr int kGemvMaxM = 8;  // up to this many tokens: VALU GEMV; beyond: MFMA GEMM
// qx layout.  Rows (M <= kGemvMaxM, read by the GEMV): row m at m * Kp.  Blocked
// (M > kGemvMaxM, read by the MFMA GEMM): 16-row x 64-k blocks of 1 KiB, block
// (m / 16, c) at (m / 16 * C + c) * 1024, where the 16-byte group q (k = 16 q .. 16 q + 15
// of chunk c) of row m sits at ((m % 16) + 16 q) * 16: the block is laid out as the
// matrix-core operand fragments, so the GEMM copies it to LDS with contiguous loads.
inline bool qx_blocked(int M) { return M > kGemvMaxM; }

// rows of the GEMM workgroup tile for M tokens (the activations are zero-padded to it)
inline int gemm_bm(int M) { return M <= 64 ? 64 : M <= 128 ? 128 : 256; }
// The GEMM epilogues address one row tile of the output (and residual) with 32-bit byte
// offsets and buffer ranges: a tile of gemm_bm(M) rows of ldo floats must span < 2^31 bytes.
inline bool gemm_ldo_ok(int M, int ldo) { return (long long)gemm_bm(M) * ldo * 4 < (1ll << 31); }

// Launchers (return hipSuccess or the launch error).
hipError_t launch_relayout(const uint8_t* src, int N, int K, v4u* tiles, hipStream_t s);
hipError_t launch_unrelayout(const v4u* tiles, int N, int K, uint8_t* dst, hipStream_t s);
// maxK > 0: every problem passes quant_rows_ok and maxK is their largest K (the
// vectorised row kernel); 0: the general kernel.
hipError_t launch_quant(const QuantArgs& a, hipStream_t s, int maxK = 0);
bool quant_rows_ok(const QuantProb& P);
// qx rows [M][Kp] (permuted) -> natural-order int8 [M][K]
hipError_t launch_unpermute(const int8_t* qx, int M, int K, int Kp, bool blocked, int8_t* q, hipStream_t s);
// mt = tokens per workgroup (1, 2, 4 or 8).
hipError_t launch_gemv(const GemvArgs& a, int mt, GemvShape shape, hipStream_t s);
hipError_t launch_gemm(const GemmArgs& a, hipStream_t s);
// Tile shapes of the MFMA GEMM for M > 64 (rows x columns per workgroup).  A launch over
// one or several problems (same M) takes 256 x 256 when that yields kGemmFillTiles tiles,
// else 192 x 128 when that yields kGemm192Min..kGemm192Max tiles (one round on the 256
// CUs: 2048 x 2560 x 6912 as 220 tiles runs 46.3 us against 49.5 us as 160 tiles of
// 256 x 128), else 256 x 128 when that yields kGemmHalfTiles (57 us as 320 tiles of
// 128 x 128), else 128 x 128 when that does, else 64 x 128 (measured on the 512-token
// prefill's projections: 4.95 ms against 5.30 ms with 128 x 128): a few large tiles leave
// most CUs idle.  192-row tiles do not divide the activations' 256-row padding: their
// loads of rows past it re-read the last padded block (see gemm_kernel).  Before all of
// these, launches whose problems are all at least kRegMinC chunks deep (K >= 4096) with an
// even chunk count (C[g], the two K halves of a region walk equal steps) and whose 128 x 160
// regions number kRegMinTiles..kRegMaxTiles take gemm_region_kernel.
enum GemmTileCfg {
    kTile128x128 = 0,
    kTile256x128 = 1,
    kTile256x256 = 2,
    kTile64x128 = 3,
    kTile192x128 = 4,
    kRegion128x160 = 5
};
constexpr int kGemmFillTiles = 192, kGemmHalfTiles = 128, kGemm192Min = 200, kGemm192Max = 256;
constexpr int kRegMinC = 64, kRegMinTiles = 224, kRegMaxTiles = 256;
inline int gemm_tile_bm(int cfg) {
    return cfg == kTile64x128 ? 64 : cfg == kTile128x128 || cfg == kRegion128x160 ? 128 : cfg == kTile192x128 ? 192 : 256;
}
inline int gemm_tile_bn(int cfg) { return cfg == kTile256x256 ? 256 : cfg == kRegion128x160 ? 160 : 128; }
int gemm_tile_cfg(int M, const int* N, const int* C, int G);
long long gemm_tile_count(int cfg, int M, int N);
// G problems with M > 64 in one tile launch: dev [G] (wg_begin = first tile of the
// problem), tile2p [total_tiles] problem of every tile, cfg from gemm_tile_cfg.
hipError_t launch_gemm_tiles(const GemmArgs* dev, const int* tile2p, const int* bnd, int nb, int total_tiles, int cfg,
                             hipStream_t s);
// M <= 64 (gemm_bm(M) == 64): G problems in one launch over all their row blocks;
// dev [G] (wg_begin set), rb2p [total_rb] problem of every global row block.
// The M = 1 qkv plan (three inline problems, E-element RMSNorm prologue, 256 Gq threads per
// workgroup) with the attention partials of its token in the same launch.
hipError_t launch_gemv_attn(const GemvArgs& args, const AttnTail& at, int Hkv, int hd, GemvShape shape,
                            hipStream_t s);
// Workgroups of that launch (source row of K elements, nw waves, Gq query heads per KV head)
// that the current device holds at once.
hipError_t gemv_attn_capacity(int K, int Kp, int nw, int Gq, int* workgroups);
hipError_t launch_gemm_group(const GemmArgs* dev, const int* rb2p, const int* bnd, int nb, int total_rb,
                             hipStream_t s);
// Once per device (current) before any launch: the function attributes the GEMM kernels
// and the prefill attention need (dynamic LDS above 64 KiB).
hipError_t gemm_prepare_device();
hipError_t model_prepare_device();

// model kernels (rt_model.hip)
hipError_t launch_embed(const uint16_t* E, const int* ids, int M, int V, int D, float* h, hipStream_t s);
hipError_t launch_rope_append(float* q, float* k, const float* v, float* Kc, float* Vc, const float* rope, int M,
                              int H, int Hkv, int hd, int Lmax, const int* pos, hipStream_t s);
hipError_t launch_attention(const float* q, const float* Kc, const float* Vc, float* out, int M, int H, int Hkv,
                            int hd, int Lmax, const int* pos, float scale, hipStream_t s);
// decode attention split over blocks of 64 keys: partials [H][S][hd + 2], S = attn_splits(Lmax)
inline int attn_splits(int Lmax) { return (Lmax + 63) / 64; }
// rope != nullptr: q/knew/vnew are the raw projection outputs of the token at *pos; the
// kernel applies RoPE, appends knew (rotated) and vnew to the caches and uses them for that
// key.  rope == nullptr: q is rotated and the caches already hold the token.
hipError_t launch_attn_partial(const float* q, const float* knew, const float* vnew, float* Kc, float* Vc,
                               const float* rope, int H, int Hkv, int hd, int Lmax, const int* pos, float scale,
                               float* work, hipStream_t s);
hipError_t launch_attn_combine(const float* work, int H, int hd, int S, float* out, hipStream_t s);
hipError_t launch_lm_head(const uint16_t* E, const float* x, const float* norm_w, float eps, int V, int D,
                          float* logits, unsigned long long* best, int* token, int* pos, int advance,
                          int* next_ids, int* out_tokens, int pos_base, int out_cap, float* next_h, hipStream_t s);

// Host policy: tokens per workgroup for M tokens.
inline int gemv_mt(int M) { return M <= 1 ? 1 : M <= 2 ? 2 : M <= 4 ? 4 : 8; }
// Host policy: launch shape so that small launches still fill the chip.
GemvShape gemv_shape(int total_rb, int m_blocks, int min_C);
// Launch shape of a plan whose GEMV quantises its input in the prologue (M = 1).
GemvShape gemv_shape_fused(int total_rb, int min_C);
// Elements per thread (4, 8 or 16) of the vectorised decode prologue for a row of K
// (K % 64 == 0) on `threads` threads, 0 when none fits.
constexpr int kVecLiveWaves = 16;  // measured: 4, 8 and 16 give the same decode time
int vec_elements(int K, int threads);

}  // namespace rt
