// Internal declarations shared by the HIP translation units of librotor_hip.so.
//
// Device layouts (all chosen for gfx950; the host-facing format is the rotor
// byte matrix [N][ceil(K/4)] described in include/rotor_hip.h):
//
//  * Weight tiles.  Kp = K rounded up to 64, C = Kp/64 "chunks" of 64 weights
//    (16 bytes) per row, Np = N rounded up to 64, Nb = Np/64 row blocks.  The
//    16-byte unit (rb, c, r) holds rotor bytes [16c, 16c+16) of row 64*rb + r and
//    lives at unit index (rb*C + c)*64 + r.  A wave that owns row block rb and reads
//    chunk c therefore issues one fully coalesced 1 KiB load (lane r <- row r), and
//    the whole row block is one contiguous C KiB stream.  Padding codes are 00 (= 0).
//
//  * Quantised activations "qx".  Per token, Kp int8 values; inside every group of
//    16 consecutive k the bytes are stored in the order
//        x0 x4 x8 x12 | x1 x5 x9 x13 | x2 x6 x10 x14 | x3 x7 x11 x15
//    so that dword i of a group holds element i of each of the 4 weight bytes of the
//    matching weight dword: the decoded weight dword for field position i of a weight
//    dword pairs with activation dword i in one v_dot4_i32_i8.  Padding is 0.
//    Rows are padded to a multiple of 8 tokens with zeros.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include <string>

namespace rt {

typedef unsigned v4u __attribute__((ext_vector_type(4)));

constexpr int kRowBlock = 64;   // rows per weight tile (one per lane)
constexpr int kChunk = 64;      // weights per 16-byte chunk
constexpr int kTokPad = 8;      // qx rows are padded to a multiple of this
constexpr int kMaxInline = 4;   // problems passed by value in kernel arguments

inline int round_up(int a, int b) { return (a + b - 1) / b * b; }

// ---- one GEMV problem (a ternary matrix applied to M tokens) -------------------
struct GemvProb {
    const v4u* w;        // weight tiles
    const int8_t* qx;    // quantised activations [Mpad][Kp] (layout above)
    const float* sx;     // [Mpad] per-token scales (unused for int32 output)
    const float* rs;     // [N] per-row scales or nullptr (then s_w)
    void* out;           // float y[M][ldo] or int32 acc[M][ldo]
    float s_w;
    int N, C, ldo;
    int wg_begin;        // first workgroup (blockIdx.x) of this problem
};

struct GemvArgs {
    const GemvProb* dev;  // device descriptor array (plans) or nullptr -> p[]
    int G, M, out_i32;
    GemvProb p[kMaxInline];
};

// ---- one quantisation problem (x fp32 [M][K] -> qx, sx) -------------------------
struct QuantProb {
    const float* x;      // fp32 [M][K]           (quantise mode)
    const int8_t* q_in;  // int8 [M][K]           (permute mode: no quantisation)
    int8_t* qx;          // [Mpad][Kp]
    float* sx;           // [Mpad]
    int8_t* q_nat;       // optional natural-order q [M][K]
    int K, Kp;
};

struct QuantArgs {
    const QuantProb* dev;
    int U, M, Mpad;
    QuantProb p[kMaxInline];
};

// Launchers (return hipSuccess or the launch error).
hipError_t launch_relayout(const uint8_t* src, int N, int K, v4u* tiles, hipStream_t s);
hipError_t launch_unrelayout(const v4u* tiles, int N, int K, uint8_t* dst, hipStream_t s);
hipError_t launch_quant(const QuantArgs& a, hipStream_t s);
// mt = tokens per workgroup (1, 2, 4 or 8), nw = waves per workgroup (K split).
hipError_t launch_gemv(const GemvArgs& a, int total_wgs, int mt, int nw, hipStream_t s);

// Host policy: tokens per workgroup for M tokens.
inline int gemv_mt(int M) { return M <= 1 ? 1 : M <= 2 ? 2 : M <= 4 ? 4 : 8; }
// Host policy: waves per workgroup so that small launches still fill the chip.
int gemv_waves(int total_wgs, int C);

}  // namespace rt
