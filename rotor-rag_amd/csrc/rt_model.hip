// Device kernels around the ternary linears for BitNet-2B-shape inference:
// embedding gather, RoPE + KV-cache append, causal GQA attention over the cache,
// bf16 LM head (fused final RMSNorm) with greedy argmax.
//
// Callers in the reference: BitNetModel.forward (src/rotor/bitnet_model.py:190-244:
// embedding :220, blocks :224-228, final norm :231, tied LM head :235),
// MultiHeadAttention.forward (src/rotor/transformer.py:206-292: KV concat :250-252,
// GQA repeat :260-263, scores/softmax/AV :267-281) and GreedySampling
// (src/rotor/generation.py:28-42).  This build's model adds RoPE and a causal mask (the
// benchmark configuration); the reference has neither.
//
// Floating-point contraction is off in this file so that a*b+c rounds twice, as the
// NumPy model of the tests computes it.
#include <algorithm>

#include "rt_rowquant.h"
#include "rt_attn_decode.h"

#pragma clang fp contract(off)

namespace rt {

__device__ __forceinline__ float bf16_to_f32(uint16_t b) { return __uint_as_float((unsigned)b << 16); }

// h[m][:] = E[ids[m]][:] (bf16 -> fp32)
__global__ void __launch_bounds__(256) embed_kernel(const uint16_t* __restrict__ E, const int* __restrict__ ids, int V,
                                                    int D, float* __restrict__ h) {
    const int m = blockIdx.x;
    int id = ids[m];
    if (id < 0 || id >= V) id = 0;  // the host validates ids; never read out of range
    const uint16_t* row = E + (size_t)id * D;
    for (int k = threadIdx.x; k < D; k += blockDim.x) h[(size_t)m * D + k] = bf16_to_f32(row[k]);
}

// RoPE (rotate-half convention) on q [M][H*hd] and k [M][Hkv*hd] in place for positions
// *pos_p + m, then k -> Kc [Hkv][hd][Lmax] (dimension-major), v -> Vc [Hkv][Lmax][hd].
// rope: [Lmax][hd/2][2] = (cos, sin) of position * theta_i.
__global__ void __launch_bounds__(256) rope_append_kernel(float* __restrict__ q, float* __restrict__ k,
                                                          const float* __restrict__ v, float* __restrict__ Kc,
                                                          float* __restrict__ Vc, const float* __restrict__ rope,
                                                          int H, int Hkv, int hd, int Lmax,
                                                          const int* __restrict__ pos_p) {
    const int m = blockIdx.x, pos = *pos_p + m, half = hd / 2;
    const float* cs = rope + (size_t)pos * half * 2;
    for (int idx = threadIdx.x; idx < (H + Hkv) * half; idx += blockDim.x) {
        const int head = idx / half, i = idx % half;
        float* base = head < H ? q + (size_t)m * H * hd + (size_t)head * hd
                               : k + (size_t)m * Hkv * hd + (size_t)(head - H) * hd;
        const float c = cs[2 * i], s = cs[2 * i + 1];
        const float x1 = base[i], x2 = base[i + half];
        base[i] = x1 * c - x2 * s;
        base[i + half] = x2 * c + x1 * s;
    }
    __syncthreads();
    for (int idx = threadIdx.x; idx < Hkv * hd; idx += blockDim.x) {
        const int kh = idx / hd, d = idx % hd;
        Kc[((size_t)kh * hd + d) * Lmax + pos] = k[(size_t)m * Hkv * hd + idx];
        Vc[((size_t)kh * Lmax + pos) * hd + d] = v[(size_t)m * Hkv * hd + idx];
    }
}

// out[m][h*hd + d] = sum_j softmax_j(q.K_j * scale) V_j[d] over keys j <= *pos_p + m.
// One 256-thread workgroup per (head, query); scores live in LDS (Lmax floats).
__global__ void __launch_bounds__(256) attention_kernel(const float* __restrict__ q, const float* __restrict__ Kc,
                                                        const float* __restrict__ Vc, float* __restrict__ out, int H,
                                                        int Hkv, int hd, int Lmax, const int* __restrict__ pos_p,
                                                        float scale) {
    extern __shared__ float smem[];  // [hd] q, [Lmax] scores, [256] reduction
    float* qs = smem;
    float* sc = smem + hd;
    float* red = sc + Lmax;
    const int h = blockIdx.x, m = blockIdx.y, t = threadIdx.x;
    const int kh = h / (H / Hkv), L = *pos_p + m + 1;
    for (int d = t; d < hd; d += 256) qs[d] = q[(size_t)m * H * hd + (size_t)h * hd + d];
    __syncthreads();
    const float* K = Kc + (size_t)kh * hd * Lmax;
    float mx = -INFINITY;
    for (int j = t; j < L; j += 256) {
        float dot = 0.0f;
        for (int d = 0; d < hd; ++d) dot += qs[d] * K[(size_t)d * Lmax + j];
        const float s = dot * scale;
        sc[j] = s;
        mx = fmaxf(mx, s);
    }
    red[t] = mx;
    __syncthreads();
    for (int w = 128; w > 0; w >>= 1) {
        if (t < w) red[t] = fmaxf(red[t], red[t + w]);
        __syncthreads();
    }
    mx = red[0];
    __syncthreads();
    float z = 0.0f;
    for (int j = t; j < L; j += 256) {
        const float p = expf(sc[j] - mx);
        sc[j] = p;
        z += p;
    }
    red[t] = z;
    __syncthreads();
    for (int w = 128; w > 0; w >>= 1) {
        if (t < w) red[t] += red[t + w];
        __syncthreads();
    }
    z = red[0];
    __syncthreads();
    // two halves of the workgroup take alternate keys, then combine
    const float* V = Vc + (size_t)kh * Lmax * hd;
    const int groups = 256 / hd;  // hd divides 256 (checked on the host)
    const int d = t % hd, gsub = t / hd;
    float acc = 0.0f;
    for (int j = gsub; j < L; j += groups) acc += sc[j] * V[(size_t)j * hd + d];
    red[t] = acc;
    __syncthreads();
    if (gsub == 0) {
        for (int g = 1; g < groups; ++g) acc += red[g * hd + d];
        out[(size_t)m * H * hd + (size_t)h * hd + d] = acc / z;
    }
}

// Prefill attention on the fp32 matrix cores (v_mfma_f32_32x32x2_f32, twice the VALU FMA
// rate).  Workgroup (kv head kh, query block) owns 32 rows r = i G + g (query i of the
// block, q-head g of the G = H / Hkv heads sharing kh); lane l of every wave works on row
// l % 32.  Its 4 waves take the visible keys in blocks of 32, wave w blocks w, w + 4, ..,
// each block staged in the wave's own LDS slice (K dimension-major as in the cache, V
// key-major), with an online softmax per wave:
//   S^T = K Q^T   (A = K[key][d] from LDS, B = Q^T from registers; the 128 dims are
//                  taken in 64 steps pairing d = s and d = 64 + s over the lane halves)
//   P^T = e^(S^T scale - m) per row, rows are lanes, so max and sum need one
//                  lane-half exchange
//   O^T += V^T P^T (A = V^T from LDS, B = P^T straight from the S^T registers: the
//                  MFMA output layout puts keys 8 (r / 4) + 4 (l / 32) + r % 4 of the
//                  lane's row in register r, and step r pairs exactly those keys)
// The 4 waves' (m, l, O) are merged through LDS at the end.  fp32 products, fp32 sums in
// the matrix cores' order.
typedef float v16f __attribute__((ext_vector_type(16)));
typedef __attribute__((address_space(3))) void lds_void;

template <int HD>
__global__ void __launch_bounds__(256) attn_prefill_mfma_kernel(const float* __restrict__ q,
                                                                const float* __restrict__ Kc,
                                                                const float* __restrict__ Vc, float* __restrict__ out,
                                                                int M, int H, int Hkv, int Lmax,
                                                                const int* __restrict__ pos_p, float scale) {
    static_assert(HD == 128, "two 64-dim halves per lane");
    constexpr int BK = 32, SLICE = HD * BK * 2;  // floats per wave: K [HD][BK], V [BK][HD]
    extern __shared__ __attribute__((aligned(16))) float lds_pf[];
    const int t = threadIdx.x, lane = t & 63, wave = t >> 6, row = lane & 31, hl = lane >> 5;
    const int G = H / Hkv, BQ = 32 / G;
    // the last query blocks see the most keys: they go out first, so that the short ones
    // fill in behind them when the grid takes more than one round of workgroups
    const int kh = blockIdx.x, i0 = ((int)gridDim.y - 1 - (int)blockIdx.y) * BQ;
    const int pos0 = *pos_p;
    const int m = i0 + row / G, hq = kh * G + row % G;
    const int lastpos = m < M ? pos0 + m : -1;     // keys <= lastpos visible to this row
    const int kend = pos0 + min(i0 + BQ, M);       // keys [0, kend) visible to some row
    const int nblk = (kend + BK - 1) / BK;
    float* Ks = lds_pf + wave * SLICE;
    float* Vs = Ks + HD * BK;
    // this lane's half of its row of Q: dims 64 hl .. 64 hl + 63
    float qr[64];
    {
        const float* qp = q + (size_t)min(m, M - 1) * H * HD + (size_t)hq * HD + 64 * hl;
#pragma unroll
        for (int i = 0; i < 16; ++i) {
            const float4 v4 = *reinterpret_cast<const float4*>(qp + 4 * i);
            qr[4 * i] = v4.x;
            qr[4 * i + 1] = v4.y;
            qr[4 * i + 2] = v4.z;
            qr[4 * i + 3] = v4.w;
        }
    }
    v16f o[HD / 32];
#pragma unroll
    for (int nb = 0; nb < HD / 32; ++nb) o[nb] = v16f{};
    float mrow = -INFINITY, lrow = 0.0f;
    const float* K = Kc + (size_t)kh * HD * Lmax;
    const float* V = Vc + (size_t)kh * Lmax * HD;
    // K and V blocks go global -> LDS directly (buffer loads with an LDS destination, range
    // checked per head: keys past Lmax read as zeros).  A block's K loads are issued as
    // soon as the previous block's K operands have been read out of the slice, its V loads
    // as soon as the previous V operands have: each has a whole block of MFMAs to land.
    // Keys past kend are masked below.
    const __amdgpu_buffer_rsrc_t krs =
        __builtin_amdgcn_make_buffer_rsrc((void*)K, 0, (unsigned)(HD * Lmax * 4), kBufDword3);
    const __amdgpu_buffer_rsrc_t vrs =
        __builtin_amdgcn_make_buffer_rsrc((void*)V, 0, (unsigned)(HD * Lmax * 4), kBufDword3);
    constexpr int kBlkLoads = HD * BK / 4 / 64;  // 16-byte loads per lane per block (16)
    auto load_k = [&](int key0) {  // Ks[d][j] = K[d][key0 + j], 8 dims per load
#pragma unroll
        for (int it = 0; it < kBlkLoads; ++it) {
            const int d = 8 * it + (lane >> 3), j = 4 * (lane & 7);
            __builtin_amdgcn_raw_ptr_buffer_load_lds(krs, (lds_void*)(Ks + 256 * it), 16, (d * Lmax + key0 + j) * 4, 0,
                                                     0, 0);
        }
    };
    auto load_v = [&](int key0) {  // Vs[j][d] = V[key0 + j][d], 2 keys per load
#pragma unroll
        for (int it = 0; it < kBlkLoads; ++it) {
            const int j = 2 * it + (lane >> 5), dq = 4 * (lane & 31);
            __builtin_amdgcn_raw_ptr_buffer_load_lds(vrs, (lds_void*)(Vs + 256 * it), 16, ((key0 + j) * HD + dq) * 4, 0,
                                                     0, 0);
        }
    };
    if (wave < nblk) {
        load_k(wave * BK);
        load_v(wave * BK);
    }
    for (int b = wave; b < nblk; b += 4) {
        const int key0 = b * BK;
        const bool more = b + 4 < nblk;
        // this block's K has landed (its V may still be in flight)
        asm volatile("s_waitcnt vmcnt(%0)" ::"n"(kBlkLoads) : "memory");
        // S^T[key][row]; the 64 A operands are read from LDS ahead of the MFMA chain (read
        // one by one in front of each MFMA, every pair of MFMAs would wait for the LDS)
        float ka[64];
#pragma unroll
        for (int st = 0; st < 64; ++st) ka[st] = Ks[(64 * hl + st) * BK + row];
        asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");  // K slice read out: refill it
        if (more) load_k((b + 4) * BK);
        __builtin_amdgcn_sched_barrier(0);  // keep the reads and loads ahead of the chain
        v16f sacc = v16f{};
#pragma unroll
        for (int st = 0; st < 64; ++st) sacc = __builtin_amdgcn_mfma_f32_32x32x2f32(ka[st], qr[st], sacc, 0, 0, 0);
        float pr[16];
        float mx = -INFINITY;
#pragma unroll
        for (int r = 0; r < 16; ++r) {
            const int key = key0 + 8 * (r >> 2) + 4 * hl + (r & 3);
            pr[r] = key <= lastpos ? sacc[r] * scale : -INFINITY;
            mx = fmaxf(mx, pr[r]);
        }
        mx = fmaxf(mx, __shfl_xor(mx, 32, 64));
        const float mnew = fmaxf(mrow, mx);
        const float alpha = mnew == -INFINITY ? 1.0f : expf(mrow - mnew);
        float ls = 0.0f;
#pragma unroll
        for (int r = 0; r < 16; ++r) {
            pr[r] = pr[r] == -INFINITY ? 0.0f : expf(pr[r] - mnew);
            ls += pr[r];
        }
        ls += __shfl_xor(ls, 32, 64);
        lrow = lrow * alpha + ls;
        mrow = mnew;
        // this block's V has landed (the next block's K may still be in flight)
        if (more) asm volatile("s_waitcnt vmcnt(%0)" ::"n"(kBlkLoads) : "memory");
        else asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
        // O^T[dim][row] = alpha O^T + V^T P^T (A operands read ahead, as above)
        float va[HD / 32][16];
#pragma unroll
        for (int nb = 0; nb < HD / 32; ++nb)
#pragma unroll
            for (int r = 0; r < 16; ++r) va[nb][r] = Vs[(8 * (r >> 2) + 4 * hl + (r & 3)) * HD + 32 * nb + row];
        asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");  // V slice read out: refill it
        if (more) load_v((b + 4) * BK);
        __builtin_amdgcn_sched_barrier(0);
#pragma unroll
        for (int nb = 0; nb < HD / 32; ++nb) {
            v16f acc = o[nb] * alpha;
#pragma unroll
            for (int r = 0; r < 16; ++r) acc = __builtin_amdgcn_mfma_f32_32x32x2f32(va[nb][r], pr[r], acc, 0, 0, 0);
            o[nb] = acc;
        }
    }
    // merge the waves: slice w becomes [32 rows][HD] of O^T, then (m, l) per row
    __syncthreads();
    float* Om = lds_pf + wave * SLICE;
    float* ml = lds_pf + 4 * SLICE;  // [4 waves][32 rows][2]
#pragma unroll
    for (int nb = 0; nb < HD / 32; ++nb)
#pragma unroll
        for (int r = 0; r < 16; ++r) Om[row * HD + 32 * nb + 8 * (r >> 2) + 4 * hl + (r & 3)] = o[nb][r];
    if (hl == 0) {
        ml[(wave * 32 + row) * 2] = mrow;
        ml[(wave * 32 + row) * 2 + 1] = lrow;
    }
    __syncthreads();
    const int orow = t >> 3, d0 = (t & 7) * (HD / 8);
    const int om = i0 + orow / G, oh = kh * G + orow % G;
    if (om >= M) return;
    float mw[4], fw[4], mmax = -INFINITY;
#pragma unroll
    for (int w = 0; w < 4; ++w) {
        mw[w] = ml[(w * 32 + orow) * 2];
        mmax = fmaxf(mmax, mw[w]);
    }
    float den = 0.0f;
#pragma unroll
    for (int w = 0; w < 4; ++w) {
        fw[w] = mw[w] == -INFINITY ? 0.0f : expf(mw[w] - mmax);
        den += fw[w] * ml[(w * 32 + orow) * 2 + 1];
    }
    float* dst = out + (size_t)om * H * HD + (size_t)oh * HD + d0;
#pragma unroll
    for (int e = 0; e < HD / 8; ++e) {
        float num = 0.0f;
#pragma unroll
        for (int w = 0; w < 4; ++w) num += fw[w] * lds_pf[w * SLICE + orow * HD + d0 + e];
        dst[e] = num / den;
    }
}

// Decode attention, split over the keys: workgroup (h, s) is the tile of query head h and
// key block s (rt_attn_decode.h), writing its partial to work[h][s][0..HD+2).
template <int HD, bool ROPE>
__global__ void __launch_bounds__(256) attn_partial_kernel(const float* __restrict__ q, const float* __restrict__ knew,
                                                           const float* __restrict__ vnew, float* __restrict__ Kc,
                                                           float* __restrict__ Vc, const float* __restrict__ rope,
                                                           int H, int Hkv, int Lmax, const int* __restrict__ pos_p,
                                                           float scale, float* __restrict__ work) {
    __shared__ AttnTileLds<HD> sm;
    // Workgroup (h, s) from an XCD-ordered index whose fastest part is the query head within
    // its KV group: the G heads that read one key block run on one XCD and share its L2
    // (decode 1.235 -> 1.218 ms/token against one workgroup per (blockIdx.x, blockIdx.y))
    const int S = gridDim.y, Gq = H / Hkv;
    const int w = xcd_order((int)(blockIdx.x + gridDim.x * blockIdx.y), (int)(gridDim.x * gridDim.y));
    const int kh = w / (Gq * S), s = (w / Gq) % S, h = kh * Gq + w % Gq, t = threadIdx.x;
    const int j0 = s * kAttnBlock;
    AttnKV<HD> kv;
    attn_kv_load<HD>(Kc, Vc, kh, j0, Lmax, t, kv);
    const int pos = *pos_p;
    float* wp = work + ((size_t)h * S + s) * (HD + 2);
    if (pos < j0) {
        attn_tile_empty<HD>(wp, nullptr, 0ull, t);
        return;
    }
    float c = 0.0f, sn = 0.0f;
    if (ROPE) attn_rope_load<HD>(rope, pos, t, c, sn);
    attn_tile<HD, ROPE>(q + (size_t)h * HD, ROPE ? knew + (size_t)kh * HD : nullptr,
                        ROPE ? vnew + (size_t)kh * HD : nullptr, c, sn, Kc, Vc, kh, h % Gq == 0, Lmax, pos, j0, scale,
                        wp, nullptr, 0ull, t, (AttnLdsPtr<HD>)&sm, kv);
}

// out[h*hd + d] from the S partials of head h (one thread per output element)
__global__ void __launch_bounds__(256) attn_combine_kernel(const float* __restrict__ work, int H, int hd, int S,
                                                           float* __restrict__ out) {
    const int i = blockIdx.x * blockDim.x + threadIdx.x;
    if (i >= H * hd) return;
    out[i] = attn_combine_element(work, hd, S, i / hd, i % hd);
}

// Final RMSNorm (f64 mean of squares, as the quantiser's) fused into the tied bf16 LM
// head: logits[r] = sum_k E[r][k] * xn[k]; the greedy token is the first index of the
// largest logit, accumulated as a 64-bit key (ordered value << 32 | ~index) with an
// atomic max.  Each wave owns `rows_per_wave` consecutive rows; lane l owns elements
// [512 s + 8 l, 512 s + 8 l + 8) of every row (D a multiple of 512).
__device__ __forceinline__ unsigned long long argmax_key(float v, unsigned idx) {
    unsigned b = __float_as_uint(v);
    b = (b & 0x80000000u) ? ~b : (b | 0x80000000u);
    return ((unsigned long long)b << 32) | (unsigned long long)(0xFFFFFFFFu - idx);
}

constexpr int kLmAuxNT = 2;  // buffer-load cache policy: non-temporal

template <int SLICES>
__global__ void __launch_bounds__(256) lm_head_kernel(const uint16_t* __restrict__ E, const float* __restrict__ x,
                                                      const float* __restrict__ norm_w, float eps, int V,
                                                      int rows_per_wave, float* __restrict__ logits,
                                                      unsigned long long* __restrict__ best) {
    constexpr int D = SLICES * 512;
    constexpr int RB = 4;  // rows per batch: a batch's RB * SLICES loads go out together
    __shared__ double redd[4];
    __shared__ float xs[D];
    const int t = threadIdx.x, lane = t & 63, wave = t >> 6;
    const int r0 = (blockIdx.x * 4 + wave) * rows_per_wave;
    const int r1 = min(r0 + rows_per_wave, V);  // this wave's rows [r0, r1)
    // Two batches alternate (A, B): the next batch's loads are in flight during the current
    // one's arithmetic, and the first two batches are issued before the RMSNorm below.
    v4u wa[RB][SLICES], wb[RB][SLICES];
    // the wave's rows as one buffer (32-bit offsets from its first row), read with the
    // non-temporal policy (streamed once): buffer loads measured 1.6 % faster than global ones
    // (with one atomic per workgroup below)
    const __amdgpu_buffer_rsrc_t er = __builtin_amdgcn_make_buffer_rsrc((void*)(E + (size_t)min(r0, V - 1) * D), 0,
                                                                        0x7FFFFFFF, kBufDword3);
    auto load_batch = [&](v4u (&w)[RB][SLICES], int rb) {
#pragma unroll
        for (int i = 0; i < RB; ++i) {
            const int r = min(rb + i, V - 1) - min(r0, V - 1);  // rows past V re-read the last row (discarded)
#pragma unroll
            for (int sl = 0; sl < SLICES; ++sl)
                w[i][sl] = __builtin_bit_cast(
                    v4u, __builtin_amdgcn_raw_buffer_load_b128(er, r * D * 2 + (sl * 64 + lane) * 16, 0, kLmAuxNT));
        }
    };
    if (r0 < r1) load_batch(wa, r0);
    if (r0 + RB < r1) load_batch(wb, r0 + RB);
    // RMSNorm of x over D (every workgroup recomputes it, each element once, into LDS)
    float xv[D / 256], wv[D / 256];
#pragma unroll
    for (int i = 0; i < D / 256; ++i) {
        xv[i] = x[t + 256 * i];
        wv[i] = norm_w[t + 256 * i];
    }
    double ss = 0.0;
#pragma unroll
    for (int i = 0; i < D / 256; ++i) ss += (double)xv[i] * (double)xv[i];
    ss = wave_reduce63(ss, 0.0, [](double x, double y) { return x + y; });
    if (lane == 63) redd[wave] = ss;
    __syncthreads();
    ss = (redd[0] + redd[1]) + (redd[2] + redd[3]);
    const float norm = sqrtf((float)(ss / (double)D) + eps);
#pragma unroll
    for (int i = 0; i < D / 256; ++i) xs[t + 256 * i] = (xv[i] / norm) * wv[i];
    __syncthreads();
    float xn[SLICES][8];
#pragma unroll
    for (int sl = 0; sl < SLICES; ++sl)
#pragma unroll
        for (int e = 0; e < 8; ++e) xn[sl][e] = xs[sl * 512 + lane * 8 + e];
    unsigned long long key = 0ull;
    auto batch_math = [&](const v4u (&w)[RB][SLICES], int rb) {
        float acc[RB];
#pragma unroll
        for (int i = 0; i < RB; ++i) {
            acc[i] = 0.0f;
#pragma unroll
            for (int sl = 0; sl < SLICES; ++sl)
#pragma unroll
                for (int e = 0; e < 4; ++e) {
                    acc[i] += __uint_as_float(w[i][sl][e] << 16) * xn[sl][2 * e];
                    acc[i] += __uint_as_float(w[i][sl][e] & 0xFFFF0000u) * xn[sl][2 * e + 1];
                }
        }
#pragma unroll
        for (int i = 0; i < RB; ++i) acc[i] = wave_reduce63(acc[i], 0.0f, [](float x, float y) { return x + y; });
        if (lane == 63) {  // the lane holding the totals
#pragma unroll
            for (int i = 0; i < RB; ++i) {
                const int r = rb + i;
                if (r < r1) {
                    logits[r] = acc[i];
                    const unsigned long long kk = argmax_key(acc[i], (unsigned)r);
                    key = kk > key ? kk : key;
                }
            }
        }
    };
    for (int rb = r0; rb < r1; rb += 2 * RB) {
        if (rb != r0 && rb + RB < r1) load_batch(wb, rb + RB);  // (the first B went out above)
        batch_math(wa, rb);
        if (rb + RB >= r1) break;
        if (rb + 2 * RB < r1) load_batch(wa, rb + 2 * RB);
        batch_math(wb, rb + RB);
    }
    // the workgroup's largest key, one atomic per workgroup
    __shared__ unsigned long long wkey[4];
    if (lane == 63) wkey[wave] = key;
    __syncthreads();
    if (t == 0) {
        const unsigned long long k01 = wkey[0] > wkey[1] ? wkey[0] : wkey[1];
        const unsigned long long k23 = wkey[2] > wkey[3] ? wkey[2] : wkey[3];
        const unsigned long long k = k01 > k23 ? k01 : k23;
        if (k) atomicMax(best, k);
    }
}

typedef float v4f __attribute__((ext_vector_type(4)));

// token = argmax; optionally also written to next_ids[0] (the next step's input) and,
// with p = *pos_p + advance, to out_tokens[p - 1 - pos_base]; then *pos_p = p.  With
// next_h, the token's embedding row E[token] (bf16 -> fp32, D values) is written there: the
// next step's input row, so that step needs no embedding launch.
__global__ void __launch_bounds__(256) argmax_finalize_kernel(unsigned long long* best, int* token, int* pos_p,
                                                              int advance, int* next_ids, int* out_tokens, int pos_base,
                                                              int out_cap, const uint16_t* __restrict__ E, int V,
                                                              int D, float* __restrict__ next_h) {
    const int t = threadIdx.x;
    // the maximum and the position are read together (one memory latency for both; without a
    // position the second read re-reads the maximum and is discarded)
    const int* pp = pos_p ? pos_p : reinterpret_cast<const int*>(best);
    const unsigned long long k = *best;
    int p = *pp;
    const int tok = (int)(0xFFFFFFFFu - (unsigned)(k & 0xFFFFFFFFull));
    if (next_h) {
        // (a row of NaN logits can leave `best` unset: read row 0 rather than out of range)
        const uint16_t* row = E + (size_t)(tok >= 0 && tok < V ? tok : 0) * D;
        const int D8 = D / 8;
        if (D % 8 == 0 && D8 <= 2 * (int)blockDim.x && (((uintptr_t)E | (uintptr_t)next_h) & 15u) == 0) {
            // eight values per 16-byte load, both of a thread's loads issued before its stores
            const int e0 = t, e1 = t + (int)blockDim.x;
            v4u u0{}, u1{};
            if (e0 < D8) u0 = reinterpret_cast<const v4u*>(row)[e0];
            if (e1 < D8) u1 = reinterpret_cast<const v4u*>(row)[e1];
            auto put = [&](int e, const v4u& u) {
                v4f lo, hi;
#pragma unroll
                for (int j = 0; j < 2; ++j) {
                    lo[2 * j] = __uint_as_float(u[j] << 16);
                    lo[2 * j + 1] = __uint_as_float(u[j] & 0xFFFF0000u);
                    hi[2 * j] = __uint_as_float(u[j + 2] << 16);
                    hi[2 * j + 1] = __uint_as_float(u[j + 2] & 0xFFFF0000u);
                }
                reinterpret_cast<v4f*>(next_h)[2 * e] = lo;
                reinterpret_cast<v4f*>(next_h)[2 * e + 1] = hi;
            };
            if (e0 < D8) put(e0, u0);
            if (e1 < D8) put(e1, u1);
        } else {
            for (int e = t; e < D; e += blockDim.x) next_h[e] = bf16_to_f32(row[e]);
        }
    }
    // Thread 0 resets *best below: every thread has its value by then (the empty asm needs it
    // in a register, so the wave waits for its load before the barrier).  The barrier does not
    // wait for the row's stores: nothing here reads them.
    asm volatile("" ::"v"(tok));
    __builtin_amdgcn_sched_barrier(0);
    __builtin_amdgcn_s_barrier();
    __builtin_amdgcn_sched_barrier(0);
    if (t != 0) return;
    *token = tok;
    *best = 0ull;  // ready for the next step
    if (next_ids) next_ids[0] = tok;
    if (pos_p) {
        p += advance;
        const int i = p - 1 - pos_base;
        if (out_tokens && i >= 0 && i < out_cap) out_tokens[i] = tok;
        *pos_p = p;
    }
}

hipError_t launch_embed(const uint16_t* E, const int* ids, int M, int V, int D, float* h, hipStream_t s) {
    hipLaunchKernelGGL(embed_kernel, dim3((unsigned)M), dim3(256), 0, s, E, ids, V, D, h);
    return hipGetLastError();
}

hipError_t launch_rope_append(float* q, float* k, const float* v, float* Kc, float* Vc, const float* rope, int M,
                              int H, int Hkv, int hd, int Lmax, const int* pos, hipStream_t s) {
    hipLaunchKernelGGL(rope_append_kernel, dim3((unsigned)M), dim3(256), 0, s, q, k, v, Kc, Vc, rope, H, Hkv, hd,
                       Lmax, pos);
    return hipGetLastError();
}

// the matrix-core prefill attention's LDS (above 64 KiB: allowed once per device, at
// context creation, so that no launch makes a function-attribute call)
constexpr size_t kAttnPrefillLds = (size_t)(4 * 128 * 32 * 2 + 4 * 32 * 2) * sizeof(float);

hipError_t model_prepare_device() {
    return hipFuncSetAttribute(reinterpret_cast<const void*>(&attn_prefill_mfma_kernel<128>),
                               hipFuncAttributeMaxDynamicSharedMemorySize, (int)kAttnPrefillLds);
}

hipError_t launch_attention(const float* q, const float* Kc, const float* Vc, float* out, int M, int H, int Hkv,
                            int hd, int Lmax, const int* pos, float scale, hipStream_t s) {
    const int G = H / Hkv;
    if (hd == 128 && G <= 32 && 32 % G == 0 && Lmax % 4 == 0) {  // matrix-core kernel
        constexpr size_t lds = kAttnPrefillLds;
        const int BQ = 32 / G;
        hipLaunchKernelGGL((attn_prefill_mfma_kernel<128>), dim3((unsigned)Hkv, (unsigned)((M + BQ - 1) / BQ)),
                           dim3(256), lds, s, q, Kc, Vc, out, M, H, Hkv, Lmax, pos, scale);
        return hipGetLastError();
    }
    const size_t lds = (size_t)(hd + Lmax + 256) * sizeof(float);
    hipLaunchKernelGGL(attention_kernel, dim3((unsigned)H, (unsigned)M), dim3(256), lds, s, q, Kc, Vc, out, H, Hkv,
                       hd, Lmax, pos, scale);
    return hipGetLastError();
}

hipError_t launch_attn_partial(const float* q, const float* knew, const float* vnew, float* Kc, float* Vc,
                               const float* rope, int H, int Hkv, int hd, int Lmax, const int* pos, float scale,
                               float* work, hipStream_t s) {
    const dim3 grid((unsigned)H, (unsigned)attn_splits(Lmax));
    const bool r = rope != nullptr;
    switch (hd * 2 + (r ? 1 : 0)) {
        case 128: hipLaunchKernelGGL((attn_partial_kernel<64, false>), grid, dim3(256), 0, s, q, knew, vnew, Kc, Vc, rope, H, Hkv, Lmax, pos, scale, work); break;
        case 129: hipLaunchKernelGGL((attn_partial_kernel<64, true>), grid, dim3(256), 0, s, q, knew, vnew, Kc, Vc, rope, H, Hkv, Lmax, pos, scale, work); break;
        case 256: hipLaunchKernelGGL((attn_partial_kernel<128, false>), grid, dim3(256), 0, s, q, knew, vnew, Kc, Vc, rope, H, Hkv, Lmax, pos, scale, work); break;
        case 257: hipLaunchKernelGGL((attn_partial_kernel<128, true>), grid, dim3(256), 0, s, q, knew, vnew, Kc, Vc, rope, H, Hkv, Lmax, pos, scale, work); break;
        default: return hipErrorInvalidValue;
    }
    return hipGetLastError();
}

hipError_t launch_attn_combine(const float* work, int H, int hd, int S, float* out, hipStream_t s) {
    hipLaunchKernelGGL(attn_combine_kernel, dim3((unsigned)((H * hd + 255) / 256)), dim3(256), 0, s, work, H, hd, S, out);
    return hipGetLastError();
}

// One round of workgroups: as many as the device holds at once (occupancy x CUs, taken
// once per device), each wave a run of consecutive rows (a multiple of the two batches).
template <int SLICES>
static hipError_t run_lm_head(const uint16_t* E, const float* x, const float* norm_w, float eps, int V, float* logits,
                              unsigned long long* best, hipStream_t s) {
    static int slots[64] = {0};
    int dev = 0;
    hipError_t e = hipGetDevice(&dev);
    if (e != hipSuccess) return e;
    if (dev < 0 || dev >= 64) return hipErrorInvalidDevice;
    if (slots[dev] == 0) {
        int per_cu = 0, cus = 0;
        e = hipOccupancyMaxActiveBlocksPerMultiprocessor(&per_cu, reinterpret_cast<const void*>(&lm_head_kernel<SLICES>),
                                                         256, 0);
        if (e == hipSuccess) e = hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev);
        if (e != hipSuccess) return e;
        slots[dev] = std::max(1, per_cu * cus);
    }
    int rpw = (V + 4 * slots[dev] - 1) / (4 * slots[dev]);
    rpw = (rpw + 7) / 8 * 8;
    // a wave reads its rows through one buffer resource with 32-bit offsets
    if ((long long)rpw * SLICES * 512 * 2 >= (1LL << 31)) return hipErrorInvalidValue;
    const unsigned blocks = (unsigned)((V + 4 * rpw - 1) / (4 * rpw));
    hipLaunchKernelGGL(lm_head_kernel<SLICES>, dim3(blocks), dim3(256), 0, s, E, x, norm_w, eps, V, rpw, logits, best);
    return hipGetLastError();
}

hipError_t launch_lm_head(const uint16_t* E, const float* x, const float* norm_w, float eps, int V, int D,
                          float* logits, unsigned long long* best, int* token, int* pos, int advance,
                          int* next_ids, int* out_tokens, int pos_base, int out_cap, float* next_h, hipStream_t s) {
    hipError_t e = hipSuccess;
    switch (D / 512) {
        case 1: e = run_lm_head<1>(E, x, norm_w, eps, V, logits, best, s); break;
        case 2: e = run_lm_head<2>(E, x, norm_w, eps, V, logits, best, s); break;
        case 4: e = run_lm_head<4>(E, x, norm_w, eps, V, logits, best, s); break;
        case 5: e = run_lm_head<5>(E, x, norm_w, eps, V, logits, best, s); break;
        case 8: e = run_lm_head<8>(E, x, norm_w, eps, V, logits, best, s); break;
        default: return hipErrorInvalidValue;
    }
    if (e != hipSuccess) return e;
    hipLaunchKernelGGL(argmax_finalize_kernel, dim3(1), dim3(next_h ? 256 : 64), 0, s, best, token, pos, advance,
                       next_ids, out_tokens, pos_base, out_cap, E, V, D, next_h);
    return hipGetLastError();
}

}  // namespace rt
