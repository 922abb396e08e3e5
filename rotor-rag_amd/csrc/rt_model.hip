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

// Decode attention, split over the keys: workgroup (h, s) handles keys
// [64 s, 64 s + 64) of query head h for the single query at *pos_p and writes a partial
// result to work[h][s][0..HD+2): the unnormalised output sum_j e^(s_j - m) V_j (HD
// values), the block maximum m and the sum of exponentials z (m = -inf, z = 0 for an
// empty block).  The partials are combined by attn_combine_kernel or, in the decode
// layer, by the prologue of the o_proj GEMV (rt_rowquant.h, kAttnNorm); both use
// attn_combine_element, so the two give identical values.
// ROPE: q, knew, vnew are the raw projection outputs of the token at *pos_p.  Every
// workgroup rotates its head's q (the arithmetic of rope_append_kernel); the workgroup
// whose block holds position *pos_p takes that key and value from LDS (rotated knew,
// vnew) instead of the cache, in the same summation order, and the first query head of
// each KV group writes them into the caches for the later steps.  Without ROPE, q is
// already rotated and the caches hold the new key.
template <int HD, bool ROPE>
__global__ void __launch_bounds__(256) attn_partial_kernel(const float* __restrict__ q, const float* __restrict__ knew,
                                                           const float* __restrict__ vnew, float* __restrict__ Kc,
                                                           float* __restrict__ Vc, const float* __restrict__ rope,
                                                           int H, int Hkv, int Lmax, const int* __restrict__ pos_p,
                                                           float scale, float* __restrict__ work) {
    constexpr int BL = 64, half = HD / 2, G = 256 / HD, KD = HD / 4, VN = BL / G;
    __shared__ float qs[HD];
    __shared__ float ks[HD];
    __shared__ float vs[HD];
    __shared__ float part[4][BL];
    __shared__ float pr[BL];
    __shared__ float ored[256];
    const int h = blockIdx.x, s = blockIdx.y, S = gridDim.y, t = threadIdx.x;
    const int lane = t & 63, wave = t >> 6;
    const int kh = h / (H / Hkv), j0 = s * BL;
    // The block's keys and values do not depend on the position: their loads go out first
    // (wave w: dims [w HD/4, (w+1) HD/4) of key j0 + lane; thread (d, g): value dim d of
    // keys g, g + G, ..), together with the position's.  Keys past Lmax re-read the last
    // cached key; keys past the position are masked below.
    const int d = t % HD, g = t / HD;
    float kreg[KD], vreg[VN];
    {
        const float* K = Kc + (size_t)kh * HD * Lmax + min(j0 + lane, Lmax - 1);
#pragma unroll
        for (int i = 0; i < KD; ++i) kreg[i] = K[(size_t)(wave * KD + i) * Lmax];
        const float* V = Vc + (size_t)kh * Lmax * HD + d;
#pragma unroll
        for (int i = 0; i < VN; ++i) vreg[i] = V[(size_t)min(j0 + g + i * G, Lmax - 1) * HD];
    }
    const int pos = *pos_p, L = pos + 1;
    const int nk = min(BL, L - j0);  // keys of this block (may be <= 0)
    float* wp = work + ((size_t)h * S + s) * (HD + 2);
    if (nk <= 0) {
        if (t == 0) {
            wp[HD] = -INFINITY;
            wp[HD + 1] = 0.0f;
        }
        return;
    }
    const bool holds_new = ROPE && pos < j0 + BL;  // this block ends with the new key
    const int lp = pos - j0;                       // its lane / key index in the block
    if (ROPE) {
        const float* cs = rope + (size_t)pos * half * 2;
        for (int i = t; i < half; i += 256) {
            const float c = cs[2 * i], sn = cs[2 * i + 1];
            const float x1 = q[(size_t)h * HD + i], x2 = q[(size_t)h * HD + i + half];
            qs[i] = x1 * c - x2 * sn;
            qs[i + half] = x2 * c + x1 * sn;
            if (holds_new) {
                const float k1 = knew[(size_t)kh * HD + i], k2 = knew[(size_t)kh * HD + i + half];
                ks[i] = k1 * c - k2 * sn;
                ks[i + half] = k2 * c + k1 * sn;
            }
        }
        if (holds_new)
            for (int e = t; e < HD; e += 256) vs[e] = vnew[(size_t)kh * HD + e];
    } else {
        for (int e = t; e < HD; e += 256) qs[e] = q[(size_t)h * HD + e];
    }
    __syncthreads();
    if (holds_new && h % (H / Hkv) == 0)  // one writer per KV head
        for (int e = t; e < HD; e += 256) {
            Kc[((size_t)kh * HD + e) * Lmax + pos] = ks[e];
            Vc[((size_t)kh * Lmax + pos) * HD + e] = vs[e];
        }
    // scores: wave w sums its dims for key j0 + lane (the new key from LDS)
    float a0 = 0.f, a1 = 0.f, a2 = 0.f, a3 = 0.f;
    if (lane < nk) {
        const bool mine = holds_new && lane == lp;
#pragma unroll
        for (int i = 0; i < KD; i += 4) {
            const int dd = wave * KD + i;
            a0 += qs[dd + 0] * (mine ? ks[dd + 0] : kreg[i + 0]);
            a1 += qs[dd + 1] * (mine ? ks[dd + 1] : kreg[i + 1]);
            a2 += qs[dd + 2] * (mine ? ks[dd + 2] : kreg[i + 2]);
            a3 += qs[dd + 3] * (mine ? ks[dd + 3] : kreg[i + 3]);
        }
    }
    part[wave][lane] = (a0 + a1) + (a2 + a3);
    __syncthreads();
    if (wave == 0) {
        float sc = lane < nk ? (((part[0][lane] + part[1][lane]) + (part[2][lane] + part[3][lane])) * scale)
                             : -INFINITY;
        float mx = sc;
        for (int off = 32; off >= 1; off >>= 1) mx = fmaxf(mx, __shfl_xor(mx, off, 64));
        const float p = lane < nk ? expf(sc - mx) : 0.0f;
        float z = p;
        for (int off = 32; off >= 1; off >>= 1) z += __shfl_xor(z, off, 64);
        pr[lane] = p;
        if (lane == 0) {
            wp[HD] = mx;
            wp[HD + 1] = z;
        }
    }
    __syncthreads();
    // unnormalised output: thread (d, g) sums keys g, g + G, ... of the block, two
    // alternating partial sums
    auto vrow = [&](int i) { return holds_new && g + i * G == lp ? vs[d] : vreg[i]; };
    float o0 = 0.f, o1 = 0.f;
#pragma unroll
    for (int i = 0; i < VN; i += 2) {
        if (g + i * G < nk) o0 += pr[g + i * G] * vrow(i);
        if (g + (i + 1) * G < nk) o1 += pr[g + (i + 1) * G] * vrow(i + 1);
    }
    ored[t] = o0 + o1;
    __syncthreads();
    if (g == 0) {
        float o = ored[d];
        for (int gg = 1; gg < G; ++gg) o += ored[gg * HD + d];
        wp[d] = o;
    }
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
    // one's arithmetic, and the first batch is issued before the RMSNorm below.
    v4u wa[RB][SLICES], wb[RB][SLICES];
    auto load_batch = [&](v4u (&w)[RB][SLICES], int rb) {
#pragma unroll
        for (int i = 0; i < RB; ++i) {
            const int r = min(rb + i, V - 1);  // rows past V re-read the last row (discarded)
            const v4u* row = reinterpret_cast<const v4u*>(E + (size_t)r * D);
#pragma unroll
            for (int sl = 0; sl < SLICES; ++sl) w[i][sl] = __builtin_nontemporal_load(row + sl * 64 + lane);
        }
    };
    if (r0 < r1) load_batch(wa, r0);
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
    for (int off = 32; off >= 1; off >>= 1) ss += __shfl_xor(ss, off, 64);
    if (lane == 0) redd[wave] = ss;
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
        for (int off = 32; off >= 1; off >>= 1)
#pragma unroll
            for (int i = 0; i < RB; ++i) acc[i] += __shfl_xor(acc[i], off, 64);
        if (lane == 0) {
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
        if (rb + RB < r1) load_batch(wb, rb + RB);
        batch_math(wa, rb);
        if (rb + RB >= r1) break;
        if (rb + 2 * RB < r1) load_batch(wa, rb + 2 * RB);
        batch_math(wb, rb + RB);
    }
    if (lane == 0 && key) atomicMax(best, key);
}

// token = argmax; optionally also written to next_ids[0] (the next step's input) and,
// with p = *pos_p + advance, to out_tokens[p - 1 - pos_base]; then *pos_p = p.
__global__ void argmax_finalize_kernel(unsigned long long* best, int* token, int* pos_p, int advance, int* next_ids,
                                       int* out_tokens, int pos_base, int out_cap) {
    const unsigned long long k = *best;
    const int tok = (int)(0xFFFFFFFFu - (unsigned)(k & 0xFFFFFFFFull));
    *token = tok;
    *best = 0ull;  // ready for the next step
    if (next_ids) next_ids[0] = tok;
    if (pos_p) {
        const int p = *pos_p + advance;
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

hipError_t launch_attention(const float* q, const float* Kc, const float* Vc, float* out, int M, int H, int Hkv,
                            int hd, int Lmax, const int* pos, float scale, hipStream_t s) {
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
    const unsigned blocks = (unsigned)((V + 4 * rpw - 1) / (4 * rpw));
    hipLaunchKernelGGL(lm_head_kernel<SLICES>, dim3(blocks), dim3(256), 0, s, E, x, norm_w, eps, V, rpw, logits, best);
    return hipGetLastError();
}

hipError_t launch_lm_head(const uint16_t* E, const float* x, const float* norm_w, float eps, int V, int D,
                          float* logits, unsigned long long* best, int* token, int* pos, int advance,
                          int* next_ids, int* out_tokens, int pos_base, int out_cap, hipStream_t s) {
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
    hipLaunchKernelGGL(argmax_finalize_kernel, dim3(1), dim3(1), 0, s, best, token, pos, advance, next_ids,
                       out_tokens, pos_base, out_cap);
    return hipGetLastError();
}

}  // namespace rt
