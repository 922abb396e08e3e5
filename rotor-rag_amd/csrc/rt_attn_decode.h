// Decode attention over one block of 64 keys for one query head: the work of a
// 256-thread tile, shared by the split-L attention kernel (rt_model.hip) and by the qkv
// GEMV launch that runs the attention partials in its trailing workgroups (rt_gemv.hip).
//
// Reference: MultiHeadAttention.forward (src/rotor/transformer.py:206-292: KV concat
// :250-252, GQA repeat :260-263, scores/softmax/AV :267-281); this build adds RoPE and a
// causal mask (the benchmark configuration).
//
// The tile (h, s) handles keys [64 s, 64 s + 64) of query head h for the single query at
// position pos and writes a partial result wp[0..HD+2): the unnormalised output
// sum_j e^(s_j - m) V_j (HD values), the block maximum m and the sum of exponentials z
// (m = -inf, z = 0 for an empty block).  The partials are combined by attn_combine_kernel,
// by the prologue of the o_proj GEMV (rt_rowquant.h, kAttnNorm) or in the qkv launch; all
// use the operation order of attn_combine_element, so they give identical values.
#pragma once

#include "rt_internal.h"

namespace rt {

constexpr int kAttnBlock = 64;  // keys per split

// Workgroup barrier for the tile's LDS hand-offs: waits for this wave's LDS accesses only.
// __syncthreads() also waits for the wave's outstanding global stores (its fence), which
// held every tile of a workgroup behind the new key's cache stores and the partials' stores
// (their round trip to memory) at each later barrier; nothing in the launch reads those.
__device__ __forceinline__ void attn_lds_barrier() {
    __builtin_amdgcn_sched_barrier(0);
    asm volatile("s_waitcnt lgkmcnt(0)\n\ts_barrier" ::: "memory");
    __builtin_amdgcn_sched_barrier(0);
}

template <int HD>
struct AttnTileLds {
    float qs[HD];
    float ks[HD];
    float vs[HD];
    float part[4][kAttnBlock];
    float pr[kAttnBlock];
    float ored[256];
};

// The tile's LDS is reached through a local-address-space pointer: through a generic one,
// a select between an LDS value and a register of the key block (the new key) becomes a
// load through a selected generic pointer, which puts the key block in scratch memory.
template <int HD>
using AttnLdsPtr = __attribute__((address_space(3))) AttnTileLds<HD>*;

// A thread's share of its key block, loaded before anything else (the keys and values do
// not depend on the position): wave w of the tile holds dims [w HD/4, (w+1) HD/4) of key
// j0 + lane; thread (d, g) = (t % HD, t / HD) value dim d of keys g, g + G, .. (G = 256 / HD).
// Keys past Lmax re-read the last cached key; keys past the position are masked later.
template <int HD>
struct AttnKV {
    static constexpr int G = 256 / HD, KD = HD / 4, VN = kAttnBlock / G;
    float k[KD];
    float v[VN];
};

template <int HD>
__device__ __forceinline__ void attn_kv_load(const float* __restrict__ Kc, const float* __restrict__ Vc, int kh, int j0,
                                             int Lmax, int t, AttnKV<HD>& kv) {
    using KV = AttnKV<HD>;
    const int lane = t & 63, wave = t >> 6, d = t % HD, g = t / HD;
    const float* K = Kc + (size_t)kh * HD * Lmax + min(j0 + lane, Lmax - 1);
#pragma unroll
    for (int i = 0; i < KV::KD; ++i) kv.k[i] = K[(size_t)(wave * KV::KD + i) * Lmax];
    const float* V = Vc + (size_t)kh * Lmax * HD + d;
#pragma unroll
    for (int i = 0; i < KV::VN; ++i) kv.v[i] = V[(size_t)min(j0 + g + i * KV::G, Lmax - 1) * HD];
}

// The RoPE factors (cos, sin) of rotation pair t (t < HD / 2) at position pos: loaded by
// the caller as early as the position is known (the tile's first step waits for them).
template <int HD>
__device__ __forceinline__ void attn_rope_load(const float* __restrict__ rope, int pos, int t, float& c, float& sn) {
    c = sn = 0.0f;
    if (t < HD / 2) {
        const float* cs = rope + (size_t)pos * HD + 2 * t;
        c = cs[0];
        sn = cs[1];
    }
}

// The tile's work once the position is known and the block holds at least one key
// (pos >= j0).  Every thread of the workgroup passes the tile's four barriers.
// qh: the head's query (HD values); kn, vn: the head's KV group's new key and value (ROPE),
// in global memory or in LDS (SRC, a pointer type); c, sn: attn_rope_load's factors (ROPE).
// ROPE: qh, kn, vn are the raw projection outputs of the token at pos.  The tile rotates
// its head's q (the arithmetic of rope_append_kernel); the tile whose block holds position
// pos takes that key and value from LDS (rotated kn, vn) instead of the cache, in the same
// summation order, and, when `writer` (one query head of its KV group), writes them into
// the caches of KV head kh for the later steps, once its partial is stored.  Without ROPE, qh is already rotated
// and the caches hold the new key.
// Value i of a partial: a plain store to wp, and (TAG, wt not null) a copy as the 64-bit
// word tag | bits(v) to wt, device-coherent, for readers in other workgroups of the same
// launch (tag = epoch << 32).
template <bool TAG>
__device__ __forceinline__ void part_store(float* wp, unsigned long long* wt, unsigned long long tag, int i,
                                           float v) {
    wp[i] = v;
    if constexpr (TAG)
        if (wt) __hip_atomic_store(wt + i, tag | __float_as_uint(v), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

template <int HD, bool ROPE, bool TAG = false, typename SRC>
__device__ __forceinline__ void attn_tile(SRC qh, SRC kn, SRC vn, float c, float sn, float* __restrict__ Kc,
                                          float* __restrict__ Vc, int kh, bool writer, int Lmax, int pos, int j0,
                                          float scale, float* __restrict__ wp, unsigned long long* __restrict__ wt,
                                          unsigned long long tag, int t, AttnLdsPtr<HD> sm, const AttnKV<HD>& kv) {
#pragma clang fp contract(off)  // every operation rounds on its own, fmaf where written
    static_assert(HD / 2 <= 256, "one rotation pair per thread");
    using KV = AttnKV<HD>;
    constexpr int BL = kAttnBlock, half = HD / 2, G = KV::G, KD = KV::KD, VN = KV::VN;
    const int lane = t & 63, wave = t >> 6, d = t % HD, g = t / HD;
    const int nk = min(BL, pos + 1 - j0);          // keys of this block (>= 1)
    const bool holds_new = ROPE && pos < j0 + BL;  // this block ends with the new key
    const int lp = pos - j0;                       // its lane / key index in the block
    if (ROPE) {
        if (t < half) {
            const int i = t;
            const float x1 = qh[i], x2 = qh[i + half];
            sm->qs[i] = x1 * c - x2 * sn;
            sm->qs[i + half] = x2 * c + x1 * sn;
            if (holds_new) {
                const float k1 = kn[i], k2 = kn[i + half];
                sm->ks[i] = k1 * c - k2 * sn;
                sm->ks[i + half] = k2 * c + k1 * sn;
            }
        }
        if (holds_new)
            for (int e = t; e < HD; e += 256) sm->vs[e] = vn[e];
    } else {
        for (int e = t; e < HD; e += 256) sm->qs[e] = qh[e];
    }
    attn_lds_barrier();
    // scores: wave w sums its dims for key j0 + lane (the new key from LDS: the one lane
    // that holds it takes its dims first, in a branch that every other wave skips).
    // Branch-free otherwise: every lane computes (keys past the block's last are discarded
    // by the softmax's mask), so the LDS reads go out together.
    float kk[KD];
#pragma unroll
    for (int i = 0; i < KD; ++i) kk[i] = kv.k[i];
    if (holds_new && lane == lp) {
#pragma unroll
        for (int i = 0; i < KD; ++i) kk[i] = sm->ks[wave * KD + i];
    }
    float a0 = 0.f, a1 = 0.f, a2 = 0.f, a3 = 0.f;
#pragma unroll
    for (int i = 0; i < KD; i += 4) {
        const int dd = wave * KD + i;
        a0 = fmaf(sm->qs[dd + 0], kk[i + 0], a0);
        a1 = fmaf(sm->qs[dd + 1], kk[i + 1], a1);
        a2 = fmaf(sm->qs[dd + 2], kk[i + 2], a2);
        a3 = fmaf(sm->qs[dd + 3], kk[i + 3], a3);
    }
    sm->part[wave][lane] = (a0 + a1) + (a2 + a3);
    attn_lds_barrier();
    if (wave == 0) {
        float sc = lane < nk
                       ? (((sm->part[0][lane] + sm->part[1][lane]) + (sm->part[2][lane] + sm->part[3][lane])) * scale)
                       : -INFINITY;
        const float mx = lane63(wave_reduce63(sc, -INFINITY, [](float x, float y) { return fmaxf(x, y); }));
        const float p = lane < nk ? expf(sc - mx) : 0.0f;
        const float z = wave_reduce63(p, 0.0f, [](float x, float y) { return x + y; });
        sm->pr[lane] = p;
        if (lane == 63) {
            part_store<TAG>(wp, wt, tag, HD, mx);
            part_store<TAG>(wp, wt, tag, HD + 1, z);
        }
    }
    attn_lds_barrier();
    // unnormalised output: thread (d, g) sums keys g, g + G, ... of the block, two
    // alternating partial sums of fused multiply-adds (as the scores' four).  The new key's value and the mask of keys past the
    // position cost VALU work only where they apply: four tiles share a CU in the qkv
    // launch, where this loop is VALU-bound.  The keys go in runs of CH; g is uniform
    // over a wave and nk over the workgroup, so a run lies wholly before nk (plain sums),
    // wholly past it (skipped) or across it (masked sums) by a uniform branch, and the
    // LDS reads of a run go out together.  Skipping a masked key leaves the sums as the
    // masked form does, so the order of the additions is the same in every block.
    float vv[VN];
#pragma unroll
    for (int i = 0; i < VN; ++i) vv[i] = kv.v[i];
    if (holds_new) {
        // the new key's slot among this thread's keys g, g + G, ..: g and lp are uniform over
        // the wave, so one indexed register write takes the place of a select per key
        const int rel = __builtin_amdgcn_readfirstlane(lp - g);
        if (rel >= 0 && rel % G == 0) vv[rel / G] = sm->vs[d];
    }
    float o0 = 0.f, o1 = 0.f;
    constexpr int CH = VN >= 8 ? 8 : VN;
    static_assert(VN % CH == 0 && CH % 2 == 0, "runs of key pairs");
#pragma unroll
    for (int c0 = 0; c0 < VN; c0 += CH) {
        const int first = g + c0 * G, last = g + (c0 + CH - 1) * G;
        if (last < nk) {
#pragma unroll
            for (int i = c0; i < c0 + CH; i += 2) {
                o0 = fmaf(sm->pr[g + i * G], vv[i], o0);
                o1 = fmaf(sm->pr[g + (i + 1) * G], vv[i + 1], o1);
            }
        } else if (first < nk) {
#pragma unroll
            for (int i = c0; i < c0 + CH; i += 2) {
                const int ja = g + i * G, jb = g + (i + 1) * G;
                const float sa = fmaf(sm->pr[ja], vv[i], o0), sb = fmaf(sm->pr[jb], vv[i + 1], o1);
                o0 = ja < nk ? sa : o0;
                o1 = jb < nk ? sb : o1;
            }
        }
    }
    sm->ored[t] = o0 + o1;
    attn_lds_barrier();
    if (g == 0) {
        float o = sm->ored[d];
        for (int gg = 1; gg < G; ++gg) o += sm->ored[gg * HD + d];
        part_store<TAG>(wp, wt, tag, d, o);
    }
    // the new key and value into the caches of KV head kh (one writer tile per KV head),
    // after the partial: only later steps read them, and nothing here waits for the stores
    if (holds_new && writer)
        for (int e = t; e < HD; e += 256) {
            Kc[((size_t)kh * HD + e) * Lmax + pos] = sm->ks[e];
            Vc[((size_t)kh * Lmax + pos) * HD + e] = sm->vs[e];
        }
}

// The partial of an empty block (no key at or before the position): m = -inf, z = 0; with
// TAG every word of the tagged copy is written (the values as 0), so a reader can wait for
// all of them.
template <int HD, bool TAG = false>
__device__ __forceinline__ void attn_tile_empty(float* __restrict__ wp, unsigned long long* __restrict__ wt,
                                                unsigned long long tag, int t) {
    if (t == 0) {
        part_store<TAG>(wp, wt, tag, HD, -INFINITY);
        part_store<TAG>(wp, wt, tag, HD + 1, 0.0f);
    }
    if constexpr (TAG)
        if (wt)
            for (int d = t; d < HD; d += 256) __hip_atomic_store(wt + d, tag, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

}  // namespace rt
