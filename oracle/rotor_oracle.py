"""CPU oracle for the rotor ternary-linear path.

TEST INFRASTRUCTURE ONLY.  Nothing in the product package (``rotor-rag_amd/``)
imports this module; only ``tests/``, ``__graft_entry__.smoke()`` and the
``cpu_baseline`` leg of ``bench.py`` may use it, and only as the checker.

Every function restates, in NumPy, the algorithm of a reference function and
cites it (paths relative to the reference repository BikerSam86/rotor-RAG).
How each function is pinned (golden vectors / closed forms / invariants /
cross-check against the reference's own C core built under ``oracle/_ref``)
is listed in ``PINNED`` at the bottom of this file; the tests in
``tests/test_oracle_*.py`` carry out those checks.
"""
from __future__ import annotations

import numpy as np

# ---------------------------------------------------------------------------
# a1: the rotor 2-bit code.  value = bit0 - bit1;  00 -> 0, 10 -> +1, 01 -> -1,
# 11 -> error (decodes to 0).  Element j of a packed byte sits in bits
# (2j+1, 2j) = (bit0, bit1), i.e. the 2-bit field (byte >> 2j) & 3 is 2*bit0+bit1.
# ---------------------------------------------------------------------------


def encode(values):
    """{-1,0,+1} -> (bit0, bit1).  src/rotor/core.py:27-53."""
    v = np.asarray(values).astype(np.int8)
    return (v == 1).astype(np.uint8), (v == -1).astype(np.uint8)


def decode(bit0, bit1):
    """(bit0, bit1) -> bit0 - bit1 as int8.  src/rotor/core.py:56-72."""
    return np.asarray(bit0).astype(np.int8) - np.asarray(bit1).astype(np.int8)


def check_errors(bit0, bit1):
    """True where both bits are set (the reserved 11 code).  src/rotor/core.py:233-243."""
    return (np.asarray(bit0) & np.asarray(bit1)).astype(bool)


def pack(bit0, bit1):
    """Pack 4 rotors per byte, element j -> bits (2j+1, 2j) = (bit0, bit1).

    src/rotor/core.py:75-110 (layout at :99-108).  Length must be a multiple of 4.
    """
    b0 = np.asarray(bit0).astype(np.uint8).reshape(-1, 4)
    b1 = np.asarray(bit1).astype(np.uint8).reshape(-1, 4)
    out = np.zeros(b0.shape[0], dtype=np.uint8)
    for j in range(4):
        out |= (b0[:, j] << (2 * j + 1)).astype(np.uint8)
        out |= (b1[:, j] << (2 * j)).astype(np.uint8)
    return out


def unpack(packed, n_rotors):
    """Inverse of :func:`pack`, truncated to ``n_rotors``.  src/rotor/core.py:113-141."""
    p = np.asarray(packed, dtype=np.uint8)[: (n_rotors + 3) // 4]
    b0 = np.stack([(p >> (2 * j + 1)) & 1 for j in range(4)], axis=1).ravel()[:n_rotors]
    b1 = np.stack([(p >> (2 * j)) & 1 for j in range(4)], axis=1).ravel()[:n_rotors]
    return b0.astype(np.uint8), b1.astype(np.uint8)


def pack_rotor(W):
    """Ternary matrix W [N, K] (int) -> rotor bytes [N, ceil(K/4)], rows packed
    independently (K padded with zero codes to a multiple of 4).

    This is the host-facing weight format of the build: the same per-byte layout as
    src/rotor/core.py:99-108 and the same row convention as the reference's BitNet
    tensors ``[out_features, in_features_packed]`` (src/rotor/transformer.py:82,90;
    native/c/rotor_core.c:221-242).
    """
    W = np.asarray(W)
    N, K = W.shape
    Kp = (K + 3) // 4 * 4
    Wp = np.zeros((N, Kp), dtype=np.int8)
    Wp[:, :K] = W
    b0, b1 = encode(Wp)
    return pack(b0.ravel(), b1.ravel()).reshape(N, Kp // 4)


def unpack_rotor(packed, K):
    """Rotor bytes [N, Kb] -> int8 W [N, K].  Field value f = (byte >> 2j) & 3,
    w = (f >> 1) - (f & 1): 00->0, 10->+1, 01->-1, 11->0
    (native/c/rotor_core.c:240-256; src/rotor/core.py:56-72,113-141)."""
    p = np.asarray(packed, dtype=np.uint8)
    N, Kb = p.shape
    f = np.stack([(p >> (2 * j)) & 3 for j in range(4)], axis=2).reshape(N, Kb * 4)
    w = ((f >> 1).astype(np.int8) - (f & 1).astype(np.int8))
    return w[:, :K].copy()


# ---------------------------------------------------------------------------
# a2/a3: BitNet bytes <-> LSB-first bit planes <-> int8 (the reference's load path)
# ---------------------------------------------------------------------------


def bitnet_to_rotor(bitnet_packed, cols=None):
    """4/byte codes [rows, cb] -> planes (bit0, bit1) [rows, ceil(cols/8)], LSB-first.

    native/c/rotor_core.c:202-260 (and the Python twin src/rotor/bitnet.py:76-151).
    ``cols`` defaults to 4*cb as in src/rotor/bitnet_fast.py:71.
    """
    p = np.asarray(bitnet_packed, dtype=np.uint8)
    rows, cb = p.shape
    cols = cb * 4 if cols is None else cols
    f = np.stack([(p >> (2 * j)) & 3 for j in range(4)], axis=2).reshape(rows, cb * 4)[:, :cols]
    nb = (cols + 7) // 8
    pos = np.zeros((rows, nb * 8), dtype=np.uint8)
    neg = np.zeros((rows, nb * 8), dtype=np.uint8)
    pos[:, :cols] = (f == 2)
    neg[:, :cols] = (f == 1)
    weights = (1 << np.arange(8, dtype=np.uint16))
    bit0 = (pos.reshape(rows, nb, 8) * weights).sum(axis=2).astype(np.uint8)
    bit1 = (neg.reshape(rows, nb, 8) * weights).sum(axis=2).astype(np.uint8)
    return bit0, bit1


def rotor_unpack_weights(bit0, bit1, rows, cols):
    """Planes [rows, ceil(cols/8)] -> int8 [rows, cols], w = bit0 - bit1, LSB-first.

    native/c/rotor_core.c:270-299 (called via src/rotor/transformer.py:157-171).
    """
    b0 = np.unpackbits(np.asarray(bit0, dtype=np.uint8).reshape(rows, -1), axis=1, bitorder="little")
    b1 = np.unpackbits(np.asarray(bit1, dtype=np.uint8).reshape(rows, -1), axis=1, bitorder="little")
    return (b0[:, :cols].astype(np.int8) - b1[:, :cols].astype(np.int8))


# ---------------------------------------------------------------------------
# a4: absmax int8 quantiser, applied per row (per token)
# ---------------------------------------------------------------------------


def quant_rows(x):
    """Per-row symmetric absmax int8 quantiser.

    The formula is src/rotor/quantization.py:137-149 (bits=8, symmetric) applied to
    each row: s = max|x| / 127 (1.0 when max|x| == 0), q = clip(round_half_even(x / s),
    -128, 127).  All arithmetic is pinned to float32 (IEEE division, NumPy's
    round-half-even), which is what the reference computes under NumPy 2 for fp32 x.
    Returns q int8 [M, K] and s float32 [M].
    """
    x = np.asarray(x, dtype=np.float32)
    x2 = x.reshape(-1, x.shape[-1])
    amax = np.max(np.abs(x2), axis=1) if x2.shape[1] else np.zeros(x2.shape[0], np.float32)
    safe = np.where(amax > 0, amax, np.float32(127.0)).astype(np.float32)
    s = np.where(amax > 0, safe / np.float32(127.0), np.float32(1.0)).astype(np.float32)
    q = np.clip(np.round(x2 / s[:, None]), -128, 127).astype(np.int8)
    return q.reshape(x.shape), s


def dequant_rows(q, s):
    """x_hat = q * s (fp32), the per-row form of src/rotor/quantization.py:169-183."""
    q = np.asarray(q)
    return (q.astype(np.float32) * np.asarray(s, np.float32).reshape(-1, 1)).reshape(q.shape)


# ---------------------------------------------------------------------------
# a5: the ternary linear
# ---------------------------------------------------------------------------


def linear_i64(q, W):
    """Exact integer accumulators acc[m, n] = sum_k q[m, k] * W[n, k] in int64."""
    return np.asarray(q, dtype=np.int64) @ np.asarray(W, dtype=np.int64).T


def linear_i64_fast(q, W):
    """Same result as :func:`linear_i64` computed with floating-point BLAS.

    Exact: every product and partial sum is an integer of magnitude at most 128 K
    (|q| <= 128, |W| <= 1): below 2**24 in float32 (K < 131072), else below 2**53 in
    float64 (K < 2**40), so no rounding occurs in any summation order.
    """
    K = np.asarray(q).shape[-1]
    assert K < (1 << 40)
    # with int8 q and ternary W, |partial sums| <= 128 K: below 2^24 they are exact in
    # float32 too (half the memory traffic of the float64 product)
    dt = np.float32 if 128 * K < (1 << 24) and np.abs(np.asarray(q)).max(initial=0) <= 128 else np.float64
    q = np.asarray(q, dtype=dt)
    W = np.asarray(W, dtype=dt)
    return (q @ W.T).astype(np.int64)


def linear_ref_f32(x, W_i8, scale):
    """The reference's CPU ternary path: ``np.dot(x_flat, weights_cache.T) * scale``.

    src/rotor/transformer.py:150 (2-D/3-D reshape rules :121-128, :152-155).  Note
    NumPy up-casts the int8 weight cache to float32 for the product (as the
    reference does on every call).
    """
    x = np.asarray(x, dtype=np.float32)
    shp = x.shape
    xf = x.reshape(-1, shp[-1])
    y = np.dot(xf, np.asarray(W_i8).T) * np.float32(scale)
    y = y.astype(np.float32)
    return y.reshape(shp[:-1] + (y.shape[-1],))


def ternary_linear(x, W_i8, scale):
    """fp32 parity reference for the W2A8 path on the *same quantised inputs*:
    q, s = quant_rows(x); x_hat = q * s; y = np.dot(x_hat, W.T) * scale.

    Returns (y, q, s, acc) where acc is the exact int64 accumulator.
    """
    x = np.asarray(x, dtype=np.float32)
    q, s = quant_rows(x.reshape(-1, x.shape[-1]))
    xh = dequant_rows(q, s)
    y = linear_ref_f32(xh, W_i8, scale).reshape(x.shape[:-1] + (np.asarray(W_i8).shape[0],))
    return y, q, s, linear_i64_fast(q, W_i8)


# ---------------------------------------------------------------------------
# a9/a10 glue (cfg 1): RMSNorm and the FFN block restated with the config semantics
# ---------------------------------------------------------------------------


def rms_norm(x, weight, eps=1e-6):
    """x / sqrt(mean(x^2) + eps) * w.  src/rotor/transformer.py:24-36 (eps :20)."""
    x = np.asarray(x, dtype=np.float32)
    norm = np.sqrt(np.mean(x ** 2, axis=-1, keepdims=True) + np.float32(eps)).astype(np.float32)
    return ((x / norm) * np.asarray(weight, np.float32)).astype(np.float32)


def rms_norm_f64acc(x, weight, eps=1e-6):
    """RMSNorm with the mean of squares accumulated in float64 and rounded once to
    float32: norm = sqrt(f32(sum(x^2) / K) + eps) in f32, h = (x / norm) * w in f32.

    The formula of src/rotor/transformer.py:24-36; the accumulation precision is the
    build's choice (order independent), the reference's fp32 pairwise mean agrees to
    about one ulp.
    """
    x = np.asarray(x, dtype=np.float32)
    K = x.shape[-1]
    ss = np.sum(x.astype(np.float64) ** 2, axis=-1, keepdims=True)
    ms = (ss / np.float64(K)).astype(np.float32)
    norm = np.sqrt(ms + np.float32(eps)).astype(np.float32)
    return ((x / norm) * np.asarray(weight, np.float32)).astype(np.float32)


def w2a8_linear_from_q(q, s, W, scale):
    """Epilogue of the W2A8 linear on given quantised activations:
    y = (f32(acc) * s_x) * s_w, acc exact."""
    acc = linear_i64_fast(q, W)
    return (acc.astype(np.float32) * np.asarray(s, np.float32).reshape(-1, 1)) * np.float32(scale), acc


def ffn_block_w2a8(x, norm_w, Wg, sg, Wu, su, Wd, sd, eps=1e-6):
    """cfg 1 exactly as the device computes it: h = rms_norm_f64acc(x); q_h = quant(h);
    g, u = W2A8 linears; a = relu(g)^2 * u; q_a = quant(a); y = W2A8 linear(q_a, Wd).
    Every intermediate is reproducible bit for bit, so the device result must match."""
    h = rms_norm_f64acc(x, norm_w, eps)
    qh, sh = quant_rows(h)
    g, acc_g = w2a8_linear_from_q(qh, sh, Wg, sg)
    u, acc_u = w2a8_linear_from_q(qh, sh, Wu, su)
    a = relu2_gate(g, u)
    qa, sa = quant_rows(a)
    y, acc_d = w2a8_linear_from_q(qa, sa, Wd, sd)
    return y, dict(h=h, qh=qh, sh=sh, g=g, u=u, a=a, qa=qa, sa=sa, acc_g=acc_g, acc_u=acc_u, acc_d=acc_d)


def relu2_gate(g, u):
    """relu(g)^2 * u in float32 (the configuration's FFN activation)."""
    g = np.asarray(g, np.float32)
    r = np.maximum(g, np.float32(0))
    return (r * r * np.asarray(u, np.float32)).astype(np.float32)


def ffn_block(x, norm_w, Wg, sg, Wu, su, Wd, sd, eps=1e-6):
    """cfg 1: RMSNorm -> gate & up ternary linears -> relu^2(gate)*up -> down.

    Every ternary linear is the W2A8 form of :func:`ternary_linear` (per-token int8
    activations); the callers it restates are GatedFFN.forward
    (src/rotor/transformer.py:320-341) with the configuration's relu^2 activation in
    place of the reference's SiLU and no sub-norm.  Returns y and the intermediates.
    """
    h = rms_norm(x, norm_w, eps)
    g, qh, sh, acc_g = ternary_linear(h, Wg, sg)
    u, _, _, acc_u = ternary_linear(h, Wu, su)
    a = relu2_gate(g, u)
    y, qa, sa, acc_d = ternary_linear(a, Wd, sd)
    return y, dict(h=h, qh=qh, sh=sh, g=g, u=u, acc_g=acc_g, acc_u=acc_u, a=a, qa=qa, sa=sa, acc_d=acc_d)


# ---------------------------------------------------------------------------
# a11: the decode model of the benchmark configuration (cfg 4), restated in NumPy
# ---------------------------------------------------------------------------


def bf16_to_f32(b):
    """uint16 bf16 bit patterns -> float32 (exact)."""
    return (np.asarray(b, np.uint16).astype(np.uint32) << 16).view(np.float32)


def f32_to_bf16(x):
    """float32 -> bf16 bit patterns, round to nearest even."""
    u = np.asarray(x, np.float32).view(np.uint32).astype(np.uint64)
    r = (u + 0x7FFF + ((u >> 16) & 1)) >> 16
    return r.astype(np.uint16)


def rope_table(max_len, head_dim, theta):
    """(cos, sin) of pos * theta^(-2i/head_dim) [max_len, head_dim/2, 2], f64 then f32."""
    i = np.arange(head_dim // 2, dtype=np.float64)
    inv = theta ** (-(2.0 * i) / head_dim)
    ang = np.arange(max_len, dtype=np.float64)[:, None] * inv[None, :]
    return np.stack([np.cos(ang), np.sin(ang)], axis=-1).astype(np.float32)


def apply_rope(x, table, pos0):
    """Rotate-half RoPE on x [M, heads, hd] for positions pos0.. in float32:
    x1' = x1*c - x2*s, x2' = x2*c + x1*s (two roundings per product, then the add)."""
    M, _, hd = x.shape
    half = hd // 2
    cs = table[pos0:pos0 + M]  # [M, half, 2]
    c, s = cs[:, None, :, 0], cs[:, None, :, 1]
    x1, x2 = x[..., :half], x[..., half:]
    return np.concatenate([x1 * c - x2 * s, x2 * c + x1 * s], axis=-1).astype(np.float32)


def causal_gqa_attention(q, K, V, pos0):
    """q [M, H, hd] (queries at pos0..), K/V [Hkv, L, hd] (all cached keys) ->
    out [M, H, hd]; scale 1/sqrt(hd); query m sees keys 0..pos0+m.  Computed in f64
    (src/rotor/transformer.py:260-281 plus the causal mask of the configuration), all
    queries of a head at once with the keys past each query masked out."""
    M, H, hd = q.shape
    Hkv = K.shape[0]
    rep = H // Hkv
    L = pos0 + M
    scale = np.float32(1.0) / np.sqrt(np.float32(hd))
    visible = np.arange(L)[None, :] <= (pos0 + np.arange(M))[:, None]  # [M, L]
    out = np.zeros((M, H, hd), np.float64)
    for kv in range(Hkv):
        kk = K[kv, :L].astype(np.float64)
        vv = V[kv, :L].astype(np.float64)
        for h in range(kv * rep, (kv + 1) * rep):
            sc = (q[:, h].astype(np.float64) @ kk.T) * np.float64(scale)
            sc = np.where(visible, sc, -np.inf)
            p = np.exp(sc - sc.max(axis=1, keepdims=True))
            out[:, h] = (p / p.sum(axis=1, keepdims=True)) @ vv
    return out.astype(np.float32)


def bitnet_forward(params, cfg, ids, cache, attn_in=None, attn_ref=None, x_out=None):
    """One forward of the cfg-4 model on token ids [M] at position len(cache)
    (cache: dict with per-layer K/V lists, updated in place).  Returns the final-normed
    hidden states [M, D] and the logits of the last token [V] (f64 accumulation).

    Layer: x += Wo(subnorm(attn(rope(Wq a), rope(Wk a), Wv a))), a = norm(x);
           x += Wd(subnorm(relu(Wg f)^2 * Wu f)), f = norm(x)  -- every linear W2A8.

    attn_in (optional, per layer [M, H*hd] fp32): attention outputs to continue each layer
    with in place of the ones computed here (teacher forcing: every other operation is
    reproducible bit for bit, attention only to fp32 summation order); attn_ref (optional
    list) receives the attention outputs computed here, layer by layer; x_out (optional
    list) receives the hidden states [M, D] before the final norm.
    """
    H, Hkv, eps = cfg["n_heads"], cfg["n_kv_heads"], cfg.get("rms_norm_eps", 1e-6)
    D = cfg["d_model"]
    hd = D // H
    pos0 = cache.get("len", 0)
    x = bf16_to_f32(params["embed"][np.asarray(ids)]).astype(np.float32)
    M = x.shape[0]
    table = params["rope"]
    for li, L in enumerate(params["layers"]):
        a = rms_norm_f64acc(x, L["input_norm"], eps)
        qa, sa = quant_rows(a)
        q = w2a8_linear_from_q(qa, sa, L["q_proj"][0], L["q_proj"][1])[0]
        k = w2a8_linear_from_q(qa, sa, L["k_proj"][0], L["k_proj"][1])[0]
        v = w2a8_linear_from_q(qa, sa, L["v_proj"][0], L["v_proj"][1])[0]
        q = apply_rope(q.reshape(M, H, hd), table, pos0)
        k = apply_rope(k.reshape(M, Hkv, hd), table, pos0)
        kv = cache.setdefault(li, {"k": np.zeros((Hkv, 0, hd), np.float32), "v": np.zeros((Hkv, 0, hd), np.float32)})
        kv["k"] = np.concatenate([kv["k"], k.transpose(1, 0, 2)], axis=1)
        kv["v"] = np.concatenate([kv["v"], v.reshape(M, Hkv, hd).transpose(1, 0, 2)], axis=1)
        o = causal_gqa_attention(q, kv["k"], kv["v"], pos0).reshape(M, H * hd)
        if attn_ref is not None:
            attn_ref.append(o)
        if attn_in is not None:
            o = np.asarray(attn_in[li], np.float32).reshape(M, H * hd)
        on = rms_norm_f64acc(o, L["attn_sub_norm"], eps) if L.get("attn_sub_norm") is not None else o
        qo, so = quant_rows(on)
        x = x + w2a8_linear_from_q(qo, so, L["o_proj"][0], L["o_proj"][1])[0]
        f = rms_norm_f64acc(x, L["post_norm"], eps)
        qf, sf = quant_rows(f)
        g = w2a8_linear_from_q(qf, sf, L["gate_proj"][0], L["gate_proj"][1])[0]
        u = w2a8_linear_from_q(qf, sf, L["up_proj"][0], L["up_proj"][1])[0]
        act = relu2_gate(g, u)
        if L.get("ffn_sub_norm") is not None:
            act = rms_norm_f64acc(act, L["ffn_sub_norm"], eps)
        qd, sd = quant_rows(act)
        x = x + w2a8_linear_from_q(qd, sd, L["down_proj"][0], L["down_proj"][1])[0]
    cache["len"] = pos0 + M
    if x_out is not None:
        x_out.append(x)
    hn = rms_norm_f64acc(x, params["final_norm"], eps)
    # the tied head in f64 (products of two f32 values are exact); the f64 copy of the
    # embedding is made once per parameter set (2.6 GB at V = 128256, D = 2560)
    e64 = params.get("_embed_f64")
    if e64 is None:
        e64 = params["_embed_f64"] = bf16_to_f32(params["embed"]).astype(np.float64)
    logits = e64 @ hn[-1].astype(np.float64)
    return hn, logits


def bitnet_greedy(params, cfg, prompt, n):
    """Greedy decode (src/rotor/generation.py:244-279 protocol): prompt, then one token
    per step; returns the n generated ids and the per-step top-2 logit gaps."""
    cache = {}
    _, logits = bitnet_forward(params, cfg, prompt, cache)
    toks, gaps = [], []
    for i in range(n):
        t = int(np.argmax(logits))
        srt = np.sort(logits)
        toks.append(t)
        gaps.append(float(srt[-1] - srt[-2]))
        if i + 1 < n:
            _, logits = bitnet_forward(params, cfg, [t], cache)
    return np.array(toks), np.array(gaps)


def make_bitnet_params(seed, cfg, max_len, sub_norms=True, fast=False):
    """Seeded random-init cfg-4 weights: ternary matrices and scales as in cfg 0,
    norm weights ~U(0.5, 1.5), bf16 embedding ~N(0, 1).  fast=True draws the ternary values
    with make_ternary_fast (the same distribution, another stream of numbers; for the
    30-layer model, where make_ternary takes minutes)."""
    rng = np.random.default_rng(seed)
    ternary = make_ternary_fast if fast else make_ternary
    D, F, H, Hkv, V = cfg["d_model"], cfg["d_ff"], cfg["n_heads"], cfg["n_kv_heads"], cfg["vocab_size"]
    hd = D // H
    shapes = {"q_proj": (H * hd, D), "k_proj": (Hkv * hd, D), "v_proj": (Hkv * hd, D), "o_proj": (D, H * hd),
              "gate_proj": (F, D), "up_proj": (F, D), "down_proj": (D, F)}
    layers = []
    for _ in range(cfg["n_layers"]):
        L = {"input_norm": rng.uniform(0.5, 1.5, D).astype(np.float32),
             "post_norm": rng.uniform(0.5, 1.5, D).astype(np.float32)}
        for name, (n, k) in shapes.items():
            L[name] = ternary(rng, n, k)
        L["attn_sub_norm"] = rng.uniform(0.5, 1.5, D).astype(np.float32) if sub_norms else None
        L["ffn_sub_norm"] = rng.uniform(0.5, 1.5, F).astype(np.float32) if sub_norms else None
        layers.append(L)
    embed = (f32_to_bf16_fast if fast else f32_to_bf16)(rng.standard_normal((V, D), dtype=np.float32))
    final_norm = rng.uniform(0.5, 1.5, D).astype(np.float32)
    return {"layers": layers, "embed": embed, "final_norm": final_norm,
            "rope": rope_table(max_len, hd, cfg.get("rope_theta", 500000.0))}


# ---------------------------------------------------------------------------
# Seeded synthetic inputs (the generators of the benchmark configurations)
# ---------------------------------------------------------------------------


def make_ternary(rng, N, K):
    """W iid with P(-1)=0.3, P(0)=0.4, P(+1)=0.3, then a per-tensor scale ~ U(0.01, 0.05)."""
    W = rng.choice(np.array([-1, 0, 1], dtype=np.int8), size=(N, K), p=[0.3, 0.4, 0.3]).astype(np.int8)
    scale = np.float32(rng.uniform(0.01, 0.05))
    return W, scale


def make_ternary_fast(rng, N, K):
    """As make_ternary, from uniform bytes in [0, 10): 0-2 -> -1, 3-6 -> 0, 7-9 -> +1
    (P = 0.3 / 0.4 / 0.3 exactly), then the scale."""
    u = rng.integers(0, 10, size=(N, K), dtype=np.uint8)
    W = (u >= 7).astype(np.int8) - (u <= 2).astype(np.int8)
    scale = np.float32(rng.uniform(0.01, 0.05))
    return W, scale


def f32_to_bf16_fast(x):
    """f32_to_bf16 in 32-bit integer arithmetic (no overflow for finite inputs)."""
    u = np.asarray(x, np.float32).view(np.uint32)
    return ((u + np.uint32(0x7FFF) + ((u >> np.uint32(16)) & np.uint32(1))) >> np.uint32(16)).astype(np.uint16)


def make_linear_case(seed, M, N, K):
    """One seeded ternary-linear case: (x fp32 [M,K] ~ N(0,1), W int8 [N,K], scale)."""
    rng = np.random.default_rng(seed)
    W, scale = make_ternary(rng, N, K)
    x = rng.standard_normal((M, K), dtype=np.float32)
    return x, W, scale


PINNED = {
    "encode/decode/pack/unpack": "reference KATs (tests/test_core.py:19-34,85-107; src/rotor/bitnet.py:95,345-354; "
                                 "tests/debug_bitnet_format.py:20-27) + oracle/_ref round-trip",
    "pack_rotor/unpack_rotor": "byte KATs 0x86/0x21/0x24/0x12/0x68/0x81/0x60/0x80 + exhaustive 256-byte table vs "
                               "oracle/_ref bitnet_to_rotor+rotor_unpack_weights",
    "bitnet_to_rotor/rotor_unpack_weights": "bit-exact vs oracle/_ref (reference C core) on random and ragged shapes",
    "quant_rows": "KAT [127,.5,1.5,2.5,-.5,-1.5,3.49,-126.5] -> [127,0,2,2,0,-2,3,-126]; zero row; invariants "
                  "(max element -> +-127, |x - q s| <= s/2, scale equivariance)",
    "linear_i64": "brute-force loops on tiny shapes; linear_i64 == linear_i64_fast; linearity in q",
    "linear_ref_f32/ternary_linear": "float64 closed form on the same quantised inputs (|diff| << 3e-4)",
    "rms_norm/relu2_gate/ffn_block": "closed forms: constant rows, unit weight, sign cases",
    "rms_norm_f64acc": "closed forms (constant rows -> +-w); agrees with rms_norm within 1 ulp",
    "ffn_block_w2a8": "composition of pinned functions; equals ffn_block when intermediates agree",
    "bf16/rope/attention/bitnet_forward": "bf16 round trip; RoPE norm preservation, pos-0 identity and frequency "
                                          "KAT; attention closed forms (one key -> V, equal keys -> mean of V, "
                                          "causal prefix, two keys -> logistic mix sig(a/sqrt(hd)) at the score "
                                          "scale 1/sqrt(hd), which 1/hd or no scale fails); incremental decode == "
                                          "full-sequence forward",
}
