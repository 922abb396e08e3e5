"""Benchmark of the MI355X ternary-linear hot path (one GPU).

    python bench.py [--gpus 1] [--steps K] [--warmup W] [--groups G] [--no-cpu]

Workload (BASELINE metric "Ternary GEMV HBM GB/s (% peak) @2560x6912"): the W2A8
ternary GEMV with N=6912 outputs, K=2560 inputs, M=1 token, on seeded synthetic
weights drawn as in the configurations (P(+1)=P(-1)=0.3, P(0)=0.4, per-tensor scale
~U(0.01,0.05)) and x ~ N(0,1).  One *step* applies G distinct weight matrices (G=128:
566 MB of 2-bit weights, more than twice the 256 MB Infinity Cache, so every step
streams its weights from HBM) to G distinct token vectors through one prepared plan,
run as ONE launch: each GEMV workgroup quantises its token (per-token absmax int8) in
its prologue, then streams its row blocks.

value      = algorithmic bytes of the G GEMVs per step / step time (GB/s), where the
             bytes of one GEMV are N*K/4 (2-bit W) + 4*K (fp32 x, read by the fused
             quantiser) + 4*N (fp32 y) + 4 (weight scale); the K steps run back to back
             between two HIP events on the launch stream;
roofline   = the same bytes over the kernel's average launch duration from that same
             timed region (one step is exactly one launch of the kernel), against 8 TB/s;
             profile_kernel_us / profile_frac: the kernel's mean duration in the committed
             rocprofv3 kernel trace of the same command (profiles/gemv_2560x6912_m1_g128.md,
             profile_commit = the commit it was taken on) and the fraction it gives;
two_launch_form = the same plan as a quantiser launch + a GEMV launch (int8 x read
             by the GEMV: N*K/4 + K + 4 + 4*N + 4 bytes per GEMV), for comparison;
cpu_baseline = the reference's CPU path np.dot(x, W_i8.T) * scale
             (src/rotor/transformer.py:150), restated in NumPy, at the configurations'
             shapes with one BLAS thread and with every core of the process's affinity,
             the reference's C core (bit planes -> int8 unpack, the 1-bit-activation
             mat-vec) restated in C and built from its own source, and a capped cfg-4
             CPU decode; `value` is the NumPy rate at the metric's shape with the faster of
             one BLAS thread and all of them (`cores` says which).  The GPU
             result of one metric problem is checked against the oracle in the same leg.
"""
from __future__ import annotations

import argparse
import ctypes
import json
import os
import sys
import time
from pathlib import Path

ROOT = Path(__file__).resolve().parent
for _p in (ROOT / "rotor-rag_amd", ROOT):
    if str(_p) not in sys.path:
        sys.path.insert(0, str(_p))

HBM_PEAK_GBS = 8000.0
INT8_PEAK_TOPS = 5000.0  # MI355X dense int8 MFMA, no sparsity
N_OUT, K_IN = 6912, 2560
METRIC = "Ternary GEMV HBM GB/s (% peak) @2560x6912; BitNet-2B-shape decode tok/s"
D_MODEL, D_FF, HEADS, KV_HEADS, VOCAB = 2560, 6912, 20, 5, 128256
# the seven projections of one BitNet-2B layer: (N, K)
LAYER_SHAPES = {"q_proj": (2560, 2560), "k_proj": (640, 2560), "v_proj": (640, 2560), "o_proj": (2560, 2560),
                "gate_proj": (6912, 2560), "up_proj": (6912, 2560), "down_proj": (2560, 6912)}
# cfg 2's timed plan: (N, K, input index) of q, k, v (input 0), o (1), gate, up (2), down (3)
LAYER_M64_SHAPES = [(2560, 2560, 0), (640, 2560, 0), (640, 2560, 0), (2560, 2560, 1), (6912, 2560, 2), (6912, 2560, 2),
                    (2560, 6912, 3)]

PROFILE = ROOT / "profiles" / "gemv_2560x6912_m1_g128.md"


def profile_fields():
    """The `key: value` lines of the committed metric profile (rocprofv3 summary): the HBM
    bytes per GEMV launch from the PMC passes (FETCH_SIZE/WRITE_SIZE scaled by a plain-copy
    calibration), the kernel's mean duration in the kernel trace and the commit profiled."""
    out = {}
    try:
        for line in PROFILE.read_text().splitlines():
            for key in ("traffic_bytes_per_launch", "profile_kernel_us", "profile_commit"):
                if line.startswith(key + ":"):
                    out[key] = line.split(":", 1)[1].strip()
    except OSError:
        pass
    return out


def gemv_bytes(M, N, K):
    """Algorithmic bytes of one GEMV over int8 activations quantised beforehand."""
    return N * K // 4 + M * K + 4 * M + 4 * M * N + 4


def gemv_bytes_fused(M, N, K):
    """Algorithmic bytes of one GEMV that quantises its fp32 input itself."""
    return N * K // 4 + 4 * M * K + 4 * M * N + 4


def make_weights_device(torch, gen, N, K, device):
    """Seeded rotor bytes [N, K/4] drawn on the device: each 2-bit field is 01 (-1)
    with p=0.3, 10 (+1) with p=0.3, 00 (0) with p=0.4."""
    u = torch.rand((N, K), generator=gen, device=device)
    f = torch.where(u < 0.3, 1, torch.where(u < 0.6, 2, 0)).to(torch.uint8).view(N, K // 4, 4)
    return (f[..., 0] | (f[..., 1] << 2) | (f[..., 2] << 4) | (f[..., 3] << 6)).contiguous()


def events(torch, n=2):
    return [torch.cuda.Event(enable_timing=True) for _ in range(n)]


# ---------------------------------------------------------------------------- GPU legs


def prefill_and_layer(torch, hip, gen, dev, reps=50, layers=20):
    """cfg 3 (prefill GEMMs, M=2048) and cfg 2 (one layer's 7 projections at M=64).

    cfg 3: the activations are quantised once, then `reps` GEMM launches run back to back
    between two events.  cfg 2: `layers` distinct layers (20 x 17.4 MB of weights, more than
    the 256 MB Infinity Cache) as one plan each, their projection launches run back to
    back in rotation, so every launch streams its weights from HBM."""
    out = {}
    M = 2048
    for name, (N, K) in {"gate_up_6912x2560": (6912, 2560), "down_2560x6912": (2560, 6912)}.items():
        w = hip.upload_device(make_weights_device(torch, gen, N, K, dev), K, 0.03)
        x = torch.randn((M, K), generator=gen, device=dev, dtype=torch.float32)
        y = torch.empty((M, N), device=dev, dtype=torch.float32)
        plan = hip.plan([w], [x], [y])
        plan.run()
        plan.gemv()
        torch.cuda.synchronize()
        a, b = events(torch)
        a.record()
        for _ in range(reps):
            plan.gemv()
        b.record()
        torch.cuda.synchronize()
        ms = a.elapsed_time(b) / reps
        ops = 2.0 * M * N * K
        kind, tm, tn, tiles = plan.describe()
        out[name] = {"M": M, "N": N, "K": K, "us": round(ms * 1e3, 2), "TOPS": round(ops / (ms * 1e-3) / 1e12, 1),
                     "mfma_util": round(ops / (ms * 1e-3) / 1e12 / INT8_PEAK_TOPS, 4),
                     "tile": f"{tm}x{tn}", "tiles": tiles, "launches": reps}
        del plan, w, x, y
    M = 64
    shapes = LAYER_M64_SHAPES
    xs_in = [torch.randn((M, K), generator=gen, device=dev, dtype=torch.float32) for K in (2560, 2560, 2560, 6912)]
    ys = [torch.empty((M, N), device=dev, dtype=torch.float32) for N, _, _ in shapes]
    plans, keep = [], []
    for _ in range(layers):
        ws = [hip.upload_device(make_weights_device(torch, gen, N, K, dev), K, 0.03) for N, K, _ in shapes]
        plans.append(hip.plan(ws, [xs_in[xi] for _, _, xi in shapes], ys))
        keep.append(ws)
    for p in plans:
        p.run()
    torch.cuda.synchronize()
    rounds = max(1, reps // 5)
    a, b = events(torch)
    a.record()
    for _ in range(rounds):
        for p in plans:
            p.gemv()
    b.record()
    torch.cuda.synchronize()
    ms = a.elapsed_time(b) / (rounds * layers)
    # the same rotation with the per-row quantisation of the fp32 inputs (cfg 2's x is fp32):
    # run() = one quantiser launch over the 4 distinct inputs + the GEMM launch
    a.record()
    for _ in range(rounds):
        for p in plans:
            p.run()
    b.record()
    torch.cuda.synchronize()
    ms_run = a.elapsed_time(b) / (rounds * layers)
    ops = sum(2.0 * M * N * K for N, K, _ in shapes)
    wbytes = sum(N * K // 4 for N, K, _ in shapes)
    abytes = wbytes + sum(M * K + 4 * M for K in (2560, 2560, 6912)) + sum(4 * M * N for N, _, _ in shapes)
    out["layer_m64_7proj"] = {
        "M": M, "us": round(ms * 1e3, 2), "TOPS": round(ops / (ms * 1e-3) / 1e12, 1),
        "GB_per_s": round(abytes / (ms * 1e-3) / 1e9, 1), "hbm_frac": round(abytes / (ms * 1e-3) / 1e9 / HBM_PEAK_GBS, 4),
        "rotation_MB": round(layers * wbytes / 1e6, 1),
        "with_quantiser_us": round(ms_run * 1e3, 2),
        "workgroups": plans[0].describe()[3],
        "note": f"7 projections of a BitNet-2B layer as one split-K launch (GEMM only: p.gemv(); with_quantiser_us: "
                f"p.run(), the per-row quantisation of the 4 distinct fp32 inputs first); {layers} distinct layers in "
                "rotation (weights stream from HBM); bytes = 2-bit weights + int8 inputs + fp32 outputs"}
    return out


def ffn_block_cfg1(torch, hip, gen, dev, blocks=24, reps=10):
    """cfg 1: RMSNorm -> gate & up -> relu^2(gate)*up -> down at batch 1 (2 launches: the
    gate/up pair plan and the down plan).  `blocks` distinct FFN blocks (24 x 13.3 MB, more
    than the 256 MB Infinity Cache) each run once in a HIP graph, which is replayed; the
    per-block latency and the HBM rate of its weights are reported."""
    from rotor import gpu_layers
    from rotor.ffn import TernaryFFNBlock

    D, F = D_MODEL, D_FF
    to_np = lambda t: t.cpu().numpy()
    blks = []
    gpu_layers._gpu_instance = hip
    try:
        for _ in range(blocks):
            blk = TernaryFFNBlock(D, F, use_gpu=True, max_tokens=1)
            blk.load(torch.rand(D, generator=gen, device=dev).add(0.5).cpu().numpy(),
                     (to_np(make_weights_device(torch, gen, F, D, dev)), 0.03),
                     (to_np(make_weights_device(torch, gen, F, D, dev)), 0.03),
                     (to_np(make_weights_device(torch, gen, D, F, dev)), 0.03))
            blks.append(blk)
    finally:
        gpu_layers._gpu_instance = None
    x = torch.randn((1, D), generator=gen, device=dev)
    for blk in blks:
        blk.forward_device(x)
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        for blk in blks:
            blk.forward_device(x)
    for _ in range(2):
        graph.replay()
    torch.cuda.synchronize()
    a, b = events(torch)
    a.record()
    for _ in range(reps):
        graph.replay()
    b.record()
    torch.cuda.synchronize()
    us = a.elapsed_time(b) / (reps * blocks) * 1e3
    wbytes = 3 * D * F // 4
    abytes = wbytes + 4 * D * 2 + 4 * D + 4 * F * 2  # weights + x, norm w, y + a (fp32) in/out
    return {"us_per_block": round(us, 2), "weight_GB_per_s": round(wbytes / (us * 1e-6) / 1e9, 1),
            "hbm_frac": round(abytes / (us * 1e-6) / 1e9 / HBM_PEAK_GBS, 4), "launches": blks[0].launches(1),
            "rotation_MB": round(blocks * wbytes / 1e6, 1),
            "note": f"batch 1; {blocks} distinct FFN blocks in one graph (weights stream from HBM), replayed "
                    "back to back"}


def build_cfg4_model(torch, hip, gen, dev, n_layers=30, max_seq_len=640, max_batch_tokens=512):
    """The cfg-4 model with seeded random-init weights drawn on the device (the
    configurations' distributions), loaded through BitNetModel.load_state."""
    from rotor import gpu_layers
    from rotor.bitnet_model import BitNetModel

    D, F, H, Hkv, V = D_MODEL, D_FF, HEADS, KV_HEADS, VOCAB
    cfg = dict(vocab_size=V, d_model=D, n_layers=n_layers, n_heads=H, n_kv_heads=Hkv, d_ff=F,
               rope_theta=500000.0, rms_norm_eps=1e-6, max_seq_len=max_seq_len, max_batch_tokens=max_batch_tokens)
    state = {"model.embed_tokens.weight": torch.randn((V, D), generator=gen, device=dev).to(torch.bfloat16),
             "model.norm.weight": torch.rand(D, generator=gen, device=dev) + 0.5}
    for i in range(n_layers):
        p = f"model.layers.{i}"
        state[f"{p}.input_layernorm.weight"] = torch.rand(D, generator=gen, device=dev) + 0.5
        state[f"{p}.post_attention_layernorm.weight"] = torch.rand(D, generator=gen, device=dev) + 0.5
        state[f"{p}.self_attn.attn_sub_norm.weight"] = torch.rand(D, generator=gen, device=dev) + 0.5
        state[f"{p}.mlp.ffn_sub_norm.weight"] = torch.rand(F, generator=gen, device=dev) + 0.5
        for name, (n, k) in LAYER_SHAPES.items():
            grp = "self_attn" if name in ("q_proj", "k_proj", "v_proj", "o_proj") else "mlp"
            state[f"{p}.{grp}.{name}.weight"] = make_weights_device(torch, gen, n, k, dev)
            state[f"{p}.{grp}.{name}.weight_scale"] = torch.rand(1, generator=gen, device=dev) * 0.04 + 0.01
    gpu_layers._gpu_instance = hip
    try:
        model = BitNetModel(cfg, use_gpu=True)
        model.load_state(state)
    finally:
        gpu_layers._gpu_instance = None
    return model


def decode_cfg4(torch, hip, gen, dev, n_layers=30, prompt_len=512, new_tokens=128):
    """cfg 4: 30-layer BitNet-2B-shape random-init model (hidden 2560, ffn 6912, 20/5 heads
    x 128, RoPE, RMSNorm, bf16 tied embedding/LM head over 128256 tokens), 512 random
    prompt ids, greedy decode of 128 tokens with the KV cache, batch 1."""
    import numpy as np

    D, V = D_MODEL, VOCAB
    model = build_cfg4_model(torch, hip, gen, dev, n_layers, prompt_len + new_tokens, prompt_len)
    prompt = np.random.default_rng(4).integers(0, V, prompt_len).astype(np.int32)
    model.generate_greedy(prompt, 8)  # warm-up (kernels, plans, graph)
    t = {}
    toks = model.generate_greedy(prompt, new_tokens, timings=t)
    decode_tok_s = (new_tokens - 1) / (t["decode_ms"] * 1e-3)
    ternary_bytes = n_layers * sum(n * k // 4 for n, k in LAYER_SHAPES.values())
    per_tok_bytes = ternary_bytes + V * D * 2
    return {
        "prefill_ms": round(t["prefill_ms"], 3),
        "prefill_tok_s": round(prompt_len / (t["prefill_ms"] * 1e-3), 1),
        "decode_ms_per_token": round(t["decode_ms"] / (new_tokens - 1), 4),
        "decode_tok_s": round(decode_tok_s, 1),
        "decode_weight_GB_per_s": round(per_tok_bytes * decode_tok_s / 1e9, 1),
        "decode_hbm_frac": round(per_tok_bytes * decode_tok_s / 1e9 / HBM_PEAK_GBS, 4),
        "prompt": prompt_len, "new_tokens": new_tokens, "layers": n_layers,
        "first_tokens": [int(x) for x in toks[:16]],
        "distinct_tokens": int(len(set(int(x) for x in toks))),
        "note": "random-init weights; decode step = one HIP graph replay (30 x (norm+quant, qkv, rope+kv, "
                "attention partials + combine, sub-norm+quant, o+residual, norm+quant, gate/up, relu2+sub-norm+quant, "
                "down+residual), fused final-norm LM head + argmax + next token's embedding).  Runs of one token are "
                "the random-init tied-embedding model's own greedy fixed points (fed token t, t's logit is the "
                "largest), held bit-exact against the oracle in tests/test_gpu_model.py",
    }


# ---------------------------------------------------------------------------- CPU legs


def host_info():
    import numpy as np

    model = "unknown"
    try:
        with open("/proc/cpuinfo") as f:
            model = next((l.split(":", 1)[1].strip() for l in f if l.startswith("model name")), model)
    except OSError:
        pass
    blas = "unknown"
    try:
        b = np.show_config(mode="dicts")["Build Dependencies"]["blas"]
        blas = f"{b.get('name')} {b.get('version')}"
    except Exception:
        pass
    return {"cpu_model": model, "cores_affinity": len(os.sched_getaffinity(0)), "os_cpu_count": os.cpu_count(),
            "numpy": np.__version__, "blas": blas}


def time_calls(fn, budget_s, min_calls=2, warm=True):
    """Median / p10 / p90 ms of fn() over about budget_s seconds (at least min_calls calls)."""
    import numpy as np

    if warm:
        fn()
    times = []
    t_end = time.perf_counter() + budget_s
    while len(times) < min_calls or (time.perf_counter() < t_end and len(times) < 5000):
        t0 = time.perf_counter()
        fn()
        times.append(time.perf_counter() - t0)
    a = np.array(times) * 1e3
    return {"calls": int(a.size), "median_ms": round(float(np.median(a)), 4),
            "p10_ms": round(float(np.percentile(a, 10)), 4), "p90_ms": round(float(np.percentile(a, 90)), 4)}


def rand_ternary(rng, N, K):
    """int8 W [N, K] with P(-1) = P(+1) = 0.3, P(0) = 0.4 (the configurations' draw)."""
    import numpy as np

    u = rng.random((N, K), dtype=np.float32)
    return ((u >= 0.7).astype(np.int8) - (u < 0.3).astype(np.int8))


def cpu_numpy_shapes(budget_s):
    """The reference formula np.dot(x, W_i8.T) * scale at the cfg 0-3 shapes, one BLAS
    thread and every core of the affinity (threadpoolctl)."""
    import numpy as np
    from threadpoolctl import threadpool_limits

    from oracle import rotor_oracle as O

    rng = np.random.default_rng(3)
    cores = len(os.sched_getaffinity(0))
    cases = {
        "cfg0_1x2560x2560": (1, [(2560, 2560)]),
        "metric_1x6912x2560": (1, [(6912, 2560)]),
        "cfg2_64_layer_7proj": (64, list(LAYER_SHAPES.values())),
        "cfg3_2048x6912x2560": (2048, [(6912, 2560)]),
        "cfg3_2048x2560x6912": (2048, [(2560, 6912)]),
    }
    out = {}
    for name, (M, shapes) in cases.items():
        Ws = [rand_ternary(rng, N, K) for N, K in shapes]
        xs = {K: rng.standard_normal((M, K), dtype=np.float32) for _, K in shapes}
        run = lambda: [O.linear_ref_f32(xs[W.shape[1]], W, 0.03) for W in Ws]
        abytes = sum(gemv_bytes_fused(M, W.shape[0], W.shape[1]) for W in Ws)
        ops = sum(2.0 * M * W.shape[0] * W.shape[1] for W in Ws)
        res = {}
        for label, threads in (("threads_1", 1), ("threads_all", cores)):
            with threadpool_limits(limits=threads, user_api="blas"):
                big = M >= 2048 and threads == 1
                t = time_calls(run, budget_s, min_calls=1 if big else 2, warm=not big)
            s = t["median_ms"] * 1e-3
            res[label] = dict(t, threads=threads, GB_per_s=round(abytes / s / 1e9, 4),
                              GOPS=round(ops / s / 1e9, 2))
        out[name] = res
        del Ws, xs
    return out


def _cpubase_libs():
    sz, vp = ctypes.c_size_t, ctypes.c_void_p
    libs = {}
    own = ROOT / "oracle" / "libcpubase.so"
    if own.exists():
        lib = ctypes.CDLL(str(own))
        lib.cb_unpack_planes.argtypes = [vp, vp, sz, sz, vp]
        lib.cb_sign_matvec.argtypes = [vp, vp, vp, sz, sz, vp, vp, vp]
        libs["port"] = (lib.cb_unpack_planes, lambda b0, b1, x, m, n, s0, s1, y: lib.cb_sign_matvec(
            b0, b1, x, m, n, s0, s1, y))
    ref = ROOT / "oracle" / "_ref" / "librotor_core.so"
    if ref.exists():  # the reference's own C core, compiled from its source by oracle/Makefile
        rl = ctypes.CDLL(str(ref))
        rl.rotor_unpack_weights.argtypes = [vp, vp, sz, sz, vp]
        rl.rotor_matvec.argtypes = [vp, vp, vp, sz, sz, vp]
        libs["reference"] = (rl.rotor_unpack_weights, lambda b0, b1, x, m, n, s0, s1, y: rl.rotor_matvec(
            b0, b1, x, m, n, y))
    return libs


def cpu_c_core(budget_s):
    """The reference's C core at the metric's shape (6912 x 2560), single-threaded: the
    load-time bit planes -> int8 unpack (native/c/rotor_core.c:270-299) and the
    1-bit-activation mat-vec (rotor_matvec, :305-331 with rotor_dot :102-162), as this
    build's C restatement (kind port) and as the reference's own source compiled by
    oracle/Makefile (kind reference)."""
    import numpy as np

    from oracle import rotor_oracle as O

    rng = np.random.default_rng(5)
    N, K = N_OUT, K_IN
    W = rand_ternary(rng, N, K)
    b0, b1 = O.bitnet_to_rotor(O.pack_rotor(W), K)
    wb0, wb1 = np.ascontiguousarray((W == 1).astype(np.uint8)), np.ascontiguousarray((W == -1).astype(np.uint8))
    x = rng.standard_normal(K).astype(np.float32)
    out = {}
    for kind, (unpack, matvec) in _cpubase_libs().items():
        dst = np.empty((N, K), np.int8)
        t_u = time_calls(lambda: unpack(b0.ctypes.data, b1.ctypes.data, N, K, dst.ctypes.data), budget_s / 4)
        assert np.array_equal(dst, W), f"{kind} unpack differs"
        y = np.empty(N, np.int32)
        s0, s1 = np.empty(K, np.uint8), np.empty(K, np.uint8)
        t_m = time_calls(lambda: matvec(wb0.ctypes.data, wb1.ctypes.data, x.ctypes.data, N, K, s0.ctypes.data,
                                        s1.ctypes.data, y.ctypes.data), budget_s / 4)
        assert np.array_equal(y.astype(np.int64), W.astype(np.int64) @ np.sign(x).astype(np.int64))
        out[kind] = {
            "unpack_planes_to_int8": dict(t_u, M_weights_per_s=round(N * K / (t_u["median_ms"] * 1e-3) / 1e6, 1)),
            "sign_matvec_1bit_activations": dict(t_m, M_weights_per_s=round(N * K / (t_m["median_ms"] * 1e-3) / 1e6, 1),
                                                 note="1-bit activations: different numerics, not parity-equivalent"),
            "threads": 1}
    return out


def cpu_decode_cfg4(torch, gen, dev, steps=2, n_layers=30):
    """Capped cfg-4 CPU decode with the reference's NumPy formulas: every ternary
    projection np.dot(a, W_i8.T) * scale (src/rotor/transformer.py:150) on the int8
    weights_cache, the tied LM head np.dot(h, E.T) in fp32 (src/rotor/bitnet_model.py:235),
    RoPE, causal GQA attention and RMSNorms as in the cfg-4 model.  Weights are drawn on the
    GPU with the same generator and copied to the host.  Cap: `steps` tokens decoded after
    a one-token prompt, so attention spans at most steps + 1 keys (at the 512-token prompt
    it would add well under 1 % of the per-token work)."""
    import numpy as np
    from threadpoolctl import threadpool_limits

    from oracle import rotor_oracle as O

    D, F, H, Hkv = D_MODEL, D_FF, HEADS, KV_HEADS
    hd = D // H
    layers = []
    for _ in range(n_layers):
        L = {}
        for name, (n, k) in LAYER_SHAPES.items():
            u = torch.rand((n, k), generator=gen, device=dev)
            L[name] = (torch.where(u < 0.3, -1, torch.where(u < 0.6, 1, 0)).to(torch.int8).cpu().numpy(), 0.03)
        for nm, n in (("in", D), ("post", D), ("attn_sub", D), ("ffn_sub", F)):
            L[nm] = np.random.default_rng(len(layers)).uniform(0.5, 1.5, n).astype(np.float32)
        layers.append(L)
    emb = torch.randn((VOCAB, D), generator=gen, device=dev).to(torch.bfloat16).float().cpu().numpy()
    final = np.ones(D, np.float32)
    rope = O.rope_table(steps + 2, hd, 500000.0)
    kc = [np.zeros((Hkv, 0, hd), np.float32) for _ in range(n_layers)]
    vc = [np.zeros((Hkv, 0, hd), np.float32) for _ in range(n_layers)]
    lin = O.linear_ref_f32

    def step(tok, pos):
        x = emb[tok][None].copy()
        for li, L in enumerate(layers):
            a = O.rms_norm(x, L["in"])
            q = lin(a, *L["q_proj"]).reshape(1, H, hd)
            k = lin(a, *L["k_proj"]).reshape(1, Hkv, hd)
            v = lin(a, *L["v_proj"]).reshape(1, Hkv, hd)
            q, k = O.apply_rope(q, rope, pos), O.apply_rope(k, rope, pos)
            kc[li] = np.concatenate([kc[li], k.transpose(1, 0, 2)], axis=1)
            vc[li] = np.concatenate([vc[li], v.transpose(1, 0, 2)], axis=1)
            o = O.causal_gqa_attention(q, kc[li], vc[li], pos).reshape(1, D)
            x = x + lin(O.rms_norm(o, L["attn_sub"]), *L["o_proj"])
            f = O.rms_norm(x, L["post"])
            g, u = lin(f, *L["gate_proj"]), lin(f, *L["up_proj"])
            x = x + lin(O.rms_norm(O.relu2_gate(g, u), L["ffn_sub"]), *L["down_proj"])
        logits = np.dot(O.rms_norm(x, final), emb.T)[0]
        return int(np.argmax(logits))

    cores = len(os.sched_getaffinity(0))
    with threadpool_limits(limits=cores, user_api="blas"):
        tok = step(1, 0)  # the one-token prompt
        t0 = time.perf_counter()
        for s in range(steps):
            tok = step(tok, s + 1)
        dt = (time.perf_counter() - t0) / steps
    return {"ms_per_token": round(dt * 1e3, 1), "tok_s": round(1.0 / dt, 4), "threads": cores,
            "layers": n_layers, "decode_steps": steps,
            "cap": f"{steps} decode steps after a 1-token prompt (attention over <= {steps + 1} keys)"}


def cpu_baseline(hip, w0, x0, y0, torch, gen, dev, budget_s=1.0, model_steps=2):
    """The reference's CPU path timed on this host, plus the parity check of one GPU
    problem (int32 bit-exact, fp32 within 3e-4 of the NumPy formula)."""
    import numpy as np

    from oracle import rotor_oracle as O

    W = O.unpack_rotor(w0.download(), K_IN)
    x = x0.cpu().numpy()
    scale = np.float32(w0.scale)
    y_ref, q, s, acc = O.ternary_linear(x, W, scale)
    parity = bool(np.allclose(y0.cpu().numpy(), y_ref, atol=3e-4, rtol=1e-5))
    acc_gpu = hip.linear_i32(w0, torch.from_numpy(q)).cpu().numpy().astype(np.int64)
    parity = parity and bool(np.array_equal(acc_gpu, acc))
    info = host_info()
    shapes = cpu_numpy_shapes(budget_s)
    c_core = cpu_c_core(budget_s)
    model = cpu_decode_cfg4(torch, gen, dev, steps=model_steps) if model_steps > 0 else None
    # the faster of the two thread settings at the metric's shape (one BLAS thread usually
    # wins at M = 1: the int8 -> fp32 cast of the weights is single-threaded either way)
    m = max(shapes["metric_1x6912x2560"].values(), key=lambda r: r["GB_per_s"])
    return {
        "value": m["GB_per_s"],
        "unit": "GB/s",
        "cores": m["threads"],
        "kind": "port",
        "sample": f"np.dot(x, W_i8.T)*scale (src/rotor/transformer.py:150) at M=1, 2560->6912 (the metric's shape), "
                  f"{m['calls']} calls, median {m['median_ms']:.3f} ms (p10 {m['p10_ms']:.3f}, p90 {m['p90_ms']:.3f}), "
                  f"{m['threads']} BLAS thread(s), the faster of 1 and all {info['cores_affinity']} cores of the "
                  f"affinity; GB/s from the same algorithmic bytes as the GPU; host {info['cpu_model']}, "
                  f"{info['blas']}, NumPy {info['numpy']}",
        "host": info,
        "numpy_formula": shapes,
        "c_core": c_core,
        "cfg4_decode": model,
    }, parity


# ---------------------------------------------------------------------------- main


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=100)
    ap.add_argument("--warmup", type=int, default=10)
    ap.add_argument("--groups", type=int, default=128)
    ap.add_argument("--no-cpu", action="store_true")
    ap.add_argument("--cpu-budget", type=float, default=1.0, help="seconds per CPU timing")
    ap.add_argument("--cpu-model-steps", type=int, default=2, help="capped cfg-4 CPU decode steps (0: skip)")
    ap.add_argument("--no-extra", action="store_true", help="skip the prefill / M=64 layer / FFN block measurements")
    ap.add_argument("--no-model", action="store_true", help="skip the cfg-4 decode measurement")
    ap.add_argument("--extra-reps", type=int, default=50,
                    help="launches per cfg-3 GEMM timing (cfg-2 rounds: a fifth of it; profiler runs use few)")
    ap.add_argument("--copy-calib", type=int, default=0, metavar="MIB",
                    help="run one plain device copy of MIB MiB first (reference point for HBM counters)")
    args = ap.parse_args()
    if args.gpus != 1:
        print("bench.py measures one GPU: this build's hot path runs on a single MI355X "
              "(multi-GPU sharding is a design note only); use --gpus 1", file=sys.stderr)
        sys.exit(2)

    import numpy as np
    import torch

    from rotor.gpu_ternary import HIPTernaryOps

    dev = torch.device("cuda", 0)
    hip = HIPTernaryOps(0)
    G = args.groups
    gen = torch.Generator(device=dev)
    gen.manual_seed(1)
    rng = np.random.default_rng(1)
    ws, xs, ys = [], [], []
    for g in range(G):
        wb = make_weights_device(torch, gen, N_OUT, K_IN, dev)
        ws.append(hip.upload_device(wb, K_IN, float(np.float32(rng.uniform(0.01, 0.05)))))
        del wb
        xs.append(torch.randn((1, K_IN), generator=gen, device=dev, dtype=torch.float32))
        ys.append(torch.empty((1, N_OUT), device=dev, dtype=torch.float32))
    plan = hip.plan(ws, xs, ys)
    torch.cuda.synchronize()
    if args.copy_calib:
        # an elementwise kernel that reads and writes exactly MIB MiB each
        src = torch.ones((args.copy_calib << 20) // 4, dtype=torch.float32, device=dev)
        dst = torch.empty_like(src)
        torch.cuda.synchronize()
        torch.neg(src, out=dst)
        torch.cuda.synchronize()
        del src, dst
    print(f"bench: {G} x ternary GEMV {K_IN}->{N_OUT}, M=1; warmup {args.warmup}, steps {args.steps}",
          file=sys.stderr, flush=True)

    for _ in range(args.warmup):
        plan.run()
    torch.cuda.synchronize()

    # Timed region: the K steps back to back between two events on torch's current stream,
    # which the backend binds its launches to (an event between launches would put a
    # marker packet, and a gap, between them).  One step is one launch of the GEMV kernel,
    # so the step time is also the kernel's average launch duration.
    t0 = time.perf_counter()
    start, end = events(torch)
    start.record()
    for _ in range(args.steps):
        plan.run()
    end.record()
    torch.cuda.synchronize()
    wall = time.perf_counter() - t0
    step_ms = start.elapsed_time(end) / args.steps
    bytes_step = G * gemv_bytes_fused(1, N_OUT, K_IN)
    value = bytes_step / (step_ms * 1e-3) / 1e9
    # isolated launches, one between two events each (includes the event gaps): diagnostic
    ev = [events(torch) for _ in range(args.steps)]
    for e0, e1 in ev:
        e0.record()
        plan.run()
        e1.record()
    torch.cuda.synchronize()
    run_ms = np.array([e0.elapsed_time(e1) for e0, e1 in ev])
    run_dist = {"p10": round(float(np.percentile(run_ms, 10)), 5), "p50": round(float(np.median(run_ms)), 5),
                "p90": round(float(np.percentile(run_ms, 90)), 5), "n": int(run_ms.size)}

    # the same plan as two launches (quantiser, then GEMV over int8 activations), back to back
    plan.quantize()
    plan.gemv()
    torch.cuda.synchronize()
    a, b = events(torch)
    a.record()
    for _ in range(args.steps):
        plan.quantize()
        plan.gemv()
    b.record()
    torch.cuda.synchronize()
    two_step_ms = a.elapsed_time(b) / args.steps
    a.record()
    for _ in range(args.steps):
        plan.gemv()
    b.record()
    torch.cuda.synchronize()
    gemv_avg = a.elapsed_time(b) / args.steps

    # single-launch latency: one rt_linear_f32 per call, rotating over the G matrices
    lat = []
    for rep in range(3):
        for g in range(G):
            e0, e1 = events(torch)
            e0.record()
            hip.linear_device(ws[g], xs[g], out=ys[g])
            e1.record()
            lat.append((e0, e1))
    torch.cuda.synchronize()
    single_ms = float(np.median([e0.elapsed_time(e1) for e0, e1 in lat[G:]]))

    extra = None
    if not args.no_extra:
        print("bench: cfg-3 prefill GEMMs, cfg-2 layer rotation, cfg-1 FFN block rotation", file=sys.stderr, flush=True)
        extra = prefill_and_layer(torch, hip, gen, dev, reps=args.extra_reps)
        extra["cfg1_ffn_block_m1"] = ffn_block_cfg1(torch, hip, gen, dev)
    cfg4 = None
    if not args.no_model:
        print("bench: cfg-4 decode (30 layers, 512 prompt + 128 greedy tokens)", file=sys.stderr, flush=True)
        cfg4 = decode_cfg4(torch, hip, gen, dev)

    # re-run the plan so ys[0] holds the plan's output for the parity check
    plan.run()
    torch.cuda.synchronize()
    cpu = None
    parity = None
    if not args.no_cpu:
        print("bench: cpu_baseline leg (reference CPU path on this host)", file=sys.stderr, flush=True)
        cpu, parity = cpu_baseline(hip, ws[0], xs[0], ys[0], torch, gen, dev, budget_s=args.cpu_budget,
                                   model_steps=args.cpu_model_steps)

    prof = profile_fields() if G == 128 else {}
    prof_us = float(prof["profile_kernel_us"]) if "profile_kernel_us" in prof else None
    out = {
        "metric": METRIC,
        "value": round(value, 2),
        "unit": "GB/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(step_ms, 5),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "i8",
        "data": "synthetic (seeded ternary weights P(+-1)=0.3, scales U(0.01,0.05), x~N(0,1))",
        "config": {
            "workload": f"W2A8 ternary GEMV 2560->6912, M=1, {G} distinct weight matrices per step "
                        f"({G * N_OUT * K_IN // 4 / 1e6:.0f} MB of 2-bit weights) in one plan, one launch "
                        "per step (each workgroup quantises its token in the GEMV prologue)",
            "N": N_OUT, "K": K_IN, "M": 1, "matrices_per_step": G,
        },
        "pct_hbm_peak": round(100 * value / HBM_PEAK_GBS, 2),
        "roofline": {
            "bound": "hbm",
            "achieved": round(value, 2),
            "peak": HBM_PEAK_GBS,
            "unit": "GB/s",
            "frac": round(value / HBM_PEAK_GBS, 4),
            "traffic": int(prof["traffic_bytes_per_launch"]) if G == 128 and "traffic_bytes_per_launch" in prof else None,
            "traffic_source": "profiles/gemv_2560x6912_m1_g128.md (rocprofv3 FETCH_SIZE+WRITE_SIZE, copy-calibrated)",
            "kernel": "rt::gemv_rows_kernel<1, 1>",
            "bytes_per_launch": bytes_step,
            "avg_launch_ms": round(step_ms, 5),
            "timing": "HIP events around the timed region's back-to-back launches (one launch per step)",
            "isolated_launch_ms_dist": run_dist,
            # the same fraction from the committed rocprofv3 kernel trace of this workload (the
            # kernel's mean duration there; another run on another box)
            "profile_kernel_us": prof_us,
            "profile_frac": round(bytes_step / (prof_us * 1e-6) / 1e9 / HBM_PEAK_GBS, 4) if prof_us else None,
            "profile_commit": prof.get("profile_commit"),
        },
        "two_launch_form": {
            "step_ms": round(two_step_ms, 5),
            "gemv_kernel_avg_ms": round(gemv_avg, 5),
            "gemv_kernel": "rt::gemv_rows_kernel<1, 0>",
            "gemv_GB_per_s": round(G * gemv_bytes(1, N_OUT, K_IN) / (gemv_avg * 1e-3) / 1e9, 1),
            "step_GB_per_s": round(G * gemv_bytes(1, N_OUT, K_IN) / (two_step_ms * 1e-3) / 1e9, 1),
        },
        "single_gemv": {
            "us_per_call": round(single_ms * 1e3, 2),
            "GB_per_s": round(gemv_bytes_fused(1, N_OUT, K_IN) / (single_ms * 1e-3) / 1e9, 1),
            "note": "one rt_linear_f32 per matrix (one launch: the GEMV quantises x in its prologue), "
                    "rotating over the G matrices; the latency a single TernaryLinear.forward call sees",
        },
        "cfg3_prefill_and_cfg2_layer": extra,
        "cfg4_decode": cfg4,
        "cpu_baseline": cpu,
        "parity_checked": parity,
        "wall_s": round(wall, 3),
    }
    print(json.dumps(out))


if __name__ == "__main__":
    main()
