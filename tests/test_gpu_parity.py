"""GPU parity of the HIP ternary-linear path against the CPU oracle (through the C ABI).

Bar: bit-exact int8 quantisation and int32 accumulators (vs int64 NumPy on the same
quantised inputs); fp32 outputs within atol 3e-4 / rtol 1e-5 of the reference's
NumPy formula np.dot(x_hat, W.T) * scale evaluated on the same quantised inputs.
"""
import numpy as np
import pytest

from oracle import rotor_oracle as O

pytestmark = pytest.mark.gpu

ATOL, RTOL = 3e-4, 1e-5

# (M, N, K): the BASELINE shapes at decode plus ragged edge cases
LINEAR_CASES = [
    (1, 2560, 2560),   # cfg 0
    (1, 6912, 2560),   # metric shape (gate/up)
    (1, 2560, 6912),   # down
    (1, 640, 2560),    # k/v
    (2, 6912, 2560),
    (3, 2560, 2560),
    (4, 640, 2560),
    (5, 2560, 6912),
    (8, 6912, 2560),
    (13, 2560, 2560),
    (64, 640, 2560),   # cfg 2 M
    (1, 1, 1),
    (1, 7, 5),
    (3, 77, 130),
    (9, 65, 63),
    (2, 129, 1000),
    # int8-MFMA GEMM path (M > 8)
    (16, 640, 2560),
    (100, 300, 256),
    (129, 2560, 2560),
    (256, 6912, 2560),
    (512, 2560, 6912),
    (2048, 6912, 2560),  # cfg 3 (gate/up)
    (2048, 2560, 6912),  # cfg 3 (down): 128 x 160 regions, K split over the waves
    (2000, 2500, 4224),  # regions with rows past M and a last region of 100 columns, 33 chunks per K half
    (2000, 2500, 4160),  # the same with an odd chunk count: no regions (192-row tiles)
    (2000, 2560, 640),   # 192-row tiles, the last one past the 256-row padding
    (200, 13824, 256),   # the same with two row tiles
]


def _case(seed, M, N, K):
    return O.make_linear_case(seed, M, N, K)


@pytest.mark.parametrize("M,K", [(1, 2560), (64, 2560), (2048, 2560 // 8), (3, 6912), (5, 17), (1, 1), (70, 100), (2, 20000), (3, 16384), (2, 2576), (2, 16400)])
def test_quantize_rows_bit_exact(hip, M, K):
    import torch

    rng = np.random.default_rng(M * 1000 + K)
    x = rng.standard_normal((M, K), dtype=np.float32) * rng.uniform(0.001, 50, size=(M, 1)).astype(np.float32)
    if M > 2:
        x[1] = 0.0  # all-zero row -> s = 1, q = 0
    q, s = hip.quantize_rows(torch.from_numpy(x))
    qo, so = O.quant_rows(x)
    assert np.array_equal(s.cpu().numpy(), so)
    assert np.array_equal(q.cpu().numpy(), qo)


def test_quantize_kat(hip):
    import json
    from pathlib import Path

    import torch

    k = json.loads((Path(__file__).parent / "golden" / "kats.json").read_text())["quant"]
    q, s = hip.quantize_rows(torch.tensor([k["x"]], dtype=torch.float32))
    assert q.cpu().numpy()[0].tolist() == k["q"] and float(s.cpu()[0]) == k["s"]


@pytest.mark.parametrize("M,N,K", LINEAR_CASES)
def test_linear_i32_bit_exact(hip, M, N, K):
    import torch

    rng = np.random.default_rng(M + 7 * N + 13 * K)
    W = rng.choice(np.array([-1, 0, 1], np.int8), size=(N, K), p=[0.3, 0.4, 0.3])
    q = rng.integers(-128, 128, size=(M, K), dtype=np.int8)  # full int8 range incl. -128
    w = hip.upload(O.pack_rotor(W), K, 1.0)
    acc = hip.linear_i32(w, torch.from_numpy(q)).cpu().numpy()
    assert np.array_equal(acc.astype(np.int64), O.linear_i64_fast(q, W))


@pytest.mark.parametrize("M,N,K", LINEAR_CASES)
def test_linear_f32_parity(hip, M, N, K):
    import torch

    x, W, scale = _case(M * 31 + N + K, M, N, K)
    w = hip.upload(O.pack_rotor(W), K, scale)
    y = hip.linear_device(w, torch.from_numpy(x)).cpu().numpy()
    y_ref, q, s, acc = O.ternary_linear(x, W, scale)
    np.testing.assert_allclose(y, y_ref, atol=ATOL, rtol=RTOL)
    # the fp32 epilogue is exactly ((float)acc * s_x) * s_w
    y_exact = (acc.astype(np.float32) * s[:, None]) * np.float32(scale)
    assert np.array_equal(y, y_exact)


@pytest.mark.parametrize("M,N,K", [(2048, 2560, 6912), (300, 2560, 2560), (2000, 2500, 4224), (2000, 2500, 4160)])
def test_gemm_residual_epilogue(hip, M, N, K):
    """The GEMM epilogue with a residual (region and tile kernels): y = r + ((acc s_x) s_w),
    each a separate fp32 operation."""
    import torch

    rng = np.random.default_rng(M + N + K)
    x = rng.standard_normal((M, K), dtype=np.float32)
    W, scale = O.make_ternary(rng, N, K)
    r = rng.standard_normal((M, N), dtype=np.float32)
    w = hip.upload(O.pack_rotor(W), K, scale)
    act = hip.activations(M, K)
    hip.act_quantize(torch.from_numpy(x).cuda(), act)
    y = hip.linear_act(w, act, residual=torch.from_numpy(r).cuda()).cpu().numpy()
    _, q, s, acc = O.ternary_linear(x, W, scale)
    assert np.array_equal(y, r + (acc.astype(np.float32) * s[:, None]) * np.float32(scale))


def test_extreme_accumulators(hip):
    import torch

    K = 6912
    W = np.stack([np.ones(K, np.int8), -np.ones(K, np.int8), np.zeros(K, np.int8)])
    q = np.full((2, K), -128, np.int8)
    q[1] = 127
    w = hip.upload(O.pack_rotor(W), K, 1.0)
    acc = hip.linear_i32(w, torch.from_numpy(q)).cpu().numpy()
    assert acc.tolist() == [[-128 * K, 128 * K, 0], [127 * K, -127 * K, 0]]


@pytest.mark.parametrize("M", [3, 16, 100])  # GEMV, split-K GEMM, tile GEMM
def test_error_codes_in_weights_decode_to_zero(hip, M):
    import torch

    rng = np.random.default_rng(9 + M)
    raw = rng.integers(0, 256, size=(70, 40), dtype=np.uint8)  # includes reserved 11 codes
    K = 160
    W = O.unpack_rotor(raw, K)
    q = rng.integers(-128, 128, size=(M, K), dtype=np.int8)
    w = hip.upload(raw, K, 1.0)
    acc = hip.linear_i32(w, torch.from_numpy(q)).cpu().numpy()
    assert np.array_equal(acc.astype(np.int64), O.linear_i64(q, W))


def test_download_canonicalises_reserved_codes(hip):
    # the device holds w + 1, so the reserved rotor code 11 (value 0) comes back as 00;
    # every other code, and the values, round-trip
    rng = np.random.default_rng(11)
    K = 157  # ragged: the last byte holds one element
    raw = rng.integers(0, 256, size=(70, (K + 3) // 4), dtype=np.uint8)
    back = hip.upload(raw, K, 1.0).download()
    W = O.unpack_rotor(raw, K)
    assert np.array_equal(O.unpack_rotor(back, K), W)
    assert np.array_equal(back, O.pack_rotor(W))


@pytest.mark.parametrize("N,K", [(2560, 2560), (77, 130), (1, 5), (640, 2560)])
def test_upload_download_roundtrip(hip, N, K):
    rng = np.random.default_rng(N + K)
    W = rng.choice(np.array([-1, 0, 1], np.int8), size=(N, K))
    p = O.pack_rotor(W)
    w = hip.upload(p, K, 0.5)
    assert np.array_equal(w.download(), p)
    # the same from device bytes
    w2 = hip.upload_device(p, K, 0.5)
    assert np.array_equal(w2.download(), p)


def test_ternary_matmul_duck_type(hip):
    x, W, _ = _case(3, 1, 300, 256)
    scales = np.random.default_rng(4).uniform(0.01, 0.05, 300).astype(np.float32)
    packed = hip.pack_ternary_weights(W)
    y = hip.ternary_matmul(packed, scales, x[0], 256, 300)
    q, s = O.quant_rows(x)
    y_ref = (O.linear_i64(q, W)[0].astype(np.float32) * s[0]) * scales
    np.testing.assert_allclose(y, y_ref, atol=ATOL, rtol=RTOL)
    assert y.shape == (300,)


# launch each plan of test_plan_matches_single_calls makes: (kind, tile_m, tile_n, workgroups)
# (two distinct inputs at M = 1: the GEMV runs after a quantiser launch, 16-wave K split)
PLAN_LAUNCH = {1: (0, 1, 64, 100), 16: (2, 64, 64, 180), 37: (2, 64, 64, 180), 64: (2, 64, 64, 180),
               130: (3, 64, 128, 150), 300: (3, 128, 128, 150), 600: (3, 192, 128, 200)}


@pytest.mark.parametrize("M", [1, 16, 37, 64, 130, 300, 600])
def test_plan_matches_single_calls(hip, M):
    """A plan launches its problems together: one grid over all row blocks for M <= 64 (the
    K = 6912 problem cut into 3 parts of about the other problems' 40 chunks, combined by
    the last part of each row block; replayed, which needs its counters reset), one grid
    over all tiles above (M = 130: 64 x 128 tiles, M = 300: 128 x 128, M = 600: 192 x 128,
    as rt_plan_describe reports), while the single calls pick their own shapes."""
    import torch

    rng = np.random.default_rng(12 + M)
    x1 = torch.from_numpy(rng.standard_normal((M, 2560), dtype=np.float32)).cuda()
    x2 = torch.from_numpy(rng.standard_normal((M, 6912), dtype=np.float32)).cuda()
    shapes = [(2560, 2560, x1), (640, 2560, x1), (640, 2560, x1), (2560, 6912, x2)]
    ws, xs, ys = [], [], []
    for i, (N, K, x) in enumerate(shapes):
        W, scale = O.make_ternary(rng, N, K)
        ws.append(hip.upload(O.pack_rotor(W), K, scale))
        xs.append(x)
        ys.append(torch.empty((M, N), dtype=torch.float32, device="cuda"))
    plan = hip.plan(ws, xs, ys)
    assert plan.describe() == PLAN_LAUNCH[M]
    for _ in range(2):  # replays give the same answer
        plan.run()
        torch.cuda.synchronize()
        for w, x, y in zip(ws, xs, ys):
            assert torch.equal(y, hip.linear_device(w, x))


# cfg 2's timed plan (bench.py LAYER_M64_SHAPES): the seven projections of a BitNet-2B
# layer at M = 64 as ONE split-K launch, q / k / v sharing input 0, o input 1, gate / up input
# 2, down (K = 6912) input 3 and cut into parts
CFG2_SHAPES = [(2560, 2560, 0), (640, 2560, 0), (640, 2560, 0), (2560, 2560, 1), (6912, 2560, 2), (6912, 2560, 2),
               (2560, 6912, 3)]


def test_cfg2_layer_plan_vs_oracle(hip):
    """The exact plan bench.py times for cfg 2: one split-K launch of 436 workgroups (the 356
    row blocks, down's 40 in three parts), every output bit-exact against the oracle's
    int64 accumulators and exact epilogue, on two runs (the parts' arrival counts reset
    themselves) and with the quantiser (run) or on activations quantised before (gemv)."""
    import torch

    from rotor import _hip as H_

    M = 64
    rng = np.random.default_rng(64)
    inputs = [rng.standard_normal((M, K), dtype=np.float32) for K in (2560, 2560, 2560, 6912)]
    xd = [torch.from_numpy(x).cuda() for x in inputs]
    Ws, ws, ys = [], [], []
    for N, K, _ in CFG2_SHAPES:
        W, scale = O.make_ternary(rng, N, K)
        Ws.append((W, scale))
        ws.append(hip.upload(O.pack_rotor(W), K, scale))
        ys.append(torch.full((M, N), float("nan"), dtype=torch.float32, device="cuda"))
    plan = hip.plan(ws, [xd[xi] for _, _, xi in CFG2_SHAPES], ys)
    assert plan.describe() == (H_.LAUNCH_SPLITK, 64, 64, 436)
    for rep in range(3):
        for y in ys:
            y.fill_(float("nan"))
        if rep < 2:
            plan.run()
        else:
            plan.gemv()  # the activations of the previous run are still in place
        torch.cuda.synchronize()
        for (W, scale), (N, K, xi), y in zip(Ws, CFG2_SHAPES, ys):
            _, q, s_, acc = O.ternary_linear(inputs[xi], W, scale)
            y_exact = (acc.astype(np.float32) * s_[:, None]) * np.float32(scale)
            assert np.array_equal(y.cpu().numpy(), y_exact), f"run {rep}: projection {N}x{K} (input {xi})"


@pytest.mark.parametrize("K_long,parts", [(1280, 2), (1920, 3), (2560, 4), (3200, 5), (7040, 8)])
def test_splitk_parts_vs_oracle(hip, K_long, parts):
    """A split-K plan (M = 33) whose long problem is cut into 2-8 parts of about the short
    problem's 10 chunks: the last part of each row block to arrive adds the other parts'
    tiles and resets the row block's count for the next run.  Ragged N on both problems;
    every output bit-exact against the oracle on three runs."""
    import torch

    from rotor import _hip as H_

    M = 33
    rng = np.random.default_rng(K_long)
    shapes = [(100, 640), (200, K_long)]  # 2 and 4 row blocks
    ws, xs, ys, cases = [], [], [], []
    for N, K in shapes:
        x = rng.standard_normal((M, K), dtype=np.float32)
        W, scale = O.make_ternary(rng, N, K)
        cases.append((x, W, scale))
        ws.append(hip.upload(O.pack_rotor(W), K, scale))
        xs.append(torch.from_numpy(x).cuda())
        ys.append(torch.empty((M, N), dtype=torch.float32, device="cuda"))
    plan = hip.plan(ws, xs, ys)
    assert plan.describe() == (H_.LAUNCH_SPLITK, 64, 64, 2 + 4 * parts)
    for rep in range(3):
        for y in ys:
            y.fill_(float("nan"))
        plan.run()
        torch.cuda.synchronize()
        for (x, W, scale), y in zip(cases, ys):
            _, q, s_, acc = O.ternary_linear(x, W, scale)
            y_exact = (acc.astype(np.float32) * s_[:, None]) * np.float32(scale)
            assert np.array_equal(y.cpu().numpy(), y_exact), f"run {rep}: {y.shape[1]}x{x.shape[1]}"


@pytest.mark.parametrize("G", [3, 16, 17, 20])
@pytest.mark.parametrize("M", [20, 100])
def test_grouped_gemm_descriptor_lookup(hip, G, M):
    """A grouped GEMM launch finds a workgroup's problem from the first units of problems
    1.. passed in its arguments (up to 16 problems) or from its unit table (17 and more):
    both give every problem's output bit-exact against its single call (split-K at M = 20,
    tiles at M = 100; problems of 1-3 row blocks and two K, two shared inputs)."""
    import torch

    rng = np.random.default_rng(1000 * G + M)
    xs_by_k = {K: torch.from_numpy(rng.standard_normal((M, K), dtype=np.float32)).cuda() for K in (256, 640)}
    ws, xs, ys = [], [], []
    for g in range(G):
        N, K = 64 * (1 + g % 3) - (g % 2) * 7, (256, 640)[g % 2]
        W, scale = O.make_ternary(rng, N, K)
        ws.append(hip.upload(O.pack_rotor(W), K, scale))
        xs.append(xs_by_k[K])
        ys.append(torch.full((M, N), float("nan"), dtype=torch.float32, device="cuda"))
    plan = hip.plan(ws, xs, ys)
    for _ in range(2):
        plan.run()
        torch.cuda.synchronize()
        for g, (w, x, y) in enumerate(zip(ws, xs, ys)):
            assert torch.equal(y, hip.linear_device(w, x)), f"problem {g}"


@pytest.mark.parametrize("K", [64, 128, 192, 256, 320, 384, 448, 576, 704])
def test_tile256_short_k(hip, K):
    """The 256 x 256 tile (cfg 3 gate/up shape) with K of 1 to 11 chunks: fewer chunks than
    its ring holds, about as many, and a few more (the ring's fill, steady state and tail),
    every output bit-exact against the oracle."""
    import torch

    from rotor import _hip as H_

    M, N = 2048, 6912
    rng = np.random.default_rng(K)
    x = rng.standard_normal((M, K), dtype=np.float32)
    W, scale = O.make_ternary(rng, N, K)
    w = hip.upload(O.pack_rotor(W), K, scale)
    y = torch.full((M, N), float("nan"), dtype=torch.float32, device="cuda")
    plan = hip.plan([w], [torch.from_numpy(x).cuda()], [y])
    assert plan.describe() == (H_.LAUNCH_TILES, 256, 256, 216)
    plan.run()
    torch.cuda.synchronize()
    _, q, s_, acc = O.ternary_linear(x, W, scale)
    assert np.array_equal(y.cpu().numpy(), (acc.astype(np.float32) * s_[:, None]) * np.float32(scale))


# Tile-GEMM plans (M > 64) and the tile shape each must take, checked bit-exact against the
# oracle problem by problem: name -> (M, [(N, K, input index)], (tile_m, tile_n, tiles)).
TILE_PLANS = {
    # the 512-token prefill's gate/up (two 6912-row problems sharing x): 256 x 128 tiles
    "gate_up_m512": (512, [(6912, 2560, 0), (6912, 2560, 0)], (256, 128, 216)),
    # one 13824-row problem at 384 < M <= 512: 256 x 128 as well
    "wide_m400": (400, [(13824, 2560, 0)], (256, 128, 216)),
    # the 512-token prefill's q/k/v and down: 64 x 128 tiles
    "qkv_m512": (512, [(2560, 2560, 0), (640, 2560, 0), (640, 2560, 0)], (64, 128, 240)),
    "down_m512": (512, [(2560, 6912, 0)], (64, 128, 160)),
    # cfg 3: 256 x 256 tiles (gate/up) and 128 x 160 regions (down)
    "cfg3_gate_up": (2048, [(6912, 2560, 0)], (256, 256, 216)),
    "cfg3_down": (2048, [(2560, 6912, 0)], (128, 160, 256)),
    # two long-K problems sharing one region launch (regions of problem 1 follow problem 0's)
    "regions_two": (1024, [(2560, 4096, 0), (2400, 4096, 1)], (128, 160, 248)),
    # ragged regions: rows past M, a last region of 100 columns, 33 chunks per K half
    "regions_ragged": (2000, [(2500, 4224, 0)], (128, 160, 256)),
    # a problem with an odd chunk count keeps the whole launch off the regions
    "regions_mixed_parity": (1024, [(2560, 4096, 0), (2400, 4160, 1)], (192, 128, 234)),
    # M = 100 (128-row activation padding): 128 x 128
    "m100": (100, [(2560, 2560, 0), (640, 2560, 1)], (128, 128, 25)),
}


@pytest.mark.parametrize("name", list(TILE_PLANS))
def test_tile_plan_shapes_vs_oracle(hip, name):
    import torch

    M, shapes, (tm, tn, tiles) = TILE_PLANS[name]
    rng = np.random.default_rng(sum(map(ord, name)))
    inputs = {}
    ws, xs, ys, Ws = [], [], [], []
    for N, K, xi in shapes:
        if xi not in inputs:
            inputs[xi] = rng.standard_normal((M, K), dtype=np.float32)
        W, scale = O.make_ternary(rng, N, K)
        Ws.append((W, scale))
        ws.append(hip.upload(O.pack_rotor(W), K, scale))
        xs.append(torch.from_numpy(inputs[xi]).cuda())
        ys.append(torch.full((M, N), float("nan"), dtype=torch.float32, device="cuda"))
    # problems sharing an input must share the tensor (one quantisation)
    by_idx = {}
    xs = [by_idx.setdefault(xi, x) for (_, _, xi), x in zip(shapes, xs)]
    plan = hip.plan(ws, xs, ys)
    from rotor import _hip as H_

    assert plan.describe() == (H_.LAUNCH_TILES, tm, tn, tiles)
    plan.run()
    torch.cuda.synchronize()
    for (W, scale), (_, _, xi), y in zip(Ws, shapes, ys):
        y_ref, q, s, acc = O.ternary_linear(inputs[xi], W, scale)
        y_exact = (acc.astype(np.float32) * s[:, None]) * np.float32(scale)
        assert np.array_equal(y.cpu().numpy(), y_exact)


# M = 1 plans whose one launch quantises in the GEMV prologue: (N, K) per problem.
# >= 1024 row blocks -> ROWS shape, each workgroup quantising its own problem's row with
# nw = 4 / 2 / 1 waves (the largest dividing every problem's row-block count); K = 6912
# exceeds one 16-group per thread (the multi-pass quantiser); few row blocks with one
# shared input -> KSPLIT prologue.
PROLOGUE_PLANS = {
    "rows_nw4": [(6912, 2560)] * 10,
    "rows_nw2_ragged": [(6912, 2500)] * 10 + [(100, 2500), (2560, 2500)],
    "rows_nw1_long_k": [(6912, 6912)] * 10 + [(50, 6912), (130, 6912)],
    "ksplit_shared": [(2560, 2560), (640, 2560), (640, 2560)],
}


@pytest.mark.parametrize("name", list(PROLOGUE_PLANS))
def test_plan_run_prologue_equals_two_launches(hip, name):
    import torch

    shapes = PROLOGUE_PLANS[name]
    rng = np.random.default_rng(len(name))
    shared = name.startswith("ksplit")
    x0 = torch.from_numpy(rng.standard_normal((1, shapes[0][1]), dtype=np.float32)).cuda()
    ws, xs, ys, Ws = [], [], [], []
    for N, K in shapes:
        W, scale = O.make_ternary(rng, N, K)
        Ws.append((W, scale))
        ws.append(hip.upload(O.pack_rotor(W), K, scale))
        xs.append(x0 if shared else torch.from_numpy(rng.standard_normal((1, K), dtype=np.float32)).cuda())
        ys.append(torch.full((1, N), float("nan"), dtype=torch.float32, device="cuda"))
    plan = hip.plan(ws, xs, ys)
    plan.run()
    torch.cuda.synchronize()
    fused = [y.clone() for y in ys]
    for y in ys:
        y.fill_(float("nan"))
    plan.quantize()
    plan.gemv()
    torch.cuda.synchronize()
    for a, b in zip(fused, ys):
        assert torch.equal(a, b)
    for g in (0, len(shapes) - 2, len(shapes) - 1):  # against the oracle
        W, scale = Ws[g]
        x = xs[g].cpu().numpy()
        y_ref, q, s, acc = O.ternary_linear(x, W, scale)
        assert np.array_equal(fused[g].cpu().numpy(), (acc.astype(np.float32) * s[:, None]) * np.float32(scale))


@pytest.mark.parametrize("N,K", [(65600, 300), (65664, 2560)])
def test_linear_f32_single_rows_prologue(hip, N, K):
    """One linear with >= 1024 row blocks at M = 1: the ROWS kernel quantises x itself
    (1025 row blocks -> one wave per workgroup, 1026 -> two)."""
    import torch

    x, W, scale = _case(N + K, 1, N, K)
    w = hip.upload(O.pack_rotor(W), K, scale)
    y = hip.linear_device(w, torch.from_numpy(x)).cpu().numpy()
    y_ref, q, s, acc = O.ternary_linear(x, W, scale)
    np.testing.assert_allclose(y, y_ref, atol=ATOL, rtol=RTOL)
    assert np.array_equal(y, (acc.astype(np.float32) * s[:, None]) * np.float32(scale))


def test_ternary_linear_layer_gpu(hip):
    from rotor import gpu_layers
    from rotor.transformer import TernaryLinear

    x, W, scale = _case(21, 6, 640, 2560)
    gpu_layers._gpu_instance = hip  # share the session backend
    try:
        layer = TernaryLinear(2560, 640, use_gpu=True)
        layer.load_from_bitnet(O.pack_rotor(W), scale)
        y = layer.forward(x.reshape(2, 3, 2560))
        assert isinstance(y, np.ndarray) and y.shape == (2, 3, 640)
        y_ref = O.ternary_linear(x, W, scale)[0]
        np.testing.assert_allclose(y.reshape(6, 640), y_ref, atol=ATOL, rtol=RTOL)
        assert np.abs(y.reshape(6, 640) - O.linear_ref_f32(x, W, scale)).max() < 0.05
    finally:
        gpu_layers._gpu_instance = None
