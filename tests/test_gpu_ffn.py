"""GPU parity of the fused activation producers and of the cfg-1 FFN block.

The device computes every intermediate exactly as oracle.ffn_block_w2a8 defines it
(RMSNorm mean of squares accumulated in f64, IEEE fp32 elementwise, absmax int8,
exact int32 accumulation), so intermediates and the block output are compared bit for
bit; the output is also checked against the reference-formula chain (fp32 RMSNorm,
np.dot on dequantised activations) within the quantisation error.
"""
import numpy as np
import pytest

from oracle import rotor_oracle as O

pytestmark = pytest.mark.gpu


def _np(t):
    return t.cpu().numpy()


@pytest.mark.parametrize("M,K", [(1, 2560), (7, 6912), (64, 2560), (3, 100), (2, 20000)])
def test_act_quantize_matches_quantize_rows(hip, M, K):
    import torch

    x = np.random.default_rng(K + M).standard_normal((M, K), dtype=np.float32) * 4
    act = hip.activations(M, K)
    hip.act_quantize(torch.from_numpy(x), act)
    q, s = act.export()
    qo, so = O.quant_rows(x)
    assert np.array_equal(_np(q), qo) and np.array_equal(_np(s), so)


@pytest.mark.parametrize("M,K", [(1, 2560), (5, 2560), (64, 2560), (2, 6912), (3, 17), (2, 20000)])
def test_act_rmsnorm_quantize_bit_exact(hip, M, K):
    import torch

    rng = np.random.default_rng(3 * K + M)
    x = rng.standard_normal((M, K), dtype=np.float32) * rng.uniform(0.1, 10, (M, 1)).astype(np.float32)
    w = rng.uniform(0.5, 1.5, K).astype(np.float32)
    act = hip.activations(M, K)
    h = torch.empty((M, K), dtype=torch.float32, device="cuda")
    hip.act_rmsnorm_quantize(torch.from_numpy(x), torch.from_numpy(w), act, 1e-6, h_out=h)
    ho = O.rms_norm_f64acc(x, w, 1e-6)
    assert np.array_equal(_np(h), ho)
    q, s = act.export()
    qo, so = O.quant_rows(ho)
    assert np.array_equal(_np(s), so) and np.array_equal(_np(q), qo)
    # the reference's fp32 RMSNorm is within a few ulp
    assert np.abs(_np(h) - O.rms_norm(x, w, 1e-6)).max() <= 4 * np.spacing(np.abs(ho).max())


@pytest.mark.parametrize("M,K", [(1, 2560), (9, 2560), (300, 6912), (2, 4160), (3, 8192), (2, 8256)])
def test_act_quantize_without_value_outputs(hip, M, K):
    """Without the fp32 value outputs the quantiser takes its vectorised row kernel (K % 64
    == 0, K <= 8192, 4 or 8 elements per thread); q and s stay bit-exact."""
    import torch

    rng = np.random.default_rng(11 * K + M)
    x = rng.standard_normal((M, K), dtype=np.float32) * rng.uniform(0.1, 10, (M, 1)).astype(np.float32)
    u = rng.standard_normal((M, K), dtype=np.float32)
    w = rng.uniform(0.5, 1.5, K).astype(np.float32)
    act = hip.activations(M, K)
    hip.act_rmsnorm_quantize(torch.from_numpy(x), torch.from_numpy(w), act, 1e-6)
    q, s = act.export()
    qo, so = O.quant_rows(O.rms_norm_f64acc(x, w, 1e-6))
    assert np.array_equal(_np(s), so) and np.array_equal(_np(q), qo)
    hip.act_relu2_mul_quantize(torch.from_numpy(x), torch.from_numpy(u), act)
    q, s = act.export()
    qo, so = O.quant_rows(O.relu2_gate(x, u))
    assert np.array_equal(_np(s), so) and np.array_equal(_np(q), qo)


@pytest.mark.parametrize("M,K", [(1, 6912), (4, 6912), (64, 6912), (2, 33)])
def test_act_relu2_mul_quantize_bit_exact(hip, M, K):
    import torch

    rng = np.random.default_rng(K * 7 + M)
    g = rng.standard_normal((M, K), dtype=np.float32) * 2
    u = rng.standard_normal((M, K), dtype=np.float32) * 2
    g[0, :5] = [0.0, -0.0, -1.0, 1.0, 3.0]
    act = hip.activations(M, K)
    a = torch.empty((M, K), dtype=torch.float32, device="cuda")
    hip.act_relu2_mul_quantize(torch.from_numpy(g), torch.from_numpy(u), act, a_out=a)
    ao = O.relu2_gate(g, u)
    assert np.array_equal(_np(a), ao)
    q, s = act.export()
    qo, so = O.quant_rows(ao)
    assert np.array_equal(_np(s), so) and np.array_equal(_np(q), qo)


@pytest.mark.parametrize("M", [1, 4, 64, 130])
def test_linear_act_equals_linear(hip, M):
    import torch

    x, W, scale = O.make_linear_case(M, M, 640, 2560)
    w = hip.upload(O.pack_rotor(W), 2560, scale)
    act = hip.activations(M, 2560)
    xt = torch.from_numpy(x).cuda()
    hip.act_quantize(xt, act)
    assert torch.equal(hip.linear_act(w, act), hip.linear_device(w, xt))


@pytest.mark.parametrize("M", [1, 3, 64])
def test_ffn_block_cfg1_bit_exact(hip, M):
    import torch

    from rotor import gpu_layers
    from rotor.ffn import TernaryFFNBlock

    D, F = 2560, 6912
    rng = np.random.default_rng(100 + M)
    Wg, sg = O.make_ternary(rng, F, D)
    Wu, su = O.make_ternary(rng, F, D)
    Wd, sd = O.make_ternary(rng, D, F)
    nw = rng.uniform(0.5, 1.5, D).astype(np.float32)
    x = rng.standard_normal((M, D), dtype=np.float32)
    gpu_layers._gpu_instance = hip
    try:
        blk = TernaryFFNBlock(D, F, use_gpu=True, max_tokens=64)
        blk.load(nw, (O.pack_rotor(Wg), sg), (O.pack_rotor(Wu), su), (O.pack_rotor(Wd), sd))
        y = blk.forward(x)
        y2 = blk.forward(x)  # buffers and plans are reused
        assert blk.launches(M) == (2 if M == 1 else 4)
        blk.pair_ok = False  # the four-launch form gives the same bits for one token too
        y4 = blk.forward(x)
    finally:
        gpu_layers._gpu_instance = None
    yo, it = O.ffn_block_w2a8(x, nw, Wg, sg, Wu, su, Wd, sd)
    assert np.array_equal(y, yo) and np.array_equal(y2, yo) and np.array_equal(y4, yo)
    y_ref, _ = O.ffn_block(x, nw, Wg, sg, Wu, su, Wd, sd)
    assert np.abs(y - y_ref).max() < 0.05 * max(1.0, np.abs(y_ref).max())


def test_ffn_block_graph_replay(hip):
    """A captured forward replays with the same result (no allocation in the path)."""
    import torch

    from rotor import gpu_layers
    from rotor.ffn import TernaryFFNBlock

    D, F = 256, 512
    rng = np.random.default_rng(7)
    Wg, sg = O.make_ternary(rng, F, D)
    Wu, su = O.make_ternary(rng, F, D)
    Wd, sd = O.make_ternary(rng, D, F)
    nw = np.ones(D, np.float32)
    gpu_layers._gpu_instance = hip
    try:
        blk = TernaryFFNBlock(D, F, use_gpu=True, max_tokens=4)
        blk.load(nw, (O.pack_rotor(Wg), sg), (O.pack_rotor(Wu), su), (O.pack_rotor(Wd), sd))
        x = torch.zeros((1, D), device="cuda")
        blk.forward_device(x)  # allocate buffers and plans outside the capture
        torch.cuda.synchronize()
        g = torch.cuda.CUDAGraph()
        with torch.cuda.graph(g):
            y = blk.forward_device(x)
        for i in range(3):
            xi = rng.standard_normal((1, D), dtype=np.float32)
            x.copy_(torch.from_numpy(xi))
            g.replay()
            torch.cuda.synchronize()
            yo, _ = O.ffn_block_w2a8(xi, nw, Wg, sg, Wu, su, Wd, sd)
            assert np.array_equal(_np(y), yo), f"replay {i}"
    finally:
        gpu_layers._gpu_instance = None


@pytest.mark.parametrize("mode,K,N", [(0, 2560, 640), (2, 2560, 2560), (3, 6912, 2560), (4, 6912, 2560), (2, 100, 77),
                                      (4, 20000, 128)])  # more groups than threads: general prologue path
def test_fused_plan_equals_act_path(hip, mode, K, N):
    """One-launch decode plans (input quantised in the GEMV prologue) give exactly the
    result of the separate quantiser + linear path, with and without the residual."""
    import torch

    from rotor import _hip

    rng = np.random.default_rng(mode * 1000 + K)
    d = lambda a: torch.from_numpy(np.ascontiguousarray(a, np.float32)).cuda()
    x = d(rng.standard_normal(K) * 2)
    aux = d(rng.uniform(0.5, 1.5, K) if mode == 2 else rng.standard_normal(K))
    aux2 = d(rng.uniform(0.5, 1.5, K))
    Ws = [O.make_ternary(rng, N, K) for _ in range(2)]
    ws = [hip.upload(O.pack_rotor(W), K, s) for W, s in Ws]
    res = d(rng.standard_normal(N))
    ys = [torch.empty(N, device="cuda"), torch.empty(N, device="cuda")]
    y_res = res.clone()
    plan = hip.plan_fused(ws, mode, x, aux if mode else None, aux2 if mode == 4 else None, 1e-6, ys=ys)
    plan2 = hip.plan_fused(ws[:1], mode, x, aux if mode else None, aux2 if mode == 4 else None, 1e-6, ys=[y_res],
                           residuals=[y_res])
    plan.run()
    plan2.run()
    act = hip.activations(1, K)
    xr = x[None]
    if mode == 0:
        hip.act_quantize(xr, act)
    elif mode == 2:
        hip.act_rmsnorm_quantize(xr, aux, act, 1e-6)
    elif mode == 3:
        hip.act_relu2_mul_quantize(xr, aux[None], act)
    else:
        hip.act_relu2_mul_norm_quantize(xr, aux[None], aux2, act, 1e-6)
    for w, y in zip(ws, ys):
        assert torch.equal(hip.linear_act(w, act)[0], y)
    assert torch.equal(hip.linear_act(ws[0], act, residual=res[None])[0], y_res)
    # and the int8 input equals the oracle's for that mode
    q, s = act.export()
    xn, an, a2n = x.cpu().numpy(), aux.cpu().numpy(), aux2.cpu().numpy()
    src = {0: xn, 2: O.rms_norm_f64acc(xn[None], an)[0], 3: O.relu2_gate(xn, an),
           4: O.rms_norm_f64acc(O.relu2_gate(xn, an)[None], a2n)[0]}[mode]
    qo, so = O.quant_rows(src[None])
    assert np.array_equal(q.cpu().numpy(), qo) and np.array_equal(s.cpu().numpy(), so)


@pytest.mark.parametrize("D,F", [(2560, 6912), (256, 320), (4096, 640), (128, 96)])
def test_gate_up_pair_plan(hip, D, F):
    """The gate/up pair plan (gate and up interleaved in 32-row groups) writes g and u
    exactly as the two-problem fused plan does, a = relu(g)^2 * u with the fp32 operations
    of oracle.relu2_gate, and per 32 outputs the f64 sum of a^2; a down-projection plan fed
    (a, ssq) through RMSNORM_SSQ gives exactly the RELU2MUL_NORM plan's output on (g, u)."""
    import torch

    from rotor import _hip

    rng = np.random.default_rng(D + F)
    d = lambda a: torch.from_numpy(np.ascontiguousarray(a, np.float32)).cuda()
    h, nw, nwf = d(rng.standard_normal(D) * 2), d(rng.uniform(0.5, 1.5, D)), d(rng.uniform(0.5, 1.5, F))
    (Wg, sg), (Wu, su), (Wd, sd) = O.make_ternary(rng, F, D), O.make_ternary(rng, F, D), O.make_ternary(rng, D, F)
    wg, wu, wd = hip.upload(O.pack_rotor(Wg), D, sg), hip.upload(O.pack_rotor(Wu), D, su), hip.upload(O.pack_rotor(Wd), F, sd)
    g, u = torch.empty(F, device="cuda"), torch.empty(F, device="cuda")
    hip.plan_fused([wg, wu], _hip.SRC_RMSNORM, h, nw, eps=1e-6, ys=[g, u]).run()
    w_gu, scales = hip.interleave_gate_up(wg, wu)
    a = torch.full((F,), float("nan"), device="cuda")
    ssq = torch.full((F // 32,), float("nan"), dtype=torch.float64, device="cuda")
    g2, u2 = torch.empty(F, device="cuda"), torch.empty(F, device="cuda")
    hip.plan_gate_up(w_gu, scales, _hip.SRC_RMSNORM, h, nw, eps=1e-6, a=a, ssq=ssq, g_out=g2, u_out=u2).run()
    gn, un, an = _np(g), _np(u), _np(a)
    assert np.array_equal(_np(g2), gn) and np.array_equal(_np(u2), un)
    assert np.array_equal(an, O.relu2_gate(gn, un))
    np.testing.assert_allclose(_np(ssq), (an.astype(np.float64).reshape(-1, 32) ** 2).sum(1), rtol=1e-12, atol=0)
    if F % 64 == 0 and F <= 8192:
        y1, y2 = torch.empty(D, device="cuda"), torch.empty(D, device="cuda")
        hip.plan_fused([wd], _hip.SRC_RELU2MUL_NORM, g, u, nwf, eps=1e-6, ys=[y1]).run()
        hip.plan_fused([wd], _hip.SRC_RMSNORM_SSQ, a, nwf, ssq, eps=1e-6, ys=[y2]).run()
        assert torch.equal(y1, y2)


def test_gate_up_pair_plan_rejects_shapes(hip):
    import torch

    from rotor import _hip

    rng = np.random.default_rng(5)
    d = lambda a: torch.from_numpy(np.ascontiguousarray(a, np.float32)).cuda()
    h, nw = d(rng.standard_normal(100)), d(np.ones(100))
    w1, w2 = (hip.upload(O.pack_rotor(O.make_ternary(rng, 64, 100)[0]), 100, 1.0) for _ in range(2))
    w_gu, scales = hip.interleave_gate_up(w1, w2)
    a, ssq = torch.empty(64, device="cuda"), torch.empty(2, dtype=torch.float64, device="cuda")
    with pytest.raises(RuntimeError, match="K % 64"):
        hip.plan_gate_up(w_gu, scales, _hip.SRC_RMSNORM, h, nw, a=a, ssq=ssq)


@pytest.mark.parametrize("D,N,F", [(2560, 2560, 6912), (640, 200, 256), (1024, 96, 512), (640, 224, 256)])
def test_output_ssq_feeds_rmsnorm_ssq(hip, D, N, F):
    """A one-problem fused decode plan with rt_plan_set_output_ssq writes, per 32 outputs
    (after the residual; a last partial group adds only its outputs), the f64 sum of their
    squares; a plan reading that row through RMSNORM_SSQ gives exactly what the same plan
    reducing the row itself (RMSNORM) gives, as a gate/up pair plan and as a q/k/v-style
    plan.  Detached, the plan writes no sums."""
    import torch

    from rotor import _hip

    rng = np.random.default_rng(D + N)
    d = lambda a: torch.from_numpy(np.ascontiguousarray(a, np.float32)).cuda()
    x, nw1, nw2 = d(rng.standard_normal(D) * 2), d(rng.uniform(0.5, 1.5, D)), d(rng.uniform(0.5, 1.5, N))
    (Wo, so), (Wq, sq) = O.make_ternary(rng, N, D), O.make_ternary(rng, 2 * 64, N)
    wo, wq = hip.upload(O.pack_rotor(Wo), D, so), hip.upload(O.pack_rotor(Wq), N, sq)
    h0 = d(rng.standard_normal(N))
    h = h0.clone()
    # one sentinel entry past the ceil(N / 32) sums: no group wholly past N is written
    ss_buf = torch.full(((N + 31) // 32 + 1,), float("nan"), dtype=torch.float64, device="cuda")
    ss = ss_buf[:-1]
    po = hip.plan_fused([wo], _hip.SRC_RMSNORM, x, nw1, eps=1e-6, ys=[h], residuals=[h])
    po.set_output_ssq(ss)
    po.run()
    torch.cuda.synchronize()
    hn = _np(h).astype(np.float64)
    hp = np.concatenate([hn, np.zeros(-N % 32)]).reshape(-1, 32)
    np.testing.assert_allclose(_np(ss), (hp ** 2).sum(1), rtol=1e-12, atol=0)
    assert np.isnan(_np(ss_buf)[-1])
    # consumers: RMSNORM_SSQ on (h, ss) == RMSNORM on h
    if N % 64 == 0:
        y1, y2 = torch.empty(2 * 64, device="cuda"), torch.empty(2 * 64, device="cuda")
        hip.plan_fused([wq], _hip.SRC_RMSNORM, h, nw2, eps=1e-6, ys=[y1]).run()
        hip.plan_fused([wq], _hip.SRC_RMSNORM_SSQ, h, nw2, ss, eps=1e-6, ys=[y2]).run()
        torch.cuda.synchronize()
        assert torch.equal(y1, y2)
        (Wg, sg), (Wu, su) = O.make_ternary(rng, F, N), O.make_ternary(rng, F, N)
        w_gu, scales = hip.interleave_gate_up(hip.upload(O.pack_rotor(Wg), N, sg), hip.upload(O.pack_rotor(Wu), N, su))
        outs = []
        for src in ((_hip.SRC_RMSNORM, h, nw2), (_hip.SRC_RMSNORM_SSQ, h, nw2, ss)):
            a = torch.empty(F, device="cuda")
            assq = torch.empty(F // 32, dtype=torch.float64, device="cuda")
            hip.plan_gate_up(w_gu, scales, *src, eps=1e-6, a=a, ssq=assq).run()
            outs.append((a, assq))
        torch.cuda.synchronize()
        assert torch.equal(outs[0][0], outs[1][0]) and torch.equal(outs[0][1], outs[1][1])
    # detached: the sums are left alone
    po.set_output_ssq(None)
    ss.fill_(-1.0)
    h.copy_(h0)
    po.run()
    torch.cuda.synchronize()
    assert (ss == -1.0).all()


def test_output_ssq_rejects_other_plans(hip):
    import torch

    from rotor import _hip

    rng = np.random.default_rng(9)
    d = lambda a: torch.from_numpy(np.ascontiguousarray(a, np.float32)).cuda()
    x, nw = d(rng.standard_normal(256)), d(np.ones(256))
    w1, w2 = (hip.upload(O.pack_rotor(O.make_ternary(rng, 64, 256)[0]), 256, 1.0) for _ in range(2))
    ss = torch.empty(4, dtype=torch.float64, device="cuda")
    two = hip.plan_fused([w1, w2], _hip.SRC_RMSNORM, x, nw, eps=1e-6, ys=[torch.empty(64, device="cuda")] * 2)
    with pytest.raises(RuntimeError, match="rt_plan_set_output_ssq"):
        two.set_output_ssq(ss)
    w_gu, scales = hip.interleave_gate_up(w1, w2)
    pair = hip.plan_gate_up(w_gu, scales, _hip.SRC_RMSNORM, x, nw, a=torch.empty(64, device="cuda"),
                            ssq=torch.empty(2, dtype=torch.float64, device="cuda"))
    with pytest.raises(RuntimeError, match="rt_plan_set_output_ssq"):
        pair.set_output_ssq(ss)
    with pytest.raises(ValueError):
        hip.plan_fused([w1], _hip.SRC_RMSNORM, x, nw, eps=1e-6, ys=[torch.empty(64, device="cuda")]).set_output_ssq(
            torch.empty(4, device="cuda"))


# (M, F, K): the tile the pair epilogue runs on -- 128 x 128 (M <= 128), 64 x 128 promoted to
# 128 x 128 (few tiles), 192 x 128, 256 x 128 (the 512-token prefill), and 256 x 256 taken as
# 256 x 128 (M = 2048)
@pytest.mark.parametrize("M,F,K", [(70, 256, 128), (200, 512, 256), (300, 1024, 640), (512, 6912, 2560),
                                   (2048, 6912, 2560)])
def test_act_gate_up_pair_equals_separate(hip, M, F, K):
    """rt_plan_create_act_gate_up: one GEMM over the interleaved gate/up matrix writes
    a = relu(g)^2 * u, bit for bit the product of the g and u an rt_plan_create_act plan over
    the two matrices writes (each rounded as the fp32 epilogue rounds y, the product in the
    order of the quantiser's relu^2 * up: (g g) u).  Rows past M are not written."""
    import torch

    rng = np.random.default_rng(M + F + K)
    (Wg, sg), (Wu, su) = O.make_ternary(rng, F, K), O.make_ternary(rng, F, K)
    wg, wu = hip.upload(O.pack_rotor(Wg), K, sg), hip.upload(O.pack_rotor(Wu), K, su)
    w_gu, scales = hip.interleave_gate_up(wg, wu)
    x = torch.from_numpy(rng.standard_normal((M, K)).astype(np.float32)).cuda()
    act = hip.activations(M, K)
    hip.act_quantize(x, act)
    g, u = torch.empty(M, F, device="cuda"), torch.empty(M, F, device="cuda")
    hip.plan_act([wg, wu], [act, act], M, [g, u]).gemv()
    a_buf = torch.full((M + 1, F), float("nan"), device="cuda")
    a = a_buf[:M]
    hip.plan_act_gate_up(w_gu, scales, act, M, a).gemv()
    torch.cuda.synchronize()
    ref = torch.where(g > 0, (g * g) * u, torch.zeros_like(g))
    assert torch.equal(a, ref)
    assert torch.isnan(a_buf[M]).all()
    with pytest.raises(RuntimeError, match="rt_plan_create_act_gate_up"):
        hip.plan_act_gate_up(w_gu, scales, hip.activations(64, K), 64, torch.empty(64, F, device="cuda"))
