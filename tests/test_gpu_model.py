"""GPU tests of the cfg-4 model path: the kernels around the linears (embedding,
RoPE + KV append, causal GQA attention, fused final-norm LM head + argmax) against the
NumPy restatement, and the whole model loaded through load_bitnet_model from a
synthetic safetensors checkpoint with the reference's tensor names.

Bars: embedding and RoPE/KV append bit-exact (same fp32 operations); attention and
logits within fp32 accumulation-order tolerance; greedy tokens equal wherever the
oracle's top-2 logit gap exceeds that tolerance.
"""
import ctypes
import json

import numpy as np
import pytest

from oracle import rotor_oracle as O

pytestmark = pytest.mark.gpu

SMALL = dict(vocab_size=1000, d_model=512, n_layers=2, n_heads=8, n_kv_heads=2, d_ff=1024, rope_theta=500000.0)


def _lib():
    from rotor import _hip

    return _hip.load(), _hip.check


# fp32 logits against the f64 head: the tolerance of BASELINE.json's north star
LOGIT_ATOL, LOGIT_RTOL = 3e-4, 1e-5


def lm_head_device_order(E32, hn):
    """The fused LM head's fp32 arithmetic in the kernel's order (rt_model.hip,
    lm_head_kernel): lane l of a wave sums, for slice s = 0 .. D/512 - 1 and j = 0 .. 7, the
    products E[v, 512 s + 8 l + j] * hn[512 s + 8 l + j], each rounded to fp32 and then added
    (contraction off); the 64 lane sums are reduced as wave_reduce63 does: rows of 16 lanes
    by row_shr 1, 2, 4, 8 (lanes whose source lies outside the row add 0), then lane 15 of
    rows 0 and 2 into rows 1 and 3 (row_bcast 15), then lane 31 into rows 2 and 3 (row_bcast
    31); lane 63 holds the logit.  E32: the bf16 embedding as fp32 [V, D]."""
    V, D = E32.shape
    S = D // 512
    E = E32.reshape(V, S, 64, 8)
    x = np.asarray(hn, np.float32).reshape(S, 64, 8)
    acc = np.zeros((V, 64), np.float32)
    for sl in range(S):
        for j in range(8):
            acc = acc + E[:, sl, :, j] * x[sl, :, j]
    lane = np.arange(64)
    for sh in (1, 2, 4, 8):
        src = np.zeros_like(acc)
        ok = lane % 16 >= sh
        src[:, ok] = acc[:, lane[ok] - sh]
        acc = acc + src
    src = np.zeros_like(acc)
    src[:, 16:32] = acc[:, 15:16]
    src[:, 48:64] = acc[:, 47:48]
    acc = acc + src
    src = np.zeros_like(acc)
    src[:, 32:64] = acc[:, 31:32]
    acc = acc + src
    return acc[:, 63]


def check_logits(lg, ref64, E32, hn, what):
    """Device LM-head logits: within LOGIT_ATOL + LOGIT_RTOL |ref| of the f64 head, and bit
    for bit the kernel's fp32 order on the same normalised hidden state."""
    np.testing.assert_allclose(lg, ref64, atol=LOGIT_ATOL, rtol=LOGIT_RTOL, err_msg=f"logits vs f64 head ({what})")
    emu = lm_head_device_order(E32, hn)
    assert np.array_equal(lg, emu), f"logits vs the kernel's fp32 order ({what}): max |diff| {np.abs(lg - emu).max()}"


def test_embed_exact(hip):
    import torch

    lib, chk = _lib()
    rng = np.random.default_rng(0)
    E = O.f32_to_bf16(rng.standard_normal((300, 512), dtype=np.float32))
    ids = np.array([0, 299, 5, 5, 123], np.int32)
    Ed = torch.from_numpy(E.view(np.int16)).cuda()
    idd = torch.from_numpy(ids).cuda()
    h = torch.empty((5, 512), device="cuda")
    hip._bind_stream()
    chk(lib.rt_embed(hip.ctx, Ed.data_ptr(), 300, 512, idd.data_ptr(), 5, h.data_ptr()))
    assert np.array_equal(h.cpu().numpy(), O.bf16_to_f32(E)[ids])


# (M, pos0, H, Hkv, hd, Lmax): hd = 128 runs the matrix-core kernel (32 (query, head) rows
# per workgroup, 32-key blocks over 4 waves: several query and key blocks, ragged last
# blocks, G = H / Hkv of 1, 4, 8, Lmax not a multiple of 32); the rest the general kernel
ATTN_CASES = [(1, 0, 20, 5, 128, 64), (1, 37, 20, 5, 128, 64), (7, 3, 8, 2, 64, 64), (16, 0, 4, 4, 64, 64),
              (100, 50, 20, 5, 128, 256), (70, 0, 8, 4, 64, 128), (130, 5, 4, 4, 64, 192), (33, 20, 6, 2, 64, 64),
              (40, 10, 8, 8, 128, 128), (50, 0, 16, 2, 128, 68), (200, 300, 20, 5, 128, 520),
              (130, 0, 4, 2, 128, 192), (20, 0, 4, 2, 128, 192), (130, 0, 8, 2, 64, 192), (512, 0, 20, 5, 128, 640)]


@pytest.mark.parametrize("M,pos0,H,Hkv,hd,Lmax", ATTN_CASES)
def test_rope_append_and_attention(hip, M, pos0, H, Hkv, hd, Lmax):
    import torch

    lib, chk = _lib()
    rng = np.random.default_rng(M * 100 + pos0)
    table = O.rope_table(Lmax, hd, 500000.0)
    # cache already holding pos0 tokens
    Kprev = rng.standard_normal((Hkv, pos0, hd)).astype(np.float32)
    Vprev = rng.standard_normal((Hkv, pos0, hd)).astype(np.float32)
    q = rng.standard_normal((M, H * hd)).astype(np.float32)
    k = rng.standard_normal((M, Hkv * hd)).astype(np.float32)
    v = rng.standard_normal((M, Hkv * hd)).astype(np.float32)
    kc = np.zeros((Hkv, hd, Lmax), np.float32)
    vc = np.zeros((Hkv, Lmax, hd), np.float32)
    kc[:, :, :pos0] = Kprev.transpose(0, 2, 1)
    vc[:, :pos0] = Vprev
    d = lambda a: torch.from_numpy(np.ascontiguousarray(a)).cuda()
    qd, kd, vd, kcd, vcd, td = d(q), d(k), d(v), d(kc), d(vc), d(table)
    pos = torch.tensor([pos0], dtype=torch.int32, device="cuda")
    out = torch.empty((M, H * hd), device="cuda")
    hip._bind_stream()
    chk(lib.rt_rope_kv_append(hip.ctx, qd.data_ptr(), kd.data_ptr(), vd.data_ptr(), kcd.data_ptr(), vcd.data_ptr(),
                              td.data_ptr(), M, H, Hkv, hd, Lmax, pos.data_ptr()))
    chk(lib.rt_attention(hip.ctx, qd.data_ptr(), kcd.data_ptr(), vcd.data_ptr(), out.data_ptr(), M, H, Hkv, hd, Lmax,
                         pos.data_ptr()))
    qr = O.apply_rope(q.reshape(M, H, hd), table, pos0)
    kr = O.apply_rope(k.reshape(M, Hkv, hd), table, pos0)
    assert np.array_equal(qd.cpu().numpy().reshape(M, H, hd), qr)
    K = np.concatenate([Kprev, kr.transpose(1, 0, 2)], axis=1)
    V = np.concatenate([Vprev, v.reshape(M, Hkv, hd).transpose(1, 0, 2)], axis=1)
    assert np.array_equal(kcd.cpu().numpy()[:, :, :pos0 + M], K.transpose(0, 2, 1))
    assert np.array_equal(vcd.cpu().numpy()[:, :pos0 + M], V)
    ref = O.causal_gqa_attention(qr, K, V, pos0).reshape(M, H * hd)
    np.testing.assert_allclose(out.cpu().numpy(), ref, atol=2e-5, rtol=1e-4)
    # again on the same context: the same output, bit for bit
    out2 = torch.full((M, H * hd), float("nan"), device="cuda")
    chk(lib.rt_attention(hip.ctx, qd.data_ptr(), kcd.data_ptr(), vcd.data_ptr(), out2.data_ptr(), M, H, Hkv, hd, Lmax,
                         pos.data_ptr()))
    assert torch.equal(out, out2)


# The last block's key count nk = pos0 % 64 + 1 walks the value sums' runs of 8 key pairs:
# hd 128 (2 key groups): runs of 16 keys, so nk 16 ends a run, 17 opens one, 25 and 31 end
# inside one; hd 64 (4 groups): runs of 32 keys.
@pytest.mark.parametrize("pos0,H,Hkv,hd,Lmax", [(0, 20, 5, 128, 640), (63, 20, 5, 128, 640), (64, 8, 2, 64, 200),
                                                (511, 20, 5, 128, 640), (639, 20, 5, 128, 640), (100, 4, 4, 64, 130),
                                                (527, 20, 5, 128, 640), (528, 20, 5, 128, 640), (600, 20, 5, 128, 640),
                                                (606, 20, 5, 128, 640), (95, 8, 2, 64, 200),
                                                (700, 8, 2, 64, 1000)])  # 16 blocks: general prologue path
def test_attention_decode_split(hip, pos0, H, Hkv, hd, Lmax):
    """Flash-decoding form equals the single-workgroup form; the workspace is reusable."""
    import torch

    lib, chk = _lib()
    rng = np.random.default_rng(pos0 + H + Lmax)
    kc = torch.from_numpy(rng.standard_normal((Hkv, hd, Lmax)).astype(np.float32)).cuda()
    vc = torch.from_numpy(rng.standard_normal((Hkv, Lmax, hd)).astype(np.float32)).cuda()
    q = torch.from_numpy(rng.standard_normal((1, H * hd)).astype(np.float32) * 2).cuda()
    pos = torch.tensor([pos0], dtype=torch.int32, device="cuda")
    ref = torch.empty((1, H * hd), device="cuda")
    out = torch.empty((1, H * hd), device="cuda")
    nbytes = lib.rt_attention_decode_workspace(H, hd, Lmax)
    ws = torch.zeros(nbytes, dtype=torch.uint8, device="cuda")
    hip._bind_stream()
    chk(lib.rt_attention(hip.ctx, q.data_ptr(), kc.data_ptr(), vc.data_ptr(), ref.data_ptr(), 1, H, Hkv, hd, Lmax,
                         pos.data_ptr()))
    for _ in range(3):
        out.zero_()
        chk(lib.rt_attention_decode(hip.ctx, q.data_ptr(), kc.data_ptr(), vc.data_ptr(), out.data_ptr(), H, Hkv, hd,
                                    Lmax, pos.data_ptr(), ws.data_ptr(), nbytes))
        np.testing.assert_allclose(out.cpu().numpy(), ref.cpu().numpy(), atol=2e-6, rtol=2e-5)
    K = kc.cpu().numpy().transpose(0, 2, 1)[:, :pos0 + 1]
    V = vc.cpu().numpy()[:, :pos0 + 1]
    o = O.causal_gqa_attention(q.cpu().numpy().reshape(1, H, hd), K, V, pos0).reshape(1, H * hd)
    np.testing.assert_allclose(out.cpu().numpy(), o, atol=2e-5, rtol=1e-4)
    # an o_proj plan that combines the partials in its prologue equals combine + norm + linear
    from rotor import _hip as H_

    W, sw = O.make_ternary(rng, 96, H * hd)
    w = hip.upload(O.pack_rotor(W), H * hd, sw)
    nw = torch.from_numpy(rng.uniform(0.5, 1.5, H * hd).astype(np.float32)).cuda()
    res = torch.from_numpy(rng.standard_normal(96).astype(np.float32)).cuda()
    y = res.clone()
    plan = hip.plan_fused([w], H_.SRC_ATTN_NORM, ws, nw, eps=1e-6, ys=[y], residuals=[y], attn_head_dim=hd,
                          attn_max_len=Lmax)
    chk(lib.rt_attention_decode_partials(hip.ctx, q.data_ptr(), kc.data_ptr(), vc.data_ptr(), H, Hkv, hd, Lmax,
                                         pos.data_ptr(), ws.data_ptr(), nbytes))
    plan.run()
    act = hip.activations(1, H * hd)
    hip.act_rmsnorm_quantize(out, nw, act, 1e-6)
    assert torch.equal(y, hip.linear_act(w, act, residual=res[None])[0])


@pytest.mark.parametrize("hd", [64, 128])
def test_attention_score_scale_two_keys(hip, hd):
    """The score scale 1/sqrt(head_dim) (src/rotor/transformer.py:266-267) on the device:
    q = a e_0 against keys [e_0, 0] and values [v0, v1] gives sig(a/sqrt(hd)) v0 +
    (1 - sig) v1, through the prefill kernel (rt_attention; hd 128: the matrix-core kernel)
    and the split decode path (rt_attention_decode); a scale of 1/hd or none would miss by
    more than 1e-2 (tests/test_oracle.py::test_attention_score_scale_kat)."""
    import torch

    from tests.test_oracle import _two_key_case, two_key_expected

    lib, chk = _lib()
    a, Lmax = 8.0, 64
    q1, K, V = _two_key_case(hd, a, hd)
    want = two_key_expected(V, a, 1.0 / np.sqrt(hd))
    kc = np.zeros((1, hd, Lmax), np.float32)
    vc = np.zeros((1, Lmax, hd), np.float32)
    kc[0, :, :2] = K[0].T
    vc[0, :2] = V[0]
    d = lambda x: torch.from_numpy(np.ascontiguousarray(x)).cuda()
    kcd, vcd = d(kc), d(vc)
    hip._bind_stream()
    # prefill: queries at positions 0 and 1, the second is the case
    q = np.zeros((2, hd), np.float32)
    q[1] = q1[0, 0]
    out = torch.empty((2, hd), device="cuda")
    pos = torch.tensor([0], dtype=torch.int32, device="cuda")
    chk(lib.rt_attention(hip.ctx, d(q).data_ptr(), kcd.data_ptr(), vcd.data_ptr(), out.data_ptr(), 2, 1, 1, hd, Lmax,
                         pos.data_ptr()))
    np.testing.assert_allclose(out.cpu().numpy()[1], want, rtol=0, atol=2e-5)
    # decode: one query at position 1
    pos1 = torch.tensor([1], dtype=torch.int32, device="cuda")
    nbytes = lib.rt_attention_decode_workspace(1, hd, Lmax)
    ws = torch.zeros(nbytes, dtype=torch.uint8, device="cuda")
    o1 = torch.empty((1, hd), device="cuda")
    chk(lib.rt_attention_decode(hip.ctx, d(q[1:]).data_ptr(), kcd.data_ptr(), vcd.data_ptr(), o1.data_ptr(), 1, 1, hd,
                                Lmax, pos1.data_ptr(), ws.data_ptr(), nbytes))
    np.testing.assert_allclose(o1.cpu().numpy()[0], want, rtol=0, atol=2e-5)


@pytest.mark.parametrize("pos0,H,Hkv,hd,Lmax", [(0, 20, 5, 128, 640), (63, 20, 5, 128, 640), (64, 8, 2, 64, 200),
                                                (639, 20, 5, 128, 640), (130, 4, 4, 64, 131), (527, 20, 5, 128, 640),
                                                (600, 20, 5, 128, 640)])
def test_rope_attention_decode_equals_separate_launches(hip, pos0, H, Hkv, hd, Lmax):
    """One launch of RoPE + KV append + split attention gives the partials, the combined
    output and the caches of rt_rope_kv_append followed by rt_attention_decode, bit for
    bit, and leaves the projection outputs untouched."""
    import torch

    from oracle.rotor_oracle import rope_table

    lib, chk = _lib()
    rng = np.random.default_rng(7 * pos0 + H + Lmax)
    f = lambda *shape: torch.from_numpy(rng.standard_normal(shape).astype(np.float32)).cuda()
    kc0, vc0 = f(Hkv, hd, Lmax), f(Hkv, Lmax, hd)
    q0, k0, v0 = f(1, H * hd) * 2, f(1, Hkv * hd), f(1, Hkv * hd)
    rope = torch.from_numpy(np.ascontiguousarray(rope_table(Lmax, hd, 500000.0), np.float32)).cuda()
    pos = torch.tensor([pos0], dtype=torch.int32, device="cuda")
    nbytes = lib.rt_attention_decode_workspace(H, hd, Lmax)
    hip._bind_stream()
    # separate launches (q and k are rotated in place there)
    q, k, kc, vc = q0.clone(), k0.clone(), kc0.clone(), vc0.clone()
    ws_ref = torch.zeros(nbytes, dtype=torch.uint8, device="cuda")
    out_ref = torch.empty((1, H * hd), device="cuda")
    chk(lib.rt_rope_kv_append(hip.ctx, q.data_ptr(), k.data_ptr(), v0.data_ptr(), kc.data_ptr(), vc.data_ptr(),
                              rope.data_ptr(), 1, H, Hkv, hd, Lmax, pos.data_ptr()))
    chk(lib.rt_attention_decode(hip.ctx, q.data_ptr(), kc.data_ptr(), vc.data_ptr(), out_ref.data_ptr(), H, Hkv, hd,
                                Lmax, pos.data_ptr(), ws_ref.data_ptr(), nbytes))
    # fused, twice (the second call sees the key already in the cache: same result)
    qf, kf, vf, kcf, vcf = q0.clone(), k0.clone(), v0.clone(), kc0.clone(), vc0.clone()
    for rep in range(2):
        ws = torch.zeros(nbytes, dtype=torch.uint8, device="cuda")
        out = torch.empty((1, H * hd), device="cuda")
        chk(lib.rt_rope_attention_decode(hip.ctx, qf.data_ptr(), kf.data_ptr(), vf.data_ptr(), kcf.data_ptr(),
                                         vcf.data_ptr(), rope.data_ptr(), H, Hkv, hd, Lmax, pos.data_ptr(),
                                         ws.data_ptr(), nbytes, out.data_ptr()))
        assert torch.equal(ws, ws_ref), f"partials differ (call {rep})"
        assert torch.equal(out, out_ref), f"output differs (call {rep})"
        assert torch.equal(kcf, kc) and torch.equal(vcf, vc), f"caches differ (call {rep})"
    assert torch.equal(qf, q0) and torch.equal(kf, k0) and torch.equal(vf, v0)
    # partials only (out = NULL) leave the same workspace
    ws = torch.zeros(nbytes, dtype=torch.uint8, device="cuda")
    chk(lib.rt_rope_attention_decode(hip.ctx, qf.data_ptr(), kf.data_ptr(), vf.data_ptr(), kcf.data_ptr(),
                                     vcf.data_ptr(), rope.data_ptr(), H, Hkv, hd, Lmax, pos.data_ptr(), ws.data_ptr(),
                                     nbytes, None))
    assert torch.equal(ws, ws_ref)


# H / Hkv = 20 / 5 (two query heads per attention workgroup, 20 workgroups per KV group at
# Lmax 640): Lmax 640: 10 key blocks, each workgroup combines at most one of a KV group's 16
# chunks of 32 outputs; 256 / 192 / 64: 4 / 3 / 1 blocks, 2 / 3 (the last one past the
# group) / 8 chunks per workgroup; 2048: no combine in the launch.  64 / 32 and 54 / 18
# (H / Hkv = 2 and 3: one workgroup per KV group and key block, 8- and 12-wave
# workgroups, K = 8192 and 6912) at Lmax <= 256, where the whole grid is resident.
@pytest.mark.parametrize("H,Hkv,pos0,Lmax", [(20, 5, 0, 640), (20, 5, 63, 640), (20, 5, 64, 640), (20, 5, 639, 640),
                                             (20, 5, 1000, 2048), (20, 5, 10, 256), (20, 5, 100, 192), (20, 5, 0, 64),
                                             (20, 5, 63, 64), (64, 32, 100, 256), (64, 32, 255, 256),
                                             (54, 18, 0, 192), (54, 18, 200, 256)])
def test_qkv_plan_with_attention_equals_separate_launches(hip, H, Hkv, pos0, Lmax):
    """The q/k/v decode plan with the attention attached (RoPE + KV append + split-L partials
    in the GEMV's launch) gives the q, k, v outputs, the partials and the caches of the plan
    followed by rt_rope_attention_decode, bit for bit.  The hand-off: the GEMV also stores
    every q/k/v output as a 64-bit word (epoch << 32 | value bits), the attention workgroups
    poll those words until they carry the launch's epoch, and the epoch follows from a count
    of finished attention workgroups, so it advances with every launch.  Checked on two runs
    in a row and on every replay of a captured graph, each with a new input row: a launch
    whose epoch did not advance would let the attention start on the previous launch's
    q/k/v and its partials would differ.  No wait gives up.  Where Lmax <= 640 the launch
    also combines the partials (rt_plan_attention_combine: the workgroups of a KV group
    share it, reading each other's partials as tagged words): its output equals
    rt_attention_decode_combine's on the reference partials bit for bit, and its per-32 sums
    of squares the f64 sums."""
    import torch

    from oracle.rotor_oracle import rope_table
    from rotor import _hip as H_

    lib, chk = _lib()
    hd = 128
    D = H * hd
    rng = np.random.default_rng(pos0 + Lmax + H)
    f = lambda *shape: torch.from_numpy(rng.standard_normal(shape).astype(np.float32)).cuda()
    ws_ = [hip.upload(O.pack_rotor(W), D, s) for W, s in (O.make_ternary(rng, n, D) for n in (D, Hkv * hd, Hkv * hd))]
    x = f(D)
    nw = torch.from_numpy(rng.uniform(0.5, 1.5, D).astype(np.float32)).cuda()
    kc0, vc0 = f(Hkv, hd, Lmax), f(Hkv, Lmax, hd)
    rope = torch.from_numpy(np.ascontiguousarray(rope_table(Lmax, hd, 500000.0), np.float32)).cuda()
    pos = torch.tensor([pos0], dtype=torch.int32, device="cuda")
    nbytes = lib.rt_attention_decode_workspace(H, hd, Lmax)
    outs = lambda: [torch.empty(D, device="cuda"), torch.empty(Hkv * hd, device="cuda"),
                    torch.empty(Hkv * hd, device="cuda")]
    hip._bind_stream()
    # the reference: the plan, then the attention launch, on the current x
    qr, kr, vr = outs()
    kc, vc = kc0.clone(), vc0.clone()
    ws_ref = torch.zeros(nbytes, dtype=torch.uint8, device="cuda")
    plan_ref = hip.plan_fused(ws_, H_.SRC_RMSNORM, x, nw, eps=1e-6, ys=[qr, kr, vr])

    def reference():
        kc.copy_(kc0)
        vc.copy_(vc0)
        ws_ref.zero_()
        plan_ref.run()
        chk(lib.rt_rope_attention_decode(hip.ctx, qr.data_ptr(), kr.data_ptr(), vr.data_ptr(), kc.data_ptr(),
                                         vc.data_ptr(), rope.data_ptr(), H, Hkv, hd, Lmax, pos.data_ptr(),
                                         ws_ref.data_ptr(), nbytes, None))
        torch.cuda.synchronize()

    # one launch
    q, k, v = outs()
    kcf, vcf = kc0.clone(), vc0.clone()
    ws = torch.zeros(nbytes, dtype=torch.uint8, device="cuda")
    plan = hip.plan_fused(ws_, H_.SRC_RMSNORM, x, nw, eps=1e-6, ys=[q, k, v])
    plan.attach_attention(kcf, vcf, rope, H, Hkv, hd, Lmax, pos, ws)
    combine = Lmax <= 640
    o_out = torch.empty(D, device="cuda")
    o_ssq = torch.empty(D // 32, dtype=torch.float64, device="cuda")
    o_ref = torch.empty(D, device="cuda")
    if combine:
        plan.attention_combine(o_out, o_ssq)

    def check(what):
        torch.cuda.synchronize()
        assert torch.equal(q, qr) and torch.equal(k, kr) and torch.equal(v, vr), f"q/k/v differ ({what})"
        assert torch.equal(ws, ws_ref), f"partials differ ({what})"
        assert torch.equal(kcf, kc) and torch.equal(vcf, vc), f"caches differ ({what})"
        if combine:
            chk(lib.rt_attention_decode_combine(hip.ctx, ws_ref.data_ptr(), nbytes, H, hd, Lmax, o_ref.data_ptr()))
            torch.cuda.synchronize()
            assert torch.equal(o_out, o_ref), f"combined output differs ({what})"
            o64 = o_ref.cpu().numpy().astype(np.float64).reshape(-1, 32)
            np.testing.assert_allclose(o_ssq.cpu().numpy(), (o64 ** 2).sum(1), rtol=1e-12, atol=0)

    def reset():
        # a new input row (so stale q/k/v words of an earlier launch would be wrong ones)
        x.copy_(f(D))
        reference()
        for t in (q, k, v, o_out, o_ssq):
            t.fill_(float("nan"))
        ws.zero_()
        kcf.copy_(kc0)
        vcf.copy_(vc0)
        torch.cuda.synchronize()

    for rep in range(2):
        reset()
        plan.run()
        check(f"run {rep}")
    assert plan.attention_timeouts() == 0
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        plan.run()
    for rep in range(3):
        reset()
        g.replay()
        check(f"replay {rep}")
    assert plan.attention_timeouts() == 0
    if not combine:  # too many key blocks for the combine in the launch
        with pytest.raises(RuntimeError, match="key blocks"):
            plan.attention_combine(o_out, o_ssq)
    # detached, the plan runs the GEMV only
    plan.attention_combine(None, None)
    plan.attach_attention(None, None, None, 0, 0, 0, 0, None, None)
    reset()
    plan.run()
    torch.cuda.synchronize()
    assert torch.equal(q, qr) and torch.equal(kcf, kc0) and not ws.any()


def test_attach_attention_rejects_other_plans(hip):
    """Plans the attention cannot join (one problem; 2 query heads per KV head) are refused
    with the library's message, and stay usable."""
    import torch

    from rotor import _hip as H_

    rng = np.random.default_rng(5)
    D, hd, Lmax = 2560, 128, 128
    w = [hip.upload(O.pack_rotor(W), D, s) for W, s in (O.make_ternary(rng, n, D) for n in (D, 640, 640))]
    x = torch.from_numpy(rng.standard_normal(D).astype(np.float32)).cuda()
    nw = torch.ones(D, device="cuda")
    kc, vc = torch.zeros(5, hd, Lmax, device="cuda"), torch.zeros(5, Lmax, hd, device="cuda")
    rope, pos = torch.zeros(Lmax, hd // 2, 2, device="cuda"), torch.zeros(1, dtype=torch.int32, device="cuda")
    ws = torch.zeros(_lib()[0].rt_attention_decode_workspace(20, hd, Lmax), dtype=torch.uint8, device="cuda")
    ys = [torch.empty(D, device="cuda"), torch.empty(640, device="cuda"), torch.empty(640, device="cuda")]
    one = hip.plan_fused(w[:1], H_.SRC_RMSNORM, x, nw, eps=1e-6, ys=ys[:1])
    with pytest.raises(RuntimeError, match="rt_plan_attach_attention"):
        one.attach_attention(kc, vc, rope, 20, 5, hd, Lmax, pos, ws)
    three = hip.plan_fused(w, H_.SRC_RMSNORM, x, nw, eps=1e-6, ys=ys)
    with pytest.raises(RuntimeError, match="rt_plan_attach_attention"):  # q must be H * hd = 10 * 128
        three.attach_attention(kc, vc, rope, 10, 5, hd, Lmax, pos, ws)
    with pytest.raises(RuntimeError, match="rt_plan_attach_attention"):  # workspace too small
        three.attach_attention(kc, vc, rope, 20, 5, hd, Lmax, pos, ws[:16])
    o, ssq = torch.empty(D, device="cuda"), torch.empty(D // 32, dtype=torch.float64, device="cuda")
    with pytest.raises(RuntimeError, match="attach the attention first"):  # no attention attached
        three.attention_combine(o, ssq)
    three.run()
    one.run()
    torch.cuda.synchronize()


@pytest.mark.parametrize("V,D", [(1000, 512), (5000, 2560), (777, 1024), (128256, 2560)])
def test_lm_head_argmax(hip, V, D):
    """Fused final norm + bf16 LM head + argmax at the cfg-4 vocabulary and others: logits
    within 3e-4 + 1e-5 |ref| of the f64 head and equal to the kernel's fp32 order; the token
    is the first index of the maximum; `best` is left zero; next_h receives the token's
    embedding row."""
    import torch

    lib, chk = _lib()
    rng = np.random.default_rng(V + D)
    E = O.f32_to_bf16(rng.standard_normal((V, D), dtype=np.float32))
    x = rng.standard_normal(D).astype(np.float32) * 3
    w = rng.uniform(0.5, 1.5, D).astype(np.float32)
    Ed = torch.from_numpy(E.view(np.int16)).cuda()
    xd, wd = torch.from_numpy(x).cuda(), torch.from_numpy(w).cuda()
    logits = torch.empty(V, device="cuda")
    best = torch.zeros(1, dtype=torch.int64, device="cuda")
    tok = torch.zeros(1, dtype=torch.int32, device="cuda")
    next_h = torch.full((D,), float("nan"), device="cuda")
    hip._bind_stream()
    for rep in range(2):  # `best` is left zero for the next call; the second writes next_h
        chk(lib.rt_lm_head_argmax(hip.ctx, Ed.data_ptr(), xd.data_ptr(), wd.data_ptr(), 1e-6, V, D, logits.data_ptr(),
                                  best.data_ptr(), tok.data_ptr(), None, 0, None, None, 0, 0,
                                  next_h.data_ptr() if rep else None))
        lg = logits.cpu().numpy()
        assert int(tok.cpu()[0]) == int(np.argmax(lg))
        assert int(best.cpu()[0]) == 0
    # the chosen token's embedding row, the next decode step's input
    assert np.array_equal(next_h.cpu().numpy(), O.bf16_to_f32(E[int(np.argmax(lg))]))
    # the same into a row that is not 16-byte aligned (the element-wise copy)
    nh_buf = torch.full((D + 1,), float("nan"), device="cuda")
    chk(lib.rt_lm_head_argmax(hip.ctx, Ed.data_ptr(), xd.data_ptr(), wd.data_ptr(), 1e-6, V, D, logits.data_ptr(),
                              best.data_ptr(), tok.data_ptr(), None, 0, None, None, 0, 0, nh_buf[1:].data_ptr()))
    assert np.array_equal(nh_buf[1:].cpu().numpy(), O.bf16_to_f32(E[int(np.argmax(lg))]))
    assert int(best.cpu()[0]) == 0
    hn = O.rms_norm_f64acc(x[None], w)[0]
    E32 = O.bf16_to_f32(E)
    ref = E32.astype(np.float64) @ hn.astype(np.float64)
    check_logits(lg, ref, E32, hn, f"V={V} D={D}")


def _state_dict(params):
    """The reference's checkpoint tensor names (src/rotor/bitnet_model.py:100-188) -> torch
    tensors of the oracle parameters (rotor bytes, per-tensor scales, bf16 embedding)."""
    import torch

    t = lambda a: torch.from_numpy(np.ascontiguousarray(a))
    st = {"model.embed_tokens.weight": t(params["embed"].view(np.int16)).view(torch.bfloat16),
          "model.norm.weight": t(params["final_norm"])}
    for i, L in enumerate(params["layers"]):
        p = f"model.layers.{i}"
        st[f"{p}.input_layernorm.weight"] = t(L["input_norm"])
        st[f"{p}.post_attention_layernorm.weight"] = t(L["post_norm"])
        st[f"{p}.self_attn.attn_sub_norm.weight"] = t(L["attn_sub_norm"])
        st[f"{p}.mlp.ffn_sub_norm.weight"] = t(L["ffn_sub_norm"])
        for name in ("q_proj", "k_proj", "v_proj", "o_proj", "gate_proj", "up_proj", "down_proj"):
            grp = "self_attn" if name in ("q_proj", "k_proj", "v_proj", "o_proj") else "mlp"
            W, s = L[name]
            st[f"{p}.{grp}.{name}.weight"] = t(O.pack_rotor(W))
            st[f"{p}.{grp}.{name}.weight_scale"] = t(np.array([s], np.float32))
    return st


def _write_checkpoint(path, params, cfg, max_len):
    from safetensors.torch import save_file

    save_file(_state_dict(params), str(path / "model.safetensors"))
    hf = {"vocab_size": cfg["vocab_size"], "hidden_size": cfg["d_model"], "num_hidden_layers": cfg["n_layers"],
          "num_attention_heads": cfg["n_heads"], "num_key_value_heads": cfg["n_kv_heads"],
          "intermediate_size": cfg["d_ff"], "rope_theta": cfg["rope_theta"], "rms_norm_eps": 1e-6,
          "max_position_embeddings": max_len}
    (path / "config.json").write_text(json.dumps(hf))


@pytest.fixture(scope="module")
def small_model(tmp_path_factory, hip):
    from rotor import gpu_layers
    from rotor.bitnet_model import load_bitnet_model

    path = tmp_path_factory.mktemp("ckpt")
    params = O.make_bitnet_params(11, SMALL, 64)
    _write_checkpoint(path, params, SMALL, 64)
    gpu_layers._gpu_instance = hip
    try:
        model = load_bitnet_model(str(path), use_gpu=True)
    finally:
        gpu_layers._gpu_instance = None
    return model, params


def test_model_forward_matches_oracle(small_model):
    """A checkpoint-loaded model: free-running, the final-normed hidden states stay close to
    the oracle's; teacher-forced on the device's attention outputs, the prompt's hidden
    states equal the oracle's bit for bit, and so does every decode step continuing the
    device cache (fused decode plans, LM-head kernel; logits within 3e-4 + 1e-5 |ref|)."""
    model, params = small_model
    ids = np.array([5, 999, 17, 3, 3, 250, 64, 1], np.int32)
    hn, _ = model.forward(ids, return_logits=False)
    hn_free, _ = O.bitnet_forward(params, SMALL, ids, {})
    np.testing.assert_allclose(hn, hn_free, atol=2e-2, rtol=2e-2)
    assert np.abs(hn - hn_free).mean() < 2e-3
    _, cache, oc, _ = _prefill_vs_oracle(model, params, SMALL, ids)
    for tok in (42, 7, 999):
        cache = _step_vs_oracle(model, params, SMALL, oc, cache, tok)
    assert cache.length == 11


def test_kv_cache_reads_as_per_layer_list(small_model):
    """The handle reads as the reference's list of per-layer {'k', 'v'} arrays
    (src/rotor/bitnet_model.py:223-228, src/rotor/transformer.py:250-257), shaped
    [1, Hkv, length, hd], equal to the oracle's cached keys (after RoPE) and values."""
    model, params = small_model
    ids = np.array([9, 8, 500, 7, 6], np.int32)
    _, cache = model.forward(ids, use_cache=True)
    _, cache = model.forward(np.array([33], np.int32), past_kv_cache=cache, use_cache=True)
    oc = {}
    O.bitnet_forward(params, SMALL, ids, oc)
    O.bitnet_forward(params, SMALL, [33], oc)
    Hkv, hd = SMALL["n_kv_heads"], SMALL["d_model"] // SMALL["n_heads"]
    assert len(cache) == SMALL["n_layers"] and cache.length == 6
    layers = list(cache)
    assert len(layers) == SMALL["n_layers"]
    for li, lc in enumerate(layers):
        assert set(lc) == {"k", "v"}
        for key in ("k", "v"):
            assert lc[key].shape == (1, Hkv, 6, hd) and lc[key].dtype == np.float32
            ref = oc[li][key]
            np.testing.assert_allclose(lc[key][0], ref, atol=2e-2 * max(1.0, np.abs(ref).max()), rtol=0)
    assert np.array_equal(cache[-1]["v"], layers[-1]["v"])
    with pytest.raises(IndexError):
        cache[SMALL["n_layers"]]
    model.forward(np.array([1], np.int32))  # a new sequence: the handle is stale
    with pytest.raises(ValueError, match="stale"):
        cache[0]


def test_model_batch_forward(small_model):
    """[batch, seq] ids: each row as its own sequence, stacked like the reference's
    [batch, seq, vocab] logits; a kept cache needs batch 1."""
    model, _ = small_model
    ids = np.array([[5, 6, 7, 8], [900, 1, 2, 3], [5, 6, 7, 9]], np.int32)
    logits, cache = model.forward(ids)
    assert logits.shape == (3, 4, SMALL["vocab_size"]) and cache is None
    for b in range(3):
        row, _ = model.forward(ids[b])
        assert np.array_equal(logits[b], row)
    assert np.array_equal(logits[0, :3], logits[2, :3])  # same prefix, causal
    with pytest.raises(ValueError):
        model.forward(ids, use_cache=True)
    with pytest.raises(ValueError):
        model.forward(np.array([[1, 2], [3, SMALL["vocab_size"]]], np.int32))


def test_model_all_position_logits_shape(small_model):
    model, _ = small_model
    logits, cache = model.forward(np.arange(6, dtype=np.int32))
    assert logits.shape == (6, SMALL["vocab_size"]) and cache is None
    logits2, _ = model.forward(np.arange(6, dtype=np.int32)[None])
    assert logits2.shape == (1, 6, SMALL["vocab_size"])
    assert np.array_equal(logits2[0], logits)


@pytest.mark.parametrize("graph", [True, False])
def test_greedy_generation_matches_oracle(small_model, graph):
    model, params = small_model
    prompt = np.array([7, 700, 70, 7, 77, 1], np.int32)
    toks, decided = _decode_vs_oracle(model, params, SMALL, prompt, 12, graph=graph)
    assert decided >= 9, f"only {decided} of 12 tokens decided by an oracle gap above the tolerance"


def test_model_rejects_bad_input(small_model):
    model, _ = small_model
    with pytest.raises(ValueError):
        model.forward(np.array([1000], np.int32))  # id out of range
    with pytest.raises(ValueError):
        model.generate_greedy(np.zeros(60, np.int32), 10)  # exceeds max_seq_len


def test_stale_kv_cache_rejected(small_model):
    """The device cache holds one sequence: a handle from before a new sequence (a forward
    without past cache, or generate_greedy) is refused; a current one continues."""
    model, _ = small_model
    _, c1 = model.forward(np.array([1, 2, 3], np.int32), use_cache=True)
    _, c2 = model.forward(np.array([4], np.int32), past_kv_cache=c1, use_cache=True)
    _, c3 = model.forward(np.array([5], np.int32), past_kv_cache=c2, use_cache=True)
    assert c3.length == 5
    with pytest.raises(ValueError):  # rejected ids: the cache and its handles stay valid
        model.forward(np.array([SMALL["vocab_size"]], np.int32), use_cache=True)
    model.forward(np.array([6], np.int32), past_kv_cache=c3)
    model.forward(np.array([7, 8], np.int32), use_cache=True)  # a new sequence
    with pytest.raises(ValueError, match="stale"):
        model.forward(np.array([6], np.int32), past_kv_cache=c3)
    _, d1 = model.forward(np.array([7], np.int32), use_cache=True)
    model.generate_greedy(np.array([1, 2], np.int32), 2)
    with pytest.raises(ValueError, match="stale"):
        model.forward(np.array([6], np.int32), past_kv_cache=d1)


# ---- prompts longer than the GEMV's 8 tokens: the prefill runs the quantiser launches, the
# grouped split-K / tile GEMM plans, residual-aliased linears and rt_attention (the MFMA
# prefill kernel for head_dim 128) -------------------------------------------------------
HD128 = dict(vocab_size=1000, d_model=512, n_layers=2, n_heads=4, n_kv_heads=2, d_ff=1024, rope_theta=500000.0)


def _prefill_vs_oracle(model, params, cfg, ids):
    """A multi-token forward checked layer by layer.  Every operation of a layer is
    reproducible bit for bit except attention, which sums in fp32 where the oracle sums in
    f64; a last-ulp difference there can flip one int8 value of the next quantisation and
    from then on every element differs a little.  So the oracle runs teacher-forced: each
    layer continues from the GPU's own attention output, which must be within 2e-5 of the
    oracle's attention on the same (bit-exact) q, k, v; the final hidden states must then
    equal the oracle's bit for bit.  Returns (hn, cache, oracle cache, oracle last logits)."""
    model._dev.trace = {}
    try:
        hn, cache = model.forward(ids, return_logits=False, use_cache=True)
    finally:
        trace, model._dev.trace = model._dev.trace, None
    attn = [a.cpu().numpy() for a in trace["attn"]]
    assert len(attn) == cfg["n_layers"]
    oc, ref = {}, []
    hn_o, logits_o = O.bitnet_forward(params, cfg, ids, oc, attn_in=attn, attn_ref=ref)
    for li, (a, r) in enumerate(zip(attn, ref)):
        np.testing.assert_allclose(a, r, atol=2e-5, rtol=1e-4, err_msg=f"attention of layer {li}")
    assert hn.shape == hn_o.shape == (len(ids), cfg["d_model"])
    assert np.array_equal(hn, hn_o), f"max |diff| {np.abs(hn - hn_o).max()}"
    return hn, cache, oc, logits_o


LONG_CFGS = {"small_hd64": SMALL, "hd128": HD128}


def _device_model(hip, params, cfg, max_len, max_tokens=512):
    from rotor import gpu_layers
    from rotor.bitnet_model import BitNetModel

    conf = dict(cfg, rms_norm_eps=1e-6, max_seq_len=max_len, max_batch_tokens=max_tokens)
    gpu_layers._gpu_instance = hip
    try:
        model = BitNetModel(conf, use_gpu=True)
        model.load_state(_state_dict(params))
    finally:
        gpu_layers._gpu_instance = None
    return model


@pytest.fixture(scope="module")
def long_models(hip):
    out = {}
    for name, cfg in LONG_CFGS.items():
        params = O.make_bitnet_params(23 + len(name), cfg, 192)
        out[name] = (_device_model(hip, params, cfg, 192), params, cfg)
    return out


@pytest.mark.parametrize("name", list(LONG_CFGS))
@pytest.mark.parametrize("P", [20, 130])
def test_long_prompt_forward_matches_oracle(long_models, name, P):
    model, params, cfg = long_models[name]
    ids = np.random.default_rng(P).integers(0, cfg["vocab_size"], P).astype(np.int32)
    hn, cache, oc, _ = _prefill_vs_oracle(model, params, cfg, ids)
    # decode steps after the long prefill (fused decode plans + LM head kernel)
    for tok in (42, 3):
        cache = _step_vs_oracle(model, params, cfg, oc, cache, tok)
    assert cache.length == P + 2


@pytest.mark.parametrize("name", list(LONG_CFGS))
def test_long_prompt_greedy_matches_oracle(long_models, name):
    model, params, cfg = long_models[name]
    prompt = np.random.default_rng(5).integers(0, cfg["vocab_size"], 130).astype(np.int32)
    toks, decided = _decode_vs_oracle(model, params, cfg, prompt, 8)
    assert decided >= 6, f"only {decided} of 8 tokens decided by an oracle gap above the tolerance"


WIDE16 = dict(vocab_size=1000, d_model=2048, n_layers=2, n_heads=16, n_kv_heads=4, d_ff=2048, rope_theta=500000.0)


def test_decode_attention_in_qkv_launch_bit_exact(hip):
    """Decode with the attention partials in the q/k/v launch gives the same logits, bit for
    bit, and the same graph-replayed greedy tokens as decode with the separate attention
    launch (hidden 2048, 16 / 4 heads of 128: the shapes the joint launch takes)."""
    params = O.make_bitnet_params(22, WIDE16, 96)
    prompt = np.array([3, 14, 15, 92, 65, 35, 89], np.int32)
    runs = []
    for fused in (False, True):
        model = _device_model(hip, params, WIDE16, 96)
        model._dev.attn_in_qkv = fused
        _, cache = model.forward(prompt, return_logits=False, use_cache=True)
        tok, lgs = 7, []
        for _ in range(4):
            lg, cache = model.forward(np.array([tok], np.int32), past_kv_cache=cache, use_cache=True)
            lgs.append(lg[0].copy())
            tok = int(np.argmax(lg[0]))
        toks = model.generate_greedy(prompt, 8, graph=True)
        runs.append((np.stack(lgs), toks, model._dev.state[1]["attn_fused"]))
    assert runs[0][2] == [False, False] and runs[1][2] == [True, True]
    assert np.array_equal(runs[0][0], runs[1][0])
    assert list(runs[0][1]) == list(runs[1][1])


def _embed32(params):
    E = params.get("_embed_f32")
    if E is None:
        E = params["_embed_f32"] = O.bf16_to_f32(params["embed"])
    return E


def _check_record(params, cfg, oc, ids, rec, attn_in, what):
    """One traced device forward (a prefill or a decode step; rec from the model's trace)
    against the oracle continuing from its cache oc, teacher-forced on the device's attention
    outputs attn_in (per layer [M, H*hd]; the only results that depend on fp32 summation
    order): the oracle's attention on the same q, k, v is within 2e-5 / 1e-4 of them; the last
    row's hidden state before the final norm equals the oracle's bit for bit; the fused LM
    head's logits pass check_logits.  Returns the oracle's f64 logits."""
    ref, xo = [], []
    hn_o, lg_o = O.bitnet_forward(params, cfg, ids, oc, attn_in=attn_in, attn_ref=ref, x_out=xo)
    for li, (a, r) in enumerate(zip(attn_in, ref)):
        np.testing.assert_allclose(a, r, atol=2e-5, rtol=1e-4, err_msg=f"attention of layer {li} ({what})")
    h = rec["h"].cpu().numpy()
    assert np.array_equal(h, xo[0][-1]), f"hidden state ({what}): max |diff| {np.abs(h - xo[0][-1]).max()}"
    check_logits(rec["logits"].cpu().numpy(), lg_o, _embed32(params), hn_o[-1], what)
    return lg_o


def _decode_vs_oracle(model, params, cfg, prompt, n, graph=True):
    """generate_greedy (the prompt, then n - 1 decode steps, graph-replayed or not) held to
    the north-star bar step by step.  The oracle (src/rotor/bitnet_model.py:190-244 under
    TextGenerator's greedy protocol, src/rotor/generation.py:244-279) continues from the
    device's attention outputs (the prefill's and every step's) and from its tokens; every
    forward passes _check_record (hidden state bit-exact, logits within 3e-4 + 1e-5 |ref| of
    the f64 head); every token is the argmax of its step's device logits, and the oracle's
    argmax wherever the oracle's top-2 gap exceeds twice the logit tolerance.
    Returns (tokens, number of steps such a gap decided)."""
    assert len(prompt) > 1
    model._dev.trace = {}
    try:
        toks = model.generate_greedy(prompt, n, graph=graph)
    finally:
        trace, model._dev.trace = model._dev.trace, None
    steps = trace.get("steps", [])
    assert len(trace["attn"]) == cfg["n_layers"] and len(steps) == n - 1
    recs = [(prompt, trace["prefill"], [a.cpu().numpy() for a in trace["attn"]])]
    recs += [([int(toks[i])], st, [a[None] for a in st["attn"].cpu().numpy()]) for i, st in enumerate(steps)]
    oc, decided = {}, 0
    for i, (ids, rec, attn) in enumerate(recs):
        lg_o = _check_record(params, cfg, oc, np.asarray(ids, np.int32), rec, attn, f"step {i}")
        lg = rec["logits"].cpu().numpy()
        assert toks[i] == int(np.argmax(lg)), f"step {i}: token {toks[i]} is not the argmax of its logits"
        top2 = np.sort(lg_o)[-2:]
        if top2[1] - top2[0] > 2 * (LOGIT_ATOL + LOGIT_RTOL * abs(top2[1])):
            assert toks[i] == int(np.argmax(lg_o)), f"step {i}: {toks[i]} != oracle {int(np.argmax(lg_o))}"
            decided += 1
    return toks, decided


def _step_vs_oracle(model, params, cfg, oc, cache, tok):
    """One decode step through BitNetModel.forward (eager: the fused decode plans and the
    LM-head kernel, continuing the device cache) held to _check_record."""
    model._dev.trace = {}
    try:
        logits, cache = model.forward(np.array([tok], np.int32), past_kv_cache=cache, use_cache=True)
    finally:
        trace, model._dev.trace = model._dev.trace, None
    (rec,) = trace["steps"]
    assert np.array_equal(logits[0], rec["logits"].cpu().numpy())
    _check_record(params, cfg, oc, np.array([tok], np.int32), rec, [a[None] for a in rec["attn"].cpu().numpy()],
                  f"decode step after {cache.length - 1} tokens")
    return cache


# ---- cfg 4 at its own widths: hidden 2560, ffn 6912, 20 / 5 heads x 128, vocab 128256,
# RoPE theta 500000, bf16 tied head ------------------------------------------------------
CFG4_WIDE = dict(vocab_size=128256, d_model=2560, n_layers=2, n_heads=20, n_kv_heads=5, d_ff=6912,
                 rope_theta=500000.0)
CFG4 = dict(CFG4_WIDE, n_layers=30)


@pytest.mark.timeout(600)
def test_cfg4_full_width_matches_oracle(hip):
    """Two layers at the full widths with a 400-token prompt, so that the prefill runs the
    grouped tile GEMMs including the 256 x 128 tile (gate/up at 384 < M <= 512), then
    graph-replayed greedy decode held to the north-star bar step by step (_decode_vs_oracle).
    The reference path this replaces: BitNetModel.forward (src/rotor/bitnet_model.py:190-244)
    driven by TextGenerator's greedy protocol (src/rotor/generation.py:244-279)."""
    cfg, P, n, Lmax = CFG4_WIDE, 400, 6, 512
    params = O.make_bitnet_params(4, cfg, Lmax)
    model = _device_model(hip, params, cfg, Lmax)
    prompt = np.random.default_rng(4).integers(0, cfg["vocab_size"], P).astype(np.int32)
    st = model._dev._state(P)
    assert st["gu"][0].describe() == (3, 256, 128, 216)  # the prefill's gate/up plan: 256 x 128 tiles
    toks, decided = _decode_vs_oracle(model, params, cfg, prompt, n)
    assert all(model._dev.state[1]["attn_fused"]), "decode runs the attention in the q/k/v launch"
    assert decided >= 4, f"only {decided} of {n} tokens decided by an oracle gap above the tolerance"


@pytest.fixture(scope="module")
def cfg4_model(hip):
    """The whole cfg-4 model: 30 layers at the full widths, random-init (seeded), room for the
    512-token prompt and 128 generated tokens."""
    params = O.make_bitnet_params(40, CFG4, 640, fast=True)
    model = _device_model(hip, params, CFG4, 640)
    return model, params


@pytest.mark.timeout(900)
def test_cfg4_30_layers_decode_matches_oracle(cfg4_model):
    """All 30 layers: a 16-token prompt (split-K GEMM prefill), then 4 graph-replayed decode
    steps, each held to the north-star bar (_decode_vs_oracle: hidden state bit-exact after
    30 layers, logits within 3e-4 + 1e-5 |ref| of the f64 head over the 128256 tokens)."""
    model, params = cfg4_model
    prompt = np.random.default_rng(16).integers(0, CFG4["vocab_size"], 16).astype(np.int32)
    toks, decided = _decode_vs_oracle(model, params, CFG4, prompt, 5)
    assert all(model._dev.state[1]["attn_fused"])
    assert decided >= 3, f"only {decided} of 5 tokens decided by an oracle gap above the tolerance"


@pytest.mark.timeout(900)
def test_cfg4_full_size_greedy(cfg4_model):
    """cfg 4 at its own size: the 512-token prompt and 128 greedy tokens.  The graph-replayed
    decode gives the tokens, and the final logits bit for bit, of the same steps run one by
    one through BitNetModel.forward (eager launches, device cache), with no attention wait
    given up; the prompt's forward and the first two steps are held to the north-star bar
    against the oracle (_decode_vs_oracle)."""
    model, params = cfg4_model
    P, n = 512, 128
    prompt = np.random.default_rng(4).integers(0, CFG4["vocab_size"], P).astype(np.int32)
    toks = model.generate_greedy(prompt, n, graph=True)  # raises if an attention wait gave up
    lg_graph = model._dev.logits.cpu().numpy()
    _, cache = model.forward(prompt, return_logits=False, use_cache=True)
    eager = [int(np.argmax(model._dev.logits.cpu().numpy()))]
    for i in range(n - 1):
        lg, cache = model.forward(np.array([eager[-1]], np.int32), past_kv_cache=cache, use_cache=True)
        eager.append(int(np.argmax(lg[0])))
    assert list(toks) == eager, f"graph {list(toks[:12])} ... eager {eager[:12]} ..."
    assert np.array_equal(lg[0], lg_graph)
    model._dev.attention_timeouts()
    toks3, decided = _decode_vs_oracle(model, params, CFG4, prompt, 3)
    assert list(toks3) == list(toks[:3])
