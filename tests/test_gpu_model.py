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
              (130, 0, 4, 2, 128, 192), (20, 0, 4, 2, 128, 192), (130, 0, 8, 2, 64, 192)]


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


@pytest.mark.parametrize("pos0,Lmax", [(0, 640), (63, 640), (64, 640), (639, 640), (1000, 2048)])
def test_qkv_plan_with_attention_equals_separate_launches(hip, pos0, Lmax):
    """The q/k/v decode plan with the attention attached (RoPE + KV append + split-L partials
    in the GEMV's launch, their workgroups waiting on per-KV-group arrival counts) gives the
    q, k, v outputs, the partials and the caches of the plan followed by
    rt_rope_attention_decode, bit for bit: on two runs in a row and on every replay of a
    captured graph (the counts start from zero on every launch); no wait gives up."""
    import torch

    from oracle.rotor_oracle import rope_table
    from rotor import _hip as H_

    lib, chk = _lib()
    H, Hkv, hd = 20, 5, 128
    D = H * hd
    rng = np.random.default_rng(pos0 + Lmax)
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
    # the plan, then the attention launch
    qr, kr, vr = outs()
    kc, vc = kc0.clone(), vc0.clone()
    ws_ref = torch.zeros(nbytes, dtype=torch.uint8, device="cuda")
    plan_ref = hip.plan_fused(ws_, H_.SRC_RMSNORM, x, nw, eps=1e-6, ys=[qr, kr, vr])
    plan_ref.run()
    chk(lib.rt_rope_attention_decode(hip.ctx, qr.data_ptr(), kr.data_ptr(), vr.data_ptr(), kc.data_ptr(),
                                     vc.data_ptr(), rope.data_ptr(), H, Hkv, hd, Lmax, pos.data_ptr(),
                                     ws_ref.data_ptr(), nbytes, None))
    # one launch
    q, k, v = outs()
    kcf, vcf = kc0.clone(), vc0.clone()
    ws = torch.zeros(nbytes, dtype=torch.uint8, device="cuda")
    plan = hip.plan_fused(ws_, H_.SRC_RMSNORM, x, nw, eps=1e-6, ys=[q, k, v])
    plan.attach_attention(kcf, vcf, rope, H, Hkv, hd, Lmax, pos, ws)

    def check(what):
        torch.cuda.synchronize()
        assert torch.equal(q, qr) and torch.equal(k, kr) and torch.equal(v, vr), f"q/k/v differ ({what})"
        assert torch.equal(ws, ws_ref), f"partials differ ({what})"
        assert torch.equal(kcf, kc) and torch.equal(vcf, vc), f"caches differ ({what})"

    def reset():
        for t in (q, k, v):
            t.fill_(float("nan"))
        ws.zero_()
        kcf.copy_(kc0)
        vcf.copy_(vc0)

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
    # detached, the plan runs the GEMV only
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
    three.run()
    one.run()
    torch.cuda.synchronize()


@pytest.mark.parametrize("V,D", [(1000, 512), (5000, 2560), (777, 1024)])
def test_lm_head_argmax(hip, V, D):
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
    hip._bind_stream()
    for _ in range(2):  # `best` is left zero for the next call
        chk(lib.rt_lm_head_argmax(hip.ctx, Ed.data_ptr(), xd.data_ptr(), wd.data_ptr(), 1e-6, V, D, logits.data_ptr(),
                                  best.data_ptr(), tok.data_ptr(), None, 0, None, None, 0, 0))
        lg = logits.cpu().numpy()
        assert int(tok.cpu()[0]) == int(np.argmax(lg))
        assert int(best.cpu()[0]) == 0
    hn = O.rms_norm_f64acc(x[None], w)[0]
    ref = O.bf16_to_f32(E).astype(np.float64) @ hn.astype(np.float64)
    np.testing.assert_allclose(lg, ref, atol=1e-3 * np.abs(ref).max(), rtol=1e-4)


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
    model, params = small_model
    ids = np.array([5, 999, 17, 3, 3, 250, 64, 1], np.int32)
    hn, cache = model.forward(ids, return_logits=False, use_cache=True)
    oc = {}
    hn_o, logits_o = O.bitnet_forward(params, SMALL, ids, oc)
    np.testing.assert_allclose(hn, hn_o, atol=2e-2, rtol=2e-2)
    assert np.abs(hn - hn_o).mean() < 2e-3
    # one decode step through the fused LM head, continuing the device cache
    logits, cache = model.forward(np.array([42], np.int32), past_kv_cache=cache, use_cache=True)
    _, logits_o = O.bitnet_forward(params, SMALL, [42], oc)
    np.testing.assert_allclose(logits[0], logits_o, atol=0.05 * np.abs(logits_o).max(), rtol=0)
    assert cache.length == 9


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
    n = 12
    toks = model.generate_greedy(prompt, n, graph=graph)
    ref, gaps = O.bitnet_greedy(params, SMALL, prompt, n)
    # tokens agree up to the first step whose top-2 gap is within numerical noise
    for i in range(n):
        if gaps[i] < 0.05:
            break
        assert toks[i] == ref[i], f"step {i}: {toks[i]} != {ref[i]} (gap {gaps[i]:.3f})"
    assert i >= 3, "oracle gaps too small to compare"


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
    # a decode step after the long prefill (fused decode plans + LM head kernel)
    logits, cache = model.forward(np.array([42], np.int32), past_kv_cache=cache, use_cache=True)
    _, logits_o = O.bitnet_forward(params, cfg, [42], oc)
    np.testing.assert_allclose(logits[0], logits_o, atol=0.05 * np.abs(logits_o).max(), rtol=0)
    assert cache.length == P + 1


@pytest.mark.parametrize("name", list(LONG_CFGS))
def test_long_prompt_greedy_matches_oracle(long_models, name):
    model, params, cfg = long_models[name]
    prompt = np.random.default_rng(5).integers(0, cfg["vocab_size"], 130).astype(np.int32)
    n = 8
    toks, ref, gaps = _greedy_vs_oracle(model, params, cfg, prompt, n)
    for i in range(n):
        if gaps[i] < 0.05:
            break
        assert toks[i] == ref[i], f"step {i}: {toks[i]} != {ref[i]} (gap {gaps[i]:.3f})"
    assert i >= 3, "oracle gaps too small to compare"


def test_decode_row_stats_handoff_bit_exact(hip):
    """Decode with the row-statistics hand-off (each RMSNorm input row's statistics written by
    the plan that produces the row, consumed by the next plan's prologue) gives the same
    logits, bit for bit, and the same graph-replayed greedy tokens as decode with every
    prologue reducing its row itself."""
    params = O.make_bitnet_params(21, SMALL, 64)
    prompt = np.array([3, 14, 15, 92, 65], np.int32)
    runs = []
    for stats in (False, True):
        model = _device_model(hip, params, SMALL, 64)
        model._dev.row_stats = stats
        _, cache = model.forward(prompt, return_logits=False, use_cache=True)
        tok, lgs = 7, []
        for _ in range(4):
            lg, cache = model.forward(np.array([tok], np.int32), past_kv_cache=cache, use_cache=True)
            lgs.append(lg[0].copy())
            tok = int(np.argmax(lg[0]))
        toks = model.generate_greedy(prompt, 6, graph=True)
        runs.append((np.stack(lgs), toks, "s_h1" in model._dev.state[1]))
    assert not runs[0][2] and runs[1][2], "the second model must run the statistics plans"
    assert np.array_equal(runs[0][0], runs[1][0])
    assert list(runs[0][1]) == list(runs[1][1])


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


def _greedy_vs_oracle(model, params, cfg, prompt, n):
    """generate_greedy (prefill, then graph-replayed decode steps) beside the oracle's greedy
    protocol (src/rotor/generation.py:244-279: argmax, one token per step), the oracle's
    prefill teacher-forced on the GPU prefill's attention outputs (see _prefill_vs_oracle).
    Returns (GPU tokens, oracle tokens, oracle top-2 gaps)."""
    model._dev.trace = {}
    try:
        toks = model.generate_greedy(prompt, n, graph=True)
    finally:
        trace, model._dev.trace = model._dev.trace, None
    attn = [a.cpu().numpy() for a in trace["attn"]]
    oc = {}
    _, lg = O.bitnet_forward(params, cfg, prompt, oc, attn_in=attn)
    ref, gaps = [], []
    for i in range(n):
        srt = np.sort(lg)
        ref.append(int(np.argmax(lg)))
        gaps.append(float(srt[-1] - srt[-2]))
        if i + 1 < n:
            _, lg = O.bitnet_forward(params, cfg, [ref[-1]], oc)
    return toks, ref, gaps


# ---- cfg 4 at its own widths: hidden 2560, ffn 6912, 20 / 5 heads x 128, vocab 128256,
# RoPE theta 500000, bf16 tied head; two layers (the oracle's time), a 400-token prompt so
# that the prefill runs the grouped tile GEMMs including the 256 x 128 tile (gate/up at
# 384 < M <= 512), then graph-replayed greedy decode steps -------------------------------
CFG4_WIDE = dict(vocab_size=128256, d_model=2560, n_layers=2, n_heads=20, n_kv_heads=5, d_ff=6912,
                 rope_theta=500000.0)


@pytest.mark.timeout(600)
def test_cfg4_full_width_matches_oracle(hip):
    """The reference path this replaces: BitNetModel.forward (src/rotor/bitnet_model.py:190-244)
    driven by TextGenerator's greedy protocol (src/rotor/generation.py:244-279)."""
    cfg, P, n, Lmax = CFG4_WIDE, 400, 6, 512
    params = O.make_bitnet_params(4, cfg, Lmax)
    model = _device_model(hip, params, cfg, Lmax)
    prompt = np.random.default_rng(4).integers(0, cfg["vocab_size"], P).astype(np.int32)
    # the prefill's gate/up plan is the 256 x 128 tile launch
    st = model._dev._state(P)
    assert st["gu"][0].describe() == (3, 256, 128, 216)
    # prefill hidden states, then one decode step through the fused LM head over 128256 rows
    hn, cache, oc, logits_o = _prefill_vs_oracle(model, params, cfg, prompt)
    t0 = int(np.argmax(logits_o))
    logits, _ = model.forward(np.array([t0], np.int32), past_kv_cache=cache, use_cache=True)
    _, logits1_o = O.bitnet_forward(params, cfg, [t0], oc)
    err = float(np.abs(logits[0] - logits1_o).max())
    assert err <= 0.02 * np.abs(logits1_o).max(), err
    # greedy decode: prefill + (n - 1) graph replays, tokens equal wherever the oracle's top-2
    # gap exceeds four times the logit deviation just measured
    toks, ref, gaps = _greedy_vs_oracle(model, params, cfg, prompt, n)
    assert all(model._dev.state[1]["attn_fused"]), "decode runs the attention in the q/k/v launch"
    assert ref[0] == t0
    tol = max(0.05, 4 * err)
    compared = 0
    for i in range(n):
        if gaps[i] < tol:
            break
        assert toks[i] == ref[i], f"step {i}: {toks[i]} != {ref[i]} (gap {gaps[i]:.3f}, tol {tol:.3f})"
        compared += 1
    assert compared >= 4, f"only {compared} steps had a top-2 gap above {tol:.3f}: {gaps}"
