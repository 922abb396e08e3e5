"""Pins the CPU oracle (oracle/rotor_oracle.py, oracle/rotor_oracle.c) before it is
trusted as the checker of the HIP path:
  * the reference's known-answer vectors (tests/golden/kats.json, with citations);
  * vectors produced by the reference's own C core (tests/golden/ref_core_vectors.npz,
    written by tests/golden/make_golden.py from native/c/rotor_core.c);
  * closed forms and invariants that a dropped term, a wrong sign or index, or a
    transposed operand would break;
  * the C restatement against the NumPy one.
"""
import ctypes
import json
from pathlib import Path

import numpy as np
import pytest

from oracle import rotor_oracle as O

ROOT = Path(__file__).resolve().parents[1]
GOLD = ROOT / "tests" / "golden"
KATS = json.loads((GOLD / "kats.json").read_text())
REF = np.load(GOLD / "ref_core_vectors.npz", allow_pickle=False)


# ---------------------------------------------------------------- format KATs


def test_encode_kat():
    k = KATS["encode"]
    b0, b1 = O.encode(k["values"])
    assert b0.tolist() == k["bit0"] and b1.tolist() == k["bit1"]
    assert O.decode(b0, b1).tolist() == k["values"]


def test_pack_kat_and_roundtrip():
    k = KATS["pack"]
    b0, b1 = O.encode(k["values"])
    packed = O.pack(b0, b1)
    assert packed.tolist() == k["packed"]
    u0, u1 = O.unpack(packed, 8)
    assert O.decode(u0, u1).tolist() == k["values"]
    assert O.pack_rotor(np.array([k["values"]])).tolist() == [k["packed"]]


@pytest.mark.parametrize("case", KATS["bytes"], ids=lambda c: hex(c["byte"]))
def test_byte_kats(case):
    w = O.unpack_rotor(np.array([[case["byte"]]], np.uint8), 4)
    assert w[0].tolist() == case["weights"]
    b0, b1 = O.bitnet_to_rotor(np.array([[case["byte"]]], np.uint8))
    if "bit0" in case:
        assert int(b0[0, 0]) == case["bit0"] and int(b1[0, 0]) == case["bit1"]
    assert O.rotor_unpack_weights(b0, b1, 1, 4)[0].tolist() == case["weights"]


def test_error_code_decodes_to_zero_and_is_flagged():
    # code 11 is reserved: value bit0 - bit1 = 0 (src/rotor/core.py:233-243; C treats it as 0)
    assert O.unpack_rotor(np.array([[0xFF]], np.uint8), 4)[0].tolist() == [0, 0, 0, 0]
    assert O.check_errors(np.array([1, 0, 1]), np.array([1, 1, 0])).tolist() == [True, False, False]


# ---------------------------------------------------------------- vs the reference C core


@pytest.mark.parametrize("name", ["all_bytes", "ragged", "square"])
def test_conversion_matches_reference_core(name):
    src, cols = REF[f"{name}_src"], int(REF[f"{name}_cols"])
    b0, b1 = O.bitnet_to_rotor(src, cols)
    assert np.array_equal(b0, REF[f"{name}_bit0"]) and np.array_equal(b1, REF[f"{name}_bit1"])
    assert np.array_equal(O.rotor_unpack_weights(b0, b1, src.shape[0], cols), REF[f"{name}_w"])
    # the 4/byte rotor code read directly gives the same weights
    assert np.array_equal(O.unpack_rotor(src, cols), REF[f"{name}_w"])


def test_pack_unpack_match_reference_core():
    v = REF["enc_values"]
    b0, b1 = O.encode(v)
    assert np.array_equal(b0, REF["enc_bit0"]) and np.array_equal(b1, REF["enc_bit1"])
    assert np.array_equal(O.pack(b0, b1), REF["enc_packed"])
    u0, u1 = O.unpack(REF["enc_packed"], len(v))
    assert np.array_equal(u0, REF["unp_bit0"]) and np.array_equal(u1, REF["unp_bit1"])


def test_exhaustive_byte_table():
    # every byte value, independent statement: field f -> {0:0, 1:-1, 2:+1, 3:0}
    table = {0: 0, 1: -1, 2: 1, 3: 0}
    allb = np.arange(256, dtype=np.uint8).reshape(1, 256)
    w = O.unpack_rotor(allb, 1024).reshape(256, 4)
    for b in range(256):
        assert w[b].tolist() == [table[(b >> (2 * j)) & 3] for j in range(4)]
    # pack_rotor inverts unpack_rotor on valid codes
    W = np.random.default_rng(0).choice([-1, 0, 1], size=(7, 33)).astype(np.int8)
    assert np.array_equal(O.unpack_rotor(O.pack_rotor(W), 33), W)


def test_live_reference_core_if_built():
    lib_path = ROOT / "oracle" / "_ref" / "librotor_core.so"
    if not lib_path.exists():
        pytest.skip("oracle/_ref not built")
    lib = ctypes.CDLL(str(lib_path))
    sz = ctypes.c_size_t
    lib.bitnet_to_rotor.argtypes = [ctypes.c_void_p, sz, sz, ctypes.c_void_p, ctypes.c_void_p]
    lib.bitnet_to_rotor.restype = None
    rng = np.random.default_rng(5)
    for rows, cols in [(1, 1), (3, 7), (11, 129), (65, 640)]:
        src = rng.integers(0, 256, size=(rows, (cols + 3) // 4), dtype=np.uint8)
        ob = (cols + 7) // 8
        b0 = np.zeros((rows, ob), np.uint8)
        b1 = np.zeros((rows, ob), np.uint8)
        lib.bitnet_to_rotor(src.ctypes.data, rows, cols, b0.ctypes.data, b1.ctypes.data)
        o0, o1 = O.bitnet_to_rotor(src, cols)
        assert np.array_equal(b0, o0) and np.array_equal(b1, o1)


def _cpubase():
    p = ROOT / "oracle" / "libcpubase.so"
    if not p.exists():
        pytest.skip("oracle/libcpubase.so not built (make -C oracle)")
    lib = ctypes.CDLL(str(p))
    sz, vp = ctypes.c_size_t, ctypes.c_void_p
    lib.cb_unpack_planes.argtypes = [vp, vp, sz, sz, vp]
    lib.cb_unpack_planes.restype = None
    lib.cb_sign_matvec.argtypes = [vp, vp, vp, sz, sz, vp, vp, vp]
    lib.cb_sign_matvec.restype = None
    return lib


@pytest.mark.parametrize("rows,cols", [(1, 1), (3, 7), (11, 129), (65, 640), (4, 2560)])
def test_cpu_baseline_unpack_planes(rows, cols):
    """The timed CPU baseline's unpack equals the oracle's rotor_unpack_weights (and so the
    reference core's, which the oracle is pinned to)."""
    lib = _cpubase()
    rng = np.random.default_rng(rows * cols)
    W = rng.choice(np.array([-1, 0, 1], np.int8), size=(rows, cols))
    b0, b1 = O.bitnet_to_rotor(O.pack_rotor(W), cols)
    out = np.zeros((rows, cols), np.int8)
    lib.cb_unpack_planes(b0.ctypes.data, b1.ctypes.data, rows, cols, out.ctypes.data)
    assert np.array_equal(out, W)
    assert np.array_equal(out, O.rotor_unpack_weights(b0, b1, rows, cols))


@pytest.mark.parametrize("m,n", [(1, 1), (5, 33), (64, 2560), (7, 8160)])
def test_cpu_baseline_sign_matvec(m, n):
    """The 1-bit-activation mat-vec of the reference core (rotor_matvec): y = W sign(x),
    brute force, with zeros in x mapping to 0; equal to the reference core's own output when
    oracle/_ref is built (n <= 8160 keeps its 8-bit lane sums exact)."""
    lib = _cpubase()
    rng = np.random.default_rng(m + n)
    W = rng.choice(np.array([-1, 0, 1], np.int8), size=(m, n))
    x = rng.standard_normal(n).astype(np.float32)
    x[::7] = 0.0
    wb0, wb1 = (W == 1).astype(np.uint8), (W == -1).astype(np.uint8)
    y = np.zeros(m, np.int32)
    s0, s1 = np.zeros(n, np.uint8), np.zeros(n, np.uint8)
    lib.cb_sign_matvec(wb0.ctypes.data, wb1.ctypes.data, x.ctypes.data, m, n, s0.ctypes.data, s1.ctypes.data,
                       y.ctypes.data)
    brute = [sum(int(W[i, k]) * (1 if x[k] > 0 else -1 if x[k] < 0 else 0) for k in range(n)) for i in range(min(m, 3))]
    assert y[:len(brute)].tolist() == brute
    assert np.array_equal(y, W.astype(np.int64) @ np.sign(x).astype(np.int64))
    ref = ROOT / "oracle" / "_ref" / "librotor_core.so"
    if ref.exists():
        rl = ctypes.CDLL(str(ref))
        sz, vp = ctypes.c_size_t, ctypes.c_void_p
        rl.rotor_matvec.argtypes = [vp, vp, vp, sz, sz, vp]
        rl.rotor_matvec.restype = None
        yr = np.zeros(m, np.int32)
        rl.rotor_matvec(wb0.ctypes.data, wb1.ctypes.data, x.ctypes.data, m, n, yr.ctypes.data)
        assert np.array_equal(y, yr)


# ---------------------------------------------------------------- quantiser


def test_quant_kat():
    k = KATS["quant"]
    q, s = O.quant_rows(np.array([k["x"]], np.float32))
    assert q[0].tolist() == k["q"] and float(s[0]) == k["s"]


def test_quant_zero_row_and_sign():
    q, s = O.quant_rows(np.zeros((2, 5), np.float32))
    assert (q == 0).all() and (s == 1.0).all()
    q, s = O.quant_rows(np.array([[-3.0, 1.5, 0.0]], np.float32))
    assert q[0].tolist() == [-127, 64, 0]  # 1.5/(3/127) = 63.5 -> 64 (half to even)


def test_quant_invariants():
    rng = np.random.default_rng(1)
    x = rng.standard_normal((40, 333), dtype=np.float32) * rng.uniform(0.01, 100, size=(40, 1)).astype(np.float32)
    q, s = O.quant_rows(x)
    assert q.dtype == np.int8 and s.dtype == np.float32
    # the largest |x| of each row maps to +-127 with the sign of x
    i = np.argmax(np.abs(x), axis=1)
    assert np.array_equal(q[np.arange(40), i], (127 * np.sign(x[np.arange(40), i])).astype(np.int8))
    assert np.abs(q.astype(int)).max() <= 127
    # reconstruction error at most half a step (plus fp32 rounding)
    err = np.abs(x - q.astype(np.float32) * s[:, None])
    assert (err <= 0.5 * s[:, None] * (1 + 1e-5)).all()
    # s = amax/127 in float32
    assert np.array_equal(s, (np.abs(x).max(axis=1) / np.float32(127)).astype(np.float32))
    # per-row independence: quantising one row alone gives the same row
    q1, s1 = O.quant_rows(x[7:8])
    assert np.array_equal(q1[0], q[7]) and s1[0] == s[7]


def test_quant_against_float64_rounding():
    # q = round(x/s) computed in float64 agrees except where x/s sits within fp32
    # rounding of a .5 tie -- none occur for these inputs
    rng = np.random.default_rng(2)
    x = rng.standard_normal((8, 1000), dtype=np.float32)
    q, s = O.quant_rows(x)
    r64 = x.astype(np.float64) / s.astype(np.float64)[:, None]
    near_tie = np.abs(np.abs(r64 - np.floor(r64)) - 0.5) < 1e-4
    assert np.array_equal(q[~near_tie], np.clip(np.round(r64), -128, 127).astype(np.int8)[~near_tie])


# ---------------------------------------------------------------- linear


def test_linear_i64_brute_force():
    rng = np.random.default_rng(3)
    q = rng.integers(-128, 128, size=(3, 9)).astype(np.int8)
    W = rng.choice([-1, 0, 1], size=(4, 9)).astype(np.int8)
    acc = O.linear_i64(q, W)
    for m in range(3):
        for n in range(4):
            assert acc[m, n] == sum(int(q[m, k]) * int(W[n, k]) for k in range(9))
    # not transposed: shape [M, N]
    assert acc.shape == (3, 4)


def test_linear_i64_fast_and_linearity():
    rng = np.random.default_rng(4)
    q1 = rng.integers(-128, 128, size=(5, 700)).astype(np.int8)
    q2 = rng.integers(-64, 64, size=(5, 700)).astype(np.int8)
    W = rng.choice([-1, 0, 1], size=(31, 700)).astype(np.int8)
    a1 = O.linear_i64(q1, W)
    assert np.array_equal(a1, O.linear_i64_fast(q1, W))
    # linearity in q
    assert np.array_equal(O.linear_i64(q1.astype(np.int64) + q2, W), a1 + O.linear_i64(q2, W))
    # extreme magnitudes: all -128 against all +1 / -1
    K = 6912
    qmin = np.full((1, K), -128, np.int8)
    Wpm = np.stack([np.ones(K, np.int8), -np.ones(K, np.int8)])
    assert O.linear_i64_fast(qmin, Wpm).tolist() == [[-128 * K, 128 * K]]


def test_ternary_linear_closed_form():
    # y = (q*s) . W * scale evaluated in float64 on the same quantised inputs
    x, W, scale = O.make_linear_case(11, 3, 50, 256)
    y, q, s, acc = O.ternary_linear(x, W, scale)
    y64 = (acc.astype(np.float64) * s.astype(np.float64)[:, None]) * np.float64(scale)
    assert np.abs(y - y64).max() < 1e-5
    assert np.array_equal(acc, O.linear_i64(q, W))
    # the reference formula on unquantised x stays within the quantisation error
    yr = O.linear_ref_f32(x, W, scale)
    assert np.abs(yr - y).max() < 0.05


def test_linear_ref_reshape_rules():
    # 3-D inputs flatten to [B*S, K] and come back as [B, S, N] (src/rotor/transformer.py:121-155)
    x = np.random.default_rng(6).standard_normal((2, 3, 16), dtype=np.float32)
    W = np.eye(4, 16, dtype=np.int8)
    y = O.linear_ref_f32(x, W, 2.0)
    assert y.shape == (2, 3, 4)
    assert np.allclose(y, 2.0 * x[..., :4])


def test_rms_norm_and_relu2_closed_forms():
    x = np.full((2, 8), 3.0, np.float32)
    assert np.allclose(O.rms_norm(x, np.ones(8), eps=0.0), 1.0)
    w = np.arange(8, dtype=np.float32)
    assert np.allclose(O.rms_norm(-x, w, eps=0.0), -w)
    g = np.array([-2.0, 0.0, 3.0], np.float32)
    u = np.array([5.0, 5.0, -2.0], np.float32)
    assert O.relu2_gate(g, u).tolist() == [0.0, 0.0, -18.0]


# ---------------------------------------------------------------- C restatement


@pytest.fixture(scope="module")
def corc():
    p = ROOT / "oracle" / "liboracle.so"
    if not p.exists():
        pytest.skip("oracle/liboracle.so not built (make -C oracle)")
    lib = ctypes.CDLL(str(p))
    v, sz = ctypes.c_void_p, ctypes.c_size_t
    lib.orc_pack_rotor.argtypes = [v, sz, sz, v]
    lib.orc_unpack_rotor.argtypes = [v, sz, sz, v]
    lib.orc_bitnet_to_rotor.argtypes = [v, sz, sz, v, v]
    lib.orc_unpack_planes.argtypes = [v, v, sz, sz, v]
    lib.orc_quant_rows.argtypes = [v, sz, sz, v, v]
    lib.orc_linear_i64.argtypes = [v, v, sz, sz, sz, v]
    lib.orc_linear_i64_packed.argtypes = [v, v, sz, sz, sz, v]
    return lib


def test_c_oracle_matches_numpy_oracle(corc):
    rng = np.random.default_rng(7)
    N, K, M = 45, 203, 6
    W = rng.choice([-1, 0, 1], size=(N, K)).astype(np.int8)
    kb = (K + 3) // 4
    p = np.zeros((N, kb), np.uint8)
    corc.orc_pack_rotor(W.ctypes.data, N, K, p.ctypes.data)
    assert np.array_equal(p, O.pack_rotor(W))
    W2 = np.zeros((N, K), np.int8)
    corc.orc_unpack_rotor(p.ctypes.data, N, K, W2.ctypes.data)
    assert np.array_equal(W2, W)
    b0 = np.zeros((N, (K + 7) // 8), np.uint8)
    b1 = np.zeros_like(b0)
    corc.orc_bitnet_to_rotor(p.ctypes.data, N, K, b0.ctypes.data, b1.ctypes.data)
    o0, o1 = O.bitnet_to_rotor(p, K)
    assert np.array_equal(b0, o0) and np.array_equal(b1, o1)
    W3 = np.zeros((N, K), np.int8)
    corc.orc_unpack_planes(b0.ctypes.data, b1.ctypes.data, N, K, W3.ctypes.data)
    assert np.array_equal(W3, W)
    x = rng.standard_normal((M, K), dtype=np.float32) * 3
    x[2] = 0
    q = np.zeros((M, K), np.int8)
    s = np.zeros(M, np.float32)
    corc.orc_quant_rows(x.ctypes.data, M, K, q.ctypes.data, s.ctypes.data)
    qo, so = O.quant_rows(x)
    assert np.array_equal(q, qo) and np.array_equal(s, so)
    acc = np.zeros((M, N), np.int64)
    corc.orc_linear_i64(q.ctypes.data, W.ctypes.data, M, N, K, acc.ctypes.data)
    assert np.array_equal(acc, O.linear_i64(q, W))
    acc2 = np.zeros((M, N), np.int64)
    corc.orc_linear_i64_packed(q.ctypes.data, p.ctypes.data, M, N, K, acc2.ctypes.data)
    assert np.array_equal(acc2, acc)


def test_rms_norm_f64acc():
    x = np.full((3, 64), -2.0, np.float32)
    w = np.linspace(0.5, 1.5, 64).astype(np.float32)
    assert np.allclose(O.rms_norm_f64acc(x, w, eps=0.0), -w, atol=0, rtol=1e-7)
    rng = np.random.default_rng(8)
    x = rng.standard_normal((5, 2560), dtype=np.float32) * 3
    a, b = O.rms_norm_f64acc(x, w[:1].repeat(2560)), O.rms_norm(x, w[:1].repeat(2560))
    assert np.abs(a - b).max() <= 2 * np.spacing(np.abs(b).max())


def test_ffn_block_w2a8_composes_pinned_parts():
    rng = np.random.default_rng(10)
    D, F = 64, 96
    x = rng.standard_normal((2, D), dtype=np.float32)
    nw = rng.uniform(0.5, 1.5, D).astype(np.float32)
    Wg, sg = O.make_ternary(rng, F, D)
    Wu, su = O.make_ternary(rng, F, D)
    Wd, sd = O.make_ternary(rng, D, F)
    y, it = O.ffn_block_w2a8(x, nw, Wg, sg, Wu, su, Wd, sd)
    assert y.shape == (2, D)
    # each stage is the pinned function applied to the previous stage
    assert np.array_equal(it["acc_g"], O.linear_i64(it["qh"], Wg))
    assert np.array_equal(it["a"], O.relu2_gate(it["g"], it["u"]))
    q, s = O.quant_rows(it["a"])
    assert np.array_equal(q, it["qa"]) and np.array_equal(s, it["sa"])
    assert np.array_equal(it["acc_d"], O.linear_i64(q, Wd))
    # and agrees with the reference-formula chain within the quantisation error
    y_ref, _ = O.ffn_block(x, nw, Wg, sg, Wu, su, Wd, sd)
    assert np.abs(y - y_ref).max() < 0.05 * max(1.0, np.abs(y_ref).max())


def test_bf16_roundtrip_and_rounding():
    x = np.array([1.0, -2.5, 3.1415927, 1e-3, 65504.0], np.float32)
    b = O.f32_to_bf16(x)
    y = O.bf16_to_f32(b)
    assert np.abs(y - x).max() <= np.abs(x).max() * 2 ** -8
    assert np.array_equal(O.f32_to_bf16(y), b)  # bf16 values are fixed points
    # round half to even on the 16 dropped bits
    assert O.f32_to_bf16(np.array([np.uint32(0x3F808000)], np.uint32).view(np.float32))[0] == 0x3F80
    assert O.f32_to_bf16(np.array([np.uint32(0x3F818000)], np.uint32).view(np.float32))[0] == 0x3F82


def test_rope_properties():
    tab = O.rope_table(16, 8, 10000.0)
    x = np.random.default_rng(0).standard_normal((3, 2, 8)).astype(np.float32)
    assert np.array_equal(O.apply_rope(x, tab, 0)[0], x[0])  # position 0 is the identity
    r = O.apply_rope(x, tab, 5)
    assert np.allclose(np.linalg.norm(r, axis=-1), np.linalg.norm(x, axis=-1), rtol=1e-5)  # rotation
    # relative-position property: <rope(q, p), rope(k, p')> depends on p - p' only
    q, k = x[:1, :1], x[1:2, :1]
    a = (O.apply_rope(q, tab, 7) * O.apply_rope(k, tab, 4)).sum()
    b = (O.apply_rope(q, tab, 10) * O.apply_rope(k, tab, 7)).sum()
    assert abs(a - b) < 1e-4


@pytest.mark.parametrize("hd,theta", [(128, 500000.0), (64, 10000.0), (8, 10000.0)])
def test_rope_frequency_kat(hd, theta):
    """Known answer for the frequencies (which the invariants above leave free): at position
    p, pair i of the rotate-half layout (dims i and i + hd/2) turns by exactly
    p * theta^(-2i/hd) radians.  The angles here come from exp/log in float64, not from the
    power the table uses, and the rotation is applied to unit vectors, so a wrong exponent
    (i/hd, 2i/(hd/2), a dropped minus) or a swapped cos/sin fails."""
    from rotor.bitnet_model import rope_table as product_table

    tab = O.rope_table(8, hd, theta)
    i = np.arange(hd // 2)
    for p in (1, 3, 7):
        ang = p * np.exp(-(2.0 * i / hd) * np.log(theta))
        np.testing.assert_allclose(tab[p, :, 0], np.cos(ang), rtol=0, atol=1e-7)
        np.testing.assert_allclose(tab[p, :, 1], np.sin(ang), rtol=0, atol=1e-7)
        # e_i (first half) rotates to (cos, sin) in dims (i, i + hd/2)
        x = np.zeros((1, 1, hd), np.float32)
        x[0, 0, 1] = 1.0
        r = O.apply_rope(x, tab, p)[0, 0]
        assert abs(r[1] - np.cos(ang[1])) < 1e-6 and abs(r[1 + hd // 2] - np.sin(ang[1])) < 1e-6
    # pair 0 turns by exactly p radians, the last pair by p * theta^(-(hd-2)/hd)
    assert abs(np.arctan2(tab[1, 0, 1], tab[1, 0, 0]) - 1.0) < 1e-7
    assert abs(np.arctan2(tab[1, -1, 1], tab[1, -1, 0]) - theta ** (-(hd - 2) / hd)) < 1e-7
    # the table the product uploads is the same
    assert np.array_equal(product_table(8, hd, theta), tab)


def test_attention_closed_forms():
    rng = np.random.default_rng(1)
    hd = 8
    q = rng.standard_normal((2, 4, hd)).astype(np.float32)
    K = rng.standard_normal((2, 2, hd)).astype(np.float32)
    V = rng.standard_normal((2, 2, hd)).astype(np.float32)
    out = O.causal_gqa_attention(q, K, V, 0)
    # query 0 sees only key 0: output = V[kv head][0]; GQA maps heads 0,1 -> kv 0, 2,3 -> kv 1
    assert np.allclose(out[0, 0], V[0, 0]) and np.allclose(out[0, 3], V[1, 0])
    # equal keys -> uniform weights -> mean of the visible values
    Ke = np.repeat(K[:, :1], 2, axis=1)
    out2 = O.causal_gqa_attention(q, Ke, V, 0)
    assert np.allclose(out2[1, 0], V[0, :2].mean(0), atol=1e-6)


def _two_key_case(hd, a, seed):
    """q = a e_0, keys [e_0, 0], values [v0, v1]: the query at position 1 sees both keys
    with scores a * scale and 0, so out = sig(a * scale) v0 + (1 - sig(a * scale)) v1."""
    rng = np.random.default_rng(seed)
    q = np.zeros((1, 1, hd), np.float32)
    q[0, 0, 0] = a
    K = np.zeros((1, 2, hd), np.float32)
    K[0, 0, 0] = 1.0
    V = rng.standard_normal((1, 2, hd)).astype(np.float32)
    return q, K, V


def two_key_expected(V, a, scale):
    w0 = 1.0 / (1.0 + np.exp(-a * scale))
    return w0 * V[0, 0].astype(np.float64) + (1.0 - w0) * V[0, 1].astype(np.float64)


@pytest.mark.parametrize("hd", [64, 128])
def test_attention_score_scale_kat(hd):
    """Known answer for the score scale 1/sqrt(head_dim) (src/rotor/transformer.py:266-267),
    which the closed forms above leave free: with two keys whose scores are a/sqrt(hd) and 0
    the output is the logistic mix sig(a/sqrt(hd)) v0 + (1 - sig) v1.  A scale of 1/hd, or
    none, gives a mix that differs by more than 1e-2 here."""
    a = 8.0
    q, K, V = _two_key_case(hd, a, hd)
    out = O.causal_gqa_attention(q, K, V, 1)[0, 0].astype(np.float64)
    np.testing.assert_allclose(out, two_key_expected(V, a, 1.0 / np.sqrt(hd)), rtol=0, atol=2e-6)
    for wrong in (1.0 / hd, 1.0):
        assert np.abs(out - two_key_expected(V, a, wrong)).max() > 1e-2


def test_bitnet_incremental_equals_full():
    cfg = dict(vocab_size=50, d_model=32, n_layers=2, n_heads=4, n_kv_heads=2, d_ff=48)
    p = O.make_bitnet_params(3, cfg, 16)
    ids = [3, 17, 42, 5]
    full_cache, inc_cache = {}, {}
    h_full, _ = O.bitnet_forward(p, cfg, ids, full_cache)
    h_a, _ = O.bitnet_forward(p, cfg, ids[:3], inc_cache)
    h_b, logits = O.bitnet_forward(p, cfg, ids[3:], inc_cache)
    assert np.allclose(h_full[:3], h_a, atol=1e-5) and np.allclose(h_full[3], h_b[0], atol=1e-5)
    assert full_cache["len"] == inc_cache["len"] == 4
