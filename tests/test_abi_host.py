"""Host-only checks of the C ABI library and of the Python host logic (no GPU work).

* librotor_hip.so loads and exports exactly the functions include/rotor_hip.h
  declares, and the ctypes table in rotor/_hip.py binds all of them;
* without a GPU, context creation fails cleanly with a status code and a message;
* the product's rotor byte handling (rotor/format.py) agrees with the oracle;
* TernaryLinear keeps the reference's surface; use_gpu=False computes the
  reference's CPU formula; use_gpu=True without a backend raises (no silent CPU
  fallback) and get_gpu() latches the failure like the reference's.
"""
import ctypes
import re
import subprocess
from pathlib import Path

import numpy as np
import pytest

from oracle import rotor_oracle as O

ROOT = Path(__file__).resolve().parents[1]
HEADER = ROOT / "include" / "rotor_hip.h"
LIB = ROOT / "rotor-rag_amd" / "rotor" / "lib" / "librotor_hip.so"


def declared_functions():
    text = HEADER.read_text()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    return sorted(set(re.findall(r"\b(rt_[a-z0-9_]+)\s*\(", text)))


def test_header_declares_expected_api():
    names = declared_functions()
    for n in ["rt_ctx_create", "rt_weights_upload", "rt_quantize_rows", "rt_linear_i32", "rt_linear_f32",
              "rt_plan_create", "rt_plan_run", "rt_last_error"]:
        assert n in names


@pytest.mark.parametrize("lang,compiler", [("c", "gcc"), ("c++", "g++")])
def test_header_compiles_standalone(lang, compiler, tmp_path):
    """The C ABI header is valid C and C++ on its own (what a cgo / JNI / ctypes user includes)."""
    r = subprocess.run([compiler, "-fsyntax-only", "-Wall", "-Werror", "-x", lang, str(HEADER)],
                       capture_output=True, text=True)
    assert r.returncode == 0, r.stderr


def test_library_exports_every_declared_symbol():
    assert LIB.exists(), "build librotor_hip.so first (__graft_entry__.build())"
    out = subprocess.run(["nm", "-D", "--defined-only", str(LIB)], capture_output=True, text=True, check=True).stdout
    exported = {l.split()[-1] for l in out.splitlines() if " T " in l}
    missing = [n for n in declared_functions() if n not in exported]
    assert not missing, f"declared but not exported: {missing}"
    lib = ctypes.CDLL(str(LIB))
    for n in declared_functions():
        assert hasattr(lib, n)


def test_ctypes_table_matches_header():
    from rotor import _hip

    assert sorted(_hip.SIGNATURES) == declared_functions()
    lib = _hip.load()
    assert lib.rt_version() == _hip.ABI_VERSION == 108


def test_no_gpu_context_creation_fails_cleanly():
    torch = pytest.importorskip("torch")
    if torch.cuda.is_available():
        pytest.skip("a GPU is visible")
    from rotor import _hip

    lib = _hip.load()
    n = ctypes.c_int(-1)
    assert lib.rt_device_count(ctypes.byref(n)) == 0 and n.value == 0
    ctx = ctypes.c_void_p()
    rc = lib.rt_ctx_create(0, ctypes.byref(ctx))
    assert rc == -4 and not ctx.value
    assert "no HIP device" in _hip.last_error()
    with pytest.raises(RuntimeError, match="status -4"):
        _hip.check(rc, "rt_ctx_create")
    # argument errors are reported, not crashed on
    assert lib.rt_sync(None) == -1 and "NULL" in _hip.last_error()
    assert lib.rt_linear_f32(None, None, None, 1, None) == -1


# ---------------------------------------------------------------- host format logic


def test_product_format_matches_oracle():
    from rotor.format import pack_rotor_rows, rotor_rows_to_planes, unpack_rotor_rows

    rng = np.random.default_rng(0)
    for N, K in [(1, 1), (3, 5), (17, 64), (9, 130)]:
        W = rng.choice([-1, 0, 1], size=(N, K)).astype(np.int8)
        p = pack_rotor_rows(W)
        assert np.array_equal(p, O.pack_rotor(W))
        assert np.array_equal(unpack_rotor_rows(p, K), W)
        b0, b1 = rotor_rows_to_planes(p, K)
        o0, o1 = O.bitnet_to_rotor(p, K)
        assert np.array_equal(b0, o0) and np.array_equal(b1, o1)
    allb = np.arange(256, dtype=np.uint8).reshape(1, 256)
    assert np.array_equal(unpack_rotor_rows(allb, 1024), O.unpack_rotor(allb, 1024))


def test_ternary_linear_cpu_mode_is_reference_formula():
    from rotor.transformer import TernaryLinear

    x, W, scale = O.make_linear_case(1, 6, 24, 40)
    layer = TernaryLinear(40, 24, use_gpu=False)
    layer.load_from_bitnet(O.pack_rotor(W), scale)
    assert np.array_equal(layer.weights_cache, W)
    y = layer.forward(x)
    assert y.shape == (6, 24)
    assert np.allclose(y, O.linear_ref_f32(x, W, scale), atol=1e-6)
    y3 = layer.forward(x.reshape(2, 3, 40))
    assert y3.shape == (2, 3, 24) and np.allclose(y3.reshape(6, 24), y)
    # reference attributes: LSB-first planes, flattened
    b0, b1 = O.bitnet_to_rotor(O.pack_rotor(W), 40)
    assert np.array_equal(layer.bit0, b0.reshape(-1)) and np.array_equal(layer.bit1, b1.reshape(-1))


def test_use_gpu_without_backend_raises_and_latches(monkeypatch, tmp_path):
    from rotor import _hip, gpu_layers
    from rotor.transformer import TernaryLinear

    gpu_layers._reset_for_tests()
    monkeypatch.setattr(_hip, "_lib", None)
    monkeypatch.setenv("ROTOR_HIP_LIB", str(tmp_path / "missing.so"))
    try:
        assert gpu_layers.get_gpu() is None
        assert "not found" in gpu_layers.last_error()
        # latched: a later call does not retry even if the library would now load
        monkeypatch.delenv("ROTOR_HIP_LIB")
        assert gpu_layers.get_gpu() is None
        with pytest.raises(RuntimeError, match="HIP backend unavailable"):
            TernaryLinear(8, 8, use_gpu=True)
    finally:
        gpu_layers._reset_for_tests()
        monkeypatch.setattr(_hip, "_lib", None)


def test_missing_library_raises():
    from rotor import _hip

    import os

    old = _hip._lib
    _hip._lib = None
    os.environ["ROTOR_HIP_LIB"] = "/nonexistent/librotor_hip.so"
    try:
        with pytest.raises(RuntimeError, match="not found"):
            _hip.load()
    finally:
        del os.environ["ROTOR_HIP_LIB"]
        _hip._lib = old
