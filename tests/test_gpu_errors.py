"""Error behaviour of the C ABI: bad arguments return RT_EINVAL with a message naming the
entry point, nothing is launched, and the context stays usable afterwards.

The reference's GPU layer reports failures by raising from PyOpenCL and its callers fall
back to NumPy (src/rotor/gpu_layers.py:14-25, src/rotor/transformer.py:74-75,145-147);
here every failure is a status + rt_last_error() message, which the Python layer turns
into RuntimeError (no fallback).
"""
import ctypes

import numpy as np
import pytest

from oracle import rotor_oracle as O

pytestmark = pytest.mark.gpu

RT_OK, RT_EINVAL = 0, -1
P = ctypes.c_void_p


@pytest.fixture(scope="module")
def lib(hip):
    from rotor import _hip

    return _hip.load()


def _err(lib):
    return lib.rt_last_error().decode()


def _upload(lib, ctx, N, K):
    # sizes are checked before the source is read: rejected shapes get a token buffer
    ok = 0 < N <= (1 << 26) and 0 < K <= (1 << 22)
    raw = np.zeros((N, (K + 3) // 4) if ok else (1, 16), np.uint8)
    out = P()
    rc = lib.rt_weights_upload(ctx, raw.ctypes.data, N, K, ctypes.c_float(1.0), ctypes.byref(out))
    return rc, out


@pytest.mark.parametrize("N,K", [(0, 64), (64, 0), (-1, 64), (64, (1 << 22) + 1), ((1 << 26) + 1, 64)])
def test_weights_upload_rejects_sizes(hip, lib, N, K):
    rc, out = _upload(lib, hip.ctx, N, K)
    assert rc == RT_EINVAL and not out.value
    assert "rt_weights_upload" in _err(lib)


def test_weights_upload_accepts_largest_k_bound(hip, lib):
    # K = 2^22 is the largest K the GEMV's int32 partial sums allow; one row uploads
    rc, out = _upload(lib, hip.ctx, 1, 1 << 22)
    assert rc == RT_OK, _err(lib)
    N, K, s = ctypes.c_int(), ctypes.c_int(), ctypes.c_float()
    assert lib.rt_weights_info(out, ctypes.byref(N), ctypes.byref(K), ctypes.byref(s)) == RT_OK
    assert (N.value, K.value, s.value) == (1, 1 << 22, 1.0)
    assert lib.rt_weights_free(out) == RT_OK


def test_null_arguments(hip, lib):
    import torch

    ctx = hip.ctx
    w = hip.upload(O.pack_rotor(np.ones((64, 64), np.int8)), 64, 1.0)
    # every operand that is not the one under test is a real buffer of the right size, so a
    # call that got past its checks would still stay in bounds
    x = torch.zeros((1, 64), dtype=torch.float32, device="cuda")
    q = torch.zeros((1, 64), dtype=torch.int8, device="cuda")
    y = torch.zeros((1, 64), dtype=torch.float32, device="cuda")
    acc = torch.zeros((1, 64), dtype=torch.int32, device="cuda")
    assert lib.rt_linear_f32(ctx, w.handle, None, 1, y.data_ptr()) == RT_EINVAL
    assert "rt_linear_f32" in _err(lib)
    assert lib.rt_linear_f32(ctx, w.handle, x.data_ptr(), 1, None) == RT_EINVAL
    assert lib.rt_linear_f32(None, w.handle, x.data_ptr(), 1, y.data_ptr()) == RT_EINVAL
    assert lib.rt_linear_i32(ctx, None, q.data_ptr(), 1, acc.data_ptr()) == RT_EINVAL
    torch.cuda.synchronize()
    assert torch.count_nonzero(y).item() == 0 and torch.count_nonzero(acc).item() == 0
    assert lib.rt_sync(None) == RT_EINVAL
    assert lib.rt_weights_info(None, None, None, None) == RT_EINVAL
    assert lib.rt_weights_free(None) == RT_OK  # like free(NULL)


def test_bad_sizes_and_shapes(hip, lib):
    import torch

    ctx = hip.ctx
    x = torch.zeros(4, 64, device="cuda")
    q = torch.zeros(4, 64, dtype=torch.int8, device="cuda")
    s = torch.zeros(4, device="cuda")
    assert lib.rt_quantize_rows(ctx, x.data_ptr(), 0, 64, q.data_ptr(), s.data_ptr()) == RT_EINVAL
    assert lib.rt_quantize_rows(ctx, x.data_ptr(), 4, 0, q.data_ptr(), s.data_ptr()) == RT_EINVAL
    w64 = hip.upload(O.pack_rotor(np.ones((64, 64), np.int8)), 64, 1.0)
    w32 = hip.upload(O.pack_rotor(np.ones((64, 32), np.int8)), 32, 1.0)
    y = torch.zeros(2, 64, device="cuda")
    # a fused plan needs one K for all weights (one input row)
    src = hip_src(x)
    ws = (P * 2)(w64.handle, w32.handle)
    ys = (P * 2)(y[0].data_ptr(), y[1].data_ptr())
    plan = P()
    rc = lib.rt_plan_create_fused(ctx, 2, ws, ctypes.byref(src), ys, None, ctypes.byref(plan))
    assert rc == RT_EINVAL and "share K" in _err(lib) and not plan.value
    # G out of range
    rc = lib.rt_plan_create_fused(ctx, 0, ws, ctypes.byref(src), ys, None, ctypes.byref(plan))
    assert rc == RT_EINVAL and "G out of range" in _err(lib)
    # activations of another K than the weights
    act = P()
    assert lib.rt_act_create(ctx, 4, 32, ctypes.byref(act)) == RT_OK
    try:
        assert lib.rt_linear_act_f32(ctx, w64.handle, act, None, y.data_ptr()) == RT_EINVAL
        assert "empty" in _err(lib) or "K" in _err(lib)
        assert lib.rt_act_quantize(ctx, x.data_ptr(), 5, act) == RT_EINVAL  # above the capacity of 4
        assert "capacity" in _err(lib)
    finally:
        assert lib.rt_act_free(act) == RT_OK
    assert lib.rt_act_create(ctx, 1, (1 << 24) + 1, ctypes.byref(act)) == RT_EINVAL


def hip_src(x):
    from rotor import _hip

    return _hip.RtSrc(_hip.SRC_QUANT, x.data_ptr(), None, None, 0.0, 0, 0)


def test_context_usable_after_errors(hip, lib):
    import torch

    _upload(lib, hip.ctx, 0, 0)  # fails
    x, W, scale = O.make_linear_case(5, 2, 130, 96)
    w = hip.upload(O.pack_rotor(W), 96, scale)
    y = hip.linear_device(w, torch.from_numpy(x)).cpu().numpy()
    y_ref, _, _, _ = O.ternary_linear(x, W, scale)
    np.testing.assert_allclose(y, y_ref, atol=3e-4, rtol=1e-5)


def test_python_layer_raises_with_message(hip):
    with pytest.raises(RuntimeError, match="too large"):
        hip.upload(np.zeros((1, (1 << 23) // 4), np.uint8), 1 << 23, 1.0)
