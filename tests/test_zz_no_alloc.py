"""rt_linear_f32_noalloc (the allocation-free variant of rt_linear_f32) through the C ABI:
its outputs equal rt_linear_f32's bit for bit, call after call on the one static buffer
(a larger input, then smaller ones, then the largest that fits), and an input whose
staged activations exceed the buffer is rejected with RT_EINVAL."""
import ctypes

import numpy as np
import pytest

from oracle import rotor_oracle as O

pytestmark = pytest.mark.gpu

RT_OK, RT_EINVAL = 0, -1


def _run(lib, ctx, fn, w, x, N):
    import torch

    y = torch.full((x.shape[0], N), float("nan"), dtype=torch.float32, device="cuda")
    rc = fn(ctx, w.handle, x.data_ptr(), x.shape[0], y.data_ptr())
    torch.cuda.synchronize()
    return rc, y


# (M, N, K) in call order: the second call is smaller than the first (tile GEMM, then
# split-K GEMM), then the GEMV sizes, the one-launch M = 1, and cfg 3's down projection
# (2048 x 6912: 14.2 MB of the 16 MiB buffer)
CALLS = [(300, 640, 2560), (37, 640, 2560), (5, 2560, 2560), (1, 6912, 2560), (2048, 2560, 6912), (3, 77, 130)]


def test_noalloc_equals_linear_f32(hip):
    import torch

    from rotor import _hip

    lib = _hip.load()
    hip._bind_stream()
    for i, (M, N, K) in enumerate(CALLS):
        x, W, scale = O.make_linear_case(100 + i, M, N, K)
        w = hip.upload(O.pack_rotor(W), K, scale)
        xd = torch.from_numpy(x).cuda()
        rc, y = _run(lib, hip.ctx, lib.rt_linear_f32_noalloc, w, xd, N)
        assert rc == RT_OK, _hip.last_error()
        rc, y_ref = _run(lib, hip.ctx, lib.rt_linear_f32, w, xd, N)
        assert rc == RT_OK, _hip.last_error()
        assert torch.equal(y, y_ref), f"call {i} (M={M}, N={N}, K={K}) differs from rt_linear_f32"
        # and the oracle's exact epilogue on the same quantised inputs
        _, q, s, acc = O.ternary_linear(x, W, scale)
        assert np.array_equal(y.cpu().numpy(), (acc.astype(np.float32) * s[:, None]) * np.float32(scale))


def test_noalloc_rejects_inputs_beyond_the_buffer(hip):
    import torch

    from rotor import _hip

    lib = _hip.load()
    K, N = 6912, 64
    W = np.zeros((N, K), np.int8)
    w = hip.upload(O.pack_rotor(W), K, 1.0)
    # 2304 padded rows x 6912 + scales = 15.9 MB fits; 2560 x 6912 = 17.7 MB does not
    for M, ok in [(2049, True), (2305, False)]:
        x = torch.zeros((M, K), dtype=torch.float32, device="cuda")
        y = torch.full((M, N), 7.0, dtype=torch.float32, device="cuda")
        rc = lib.rt_linear_f32_noalloc(hip.ctx, w.handle, x.data_ptr(), M, y.data_ptr())
        torch.cuda.synchronize()
        if ok:
            assert rc == RT_OK, _hip.last_error()
            assert torch.count_nonzero(y).item() == 0
        else:
            assert rc == RT_EINVAL and "static buffer" in _hip.last_error()
            assert torch.all(y == 7.0).item()  # nothing was launched
    assert lib.rt_linear_f32_noalloc(hip.ctx, w.handle, None, 1, None) == RT_EINVAL


# The allocation-free call captured in a HIP graph: every replay, each on a new input written
# in place between replays (with the process's own eager launches and synchronisations in
# between), equals the eager rt_linear_f32 bit for bit.  The child process captures each
# shape BEFORE any launch of its kernels in that process (the tile GEMM, the split-K GEMM, the
# 128 x 160 region GEMM, the one-launch M = 1 GEMV): the first launch of a kernel then happens
# under the capture.
_CAPTURE_CHILD = r"""
import sys
sys.path[:0] = [sys.argv[1] + "/rotor-rag_amd", sys.argv[1]]
import numpy as np, torch
from oracle import rotor_oracle as O
from rotor import _hip
from rotor.gpu_ternary import HIPTernaryOps
hip = HIPTernaryOps(0)
lib = _hip.load()
for i, (M, N, K) in enumerate([(300, 640, 2560), (37, 640, 2560), (2048, 2560, 6912), (1, 6912, 2560)]):
    print(f"capture case {i}: M={M} N={N} K={K}", flush=True)
    x, W, scale = O.make_linear_case(200 + i, M, N, K)
    w = hip.upload(O.pack_rotor(W), K, scale)
    xd = torch.from_numpy(x).cuda()
    y = torch.full((M, N), float("nan"), device="cuda")
    y_ref = torch.empty((M, N), device="cuda")
    torch.cuda.synchronize()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        hip._bind_stream()
        rc = lib.rt_linear_f32_noalloc(hip.ctx, w.handle, xd.data_ptr(), M, y.data_ptr())
    assert rc == 0, _hip.last_error()
    hip._bind_stream()
    for rep in range(3):
        xd.copy_(torch.randn((M, K), device="cuda"))
        y.fill_(float("nan"))
        torch.cuda.synchronize()
        g.replay()
        assert lib.rt_linear_f32(hip.ctx, w.handle, xd.data_ptr(), M, y_ref.data_ptr()) == 0, _hip.last_error()
        torch.cuda.synchronize()
        assert torch.equal(y, y_ref), f"case {i} replay {rep}: max |diff| {(y - y_ref).abs().max().item()}"
    del g
print("CAPTURE_OK", flush=True)
"""


def test_noalloc_captured_in_a_graph(hip):
    import subprocess
    import sys
    from pathlib import Path

    root = Path(__file__).resolve().parents[1]
    r = subprocess.run([sys.executable, "-c", _CAPTURE_CHILD, str(root)], capture_output=True, text=True,
                       timeout=240)
    assert r.returncode == 0 and "CAPTURE_OK" in r.stdout, (r.stdout[-2000:], r.stderr[-3000:])
