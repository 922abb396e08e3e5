"""HIP backend of the ternary linear for MI355X (gfx950).

Drop-in for the reference's OpenCL plug-in ``GPUTernaryOps``
(src/rotor/gpu_ternary.py:73-208): same duck type -- ``pack_ternary_weights(W)`` and
``ternary_matmul(packed, scales, input_vec, in_dim, out_dim)`` -- plus batched entry
points (``linear``, ``linear_i32``, ``quantize_rows``, ``plan``) that the reference
lacks (it loops over tokens, src/rotor/transformer.py:134-143).

Differences from the reference, by design:
  * weights are uploaded once and stay resident (the reference re-uploads them on
    every call, src/rotor/gpu_ternary.py:160-164);
  * activations are quantised per token to int8 (absmax, src/rotor/quantization.py:
    137-149 per row) and accumulated exactly in int32 (W2A8);
  * any failure raises ``RuntimeError``; nothing falls back to the CPU.

PyTorch supplies device memory and the stream; the compute is the HIP library.
"""
from __future__ import annotations

import ctypes

import numpy as np

from . import _hip
from .format import pack_rotor_rows, unpack_rotor_rows


def _torch():
    import torch

    return torch


class DeviceTernaryWeights:
    """A device-resident ternary matrix (opaque ``rt_weights`` handle)."""

    def __init__(self, backend: "HIPTernaryOps", handle: ctypes.c_void_p, N: int, K: int, scale: float):
        self._backend = backend
        self.handle = handle
        self.out_features = N
        self.in_features = K
        self.scale = float(scale)

    @property
    def shape(self):
        return (self.out_features, self.in_features)

    def download(self) -> np.ndarray:
        """Rotor bytes [N, ceil(K/4)] read back from the device (inverse of the upload)."""
        out = np.empty((self.out_features, (self.in_features + 3) // 4), dtype=np.uint8)
        lib = _hip.load()
        _hip.check(lib.rt_weights_download(self._backend.ctx, self.handle, out.ctypes.data), "rt_weights_download")
        return out

    def free(self) -> None:
        if self.handle:
            _hip.load().rt_weights_free(self.handle)
            self.handle = None

    def __del__(self):
        try:
            self.free()
        except Exception:
            pass


class LinearPlan:
    """G ternary linears prepared for one launch (see rt_plan_create)."""

    def __init__(self, backend, handle, keep):
        self._backend = backend
        self.handle = handle
        self._keep = keep  # tensors / weights the plan's device pointers refer to

    def run(self) -> None:
        """Run the plan: one launch at M = 1 when the GEMV quantises in its prologue,
        else quantize() then gemv()."""
        b = self._backend
        b._bind_stream()
        _hip.check(_hip.load().rt_plan_run(b.ctx, self.handle), "rt_plan_run")

    def quantize(self) -> None:
        """Two-launch form of run(), first launch: per-token quantisation of the distinct inputs."""
        b = self._backend
        b._bind_stream()
        _hip.check(_hip.load().rt_plan_quantize(b.ctx, self.handle), "rt_plan_quantize")

    def gemv(self) -> None:
        """Two-launch form of run(), second launch: the ternary GEMV over all problems."""
        b = self._backend
        b._bind_stream()
        _hip.check(_hip.load().rt_plan_gemv(b.ctx, self.handle), "rt_plan_gemv")

    def attach_attention(self, k_cache, v_cache, rope, H: int, Hkv: int, hd: int, Lmax: int, pos, workspace) -> None:
        """Run the decode RoPE + KV append + attention partials of the token inside run()'s
        launch of this q/k/v plan (rt_plan_attach_attention; the arguments of
        rt_rope_attention_decode).  k_cache=None detaches."""
        if k_cache is None:
            _hip.check(_hip.load().rt_plan_attach_attention(self.handle, None, None, None, 0, 0, 0, 0, None, None, 0),
                       "rt_plan_attach_attention")
            return
        _hip.check(_hip.load().rt_plan_attach_attention(self.handle, k_cache.data_ptr(), v_cache.data_ptr(),
                                                        rope.data_ptr(), H, Hkv, hd, Lmax, pos.data_ptr(),
                                                        workspace.data_ptr(), workspace.numel() * workspace.element_size()),
                   "rt_plan_attach_attention")
        self._keep = (self._keep, k_cache, v_cache, rope, pos, workspace)

    def attention_combine(self, out, ssq) -> None:
        """Also combine the attention partials in run()'s launch (rt_plan_attention_combine):
        out fp32 [H*hd] receives the attention output, ssq float64 [H*hd/32] the sums of its
        squares per 32 outputs (an SRC_RMSNORM_SSQ plan's x and aux2).  (None, None) detaches."""
        if (out is None) != (ssq is None):
            raise ValueError("attention_combine: give both out and ssq, or neither")
        if out is not None:
            torch = _torch()
            if (out.dtype != torch.float32 or ssq.dtype != torch.float64 or not out.is_contiguous()
                    or not ssq.is_contiguous() or ssq.numel() * 32 < out.numel()):
                raise ValueError("attention_combine: out float32 [H*hd], ssq float64 [H*hd/32], contiguous")
        ptr = lambda t: t.data_ptr() if t is not None else None
        _hip.check(_hip.load().rt_plan_attention_combine(self.handle, ptr(out), ptr(ssq)), "rt_plan_attention_combine")
        self._keep = (self._keep, out, ssq)

    def set_output_ssq(self, ssq) -> None:
        """Also write, per 32 outputs (after the residual), the float64 sum of their squares
        into ssq [ceil(N/32)] (rt_plan_set_output_ssq; one-problem fused decode plans): the
        aux2 of an SRC_RMSNORM_SSQ plan reading this plan's output.  None detaches."""
        if ssq is not None:
            torch = _torch()
            if ssq.dtype != torch.float64 or not ssq.is_contiguous():
                raise ValueError("set_output_ssq: ssq float64, contiguous")
        _hip.check(_hip.load().rt_plan_set_output_ssq(self.handle, ssq.data_ptr() if ssq is not None else None),
                   "rt_plan_set_output_ssq")
        self._keep = (self._keep, ssq)

    def attention_timeouts(self) -> int:
        """Attention waits of this plan's launches that gave up (rt_plan_attention_timeouts;
        synchronises the device).  Never expected: a non-zero count means wrong results."""
        n = ctypes.c_int()
        _hip.check(_hip.load().rt_plan_attention_timeouts(self.handle, ctypes.byref(n)), "rt_plan_attention_timeouts")
        return n.value

    def describe(self):
        """(kind, tile_m, tile_n, workgroups) of the launch the plan makes (rt_plan_describe);
        kind is one of _hip.LAUNCH_*."""
        v = [ctypes.c_int() for _ in range(4)]
        _hip.check(_hip.load().rt_plan_describe(self.handle, *[ctypes.byref(x) for x in v]), "rt_plan_describe")
        return tuple(x.value for x in v)

    def free(self) -> None:
        if self.handle:
            _hip.load().rt_plan_free(self.handle)
            self.handle = None

    def __del__(self):
        try:
            self.free()
        except Exception:
            pass


class DeviceActivations:
    """Reusable quantised activations (opaque ``rt_act``): up to ``capacity`` tokens of
    ``in_features`` int8 values in the device layout, plus per-token scales."""

    def __init__(self, backend, handle, capacity: int, K: int):
        self._backend = backend
        self.handle = handle
        self.capacity = capacity
        self.in_features = K
        self.tokens = 0

    def export(self):
        """(q int8 [M, K], s fp32 [M]) device tensors of the tokens held, natural order."""
        torch = _torch()
        b = self._backend
        q = torch.empty((self.tokens, self.in_features), dtype=torch.int8, device=b.device)
        s = torch.empty((self.tokens,), dtype=torch.float32, device=b.device)
        b._bind_stream()
        _hip.check(_hip.load().rt_act_export(b.ctx, self.handle, q.data_ptr(), s.data_ptr()), "rt_act_export")
        return q, s

    def free(self) -> None:
        if self.handle:
            _hip.load().rt_act_free(self.handle)
            self.handle = None

    def __del__(self):
        try:
            self.free()
        except Exception:
            pass


class HIPTernaryOps:
    """GPUTernaryOps-compatible HIP backend bound to one device."""

    def __init__(self, device: int = 0):
        torch = _torch()
        self.lib = _hip.load()
        if not torch.cuda.is_available():
            raise RuntimeError("HIPTernaryOps: no GPU visible to PyTorch-ROCm")
        self.device_index = int(device)
        self.device = torch.device("cuda", self.device_index)
        ctx = ctypes.c_void_p()
        _hip.check(self.lib.rt_ctx_create(self.device_index, ctypes.byref(ctx)), "rt_ctx_create")
        self.ctx = ctx
        self._bind_stream()

    # -- plumbing -----------------------------------------------------------------
    def _bind_stream(self):
        torch = _torch()
        s = torch.cuda.current_stream(self.device)
        _hip.check(self.lib.rt_ctx_set_stream(self.ctx, ctypes.c_void_p(s.cuda_stream)), "rt_ctx_set_stream")

    def _dev(self, a, dtype):
        """numpy/torch -> contiguous device tensor of `dtype` on this device."""
        torch = _torch()
        if isinstance(a, torch.Tensor):
            t = a.to(device=self.device, dtype=dtype)
        else:
            t = torch.from_numpy(np.ascontiguousarray(a)).to(device=self.device, dtype=dtype)
        return t.contiguous()

    def synchronize(self):
        _hip.check(self.lib.rt_sync(self.ctx), "rt_sync")

    # -- weights ------------------------------------------------------------------
    def upload(self, rotor_bytes, in_features: int, scale: float = 1.0) -> DeviceTernaryWeights:
        """Rotor bytes [N, ceil(K/4)] (host) -> device-resident weights."""
        p = np.ascontiguousarray(rotor_bytes, dtype=np.uint8)
        if p.ndim != 2 or p.shape[1] != (in_features + 3) // 4:
            raise ValueError(f"rotor bytes of shape {p.shape} do not hold rows of {in_features} weights")
        h = ctypes.c_void_p()
        _hip.check(self.lib.rt_weights_upload(self.ctx, p.ctypes.data, p.shape[0], int(in_features),
                                              float(scale), ctypes.byref(h)), "rt_weights_upload")
        return DeviceTernaryWeights(self, h, p.shape[0], int(in_features), scale)

    def upload_device(self, rotor_bytes_dev, in_features: int, scale: float = 1.0) -> DeviceTernaryWeights:
        """Rotor bytes already on the device (uint8 tensor [N, ceil(K/4)])."""
        t = self._dev(rotor_bytes_dev, _torch().uint8)
        if t.ndim != 2 or t.shape[1] != (in_features + 3) // 4:
            raise ValueError(f"rotor bytes of shape {tuple(t.shape)} do not hold rows of {in_features} weights")
        self._bind_stream()
        h = ctypes.c_void_p()
        _hip.check(self.lib.rt_weights_upload_device(self.ctx, t.data_ptr(), t.shape[0], int(in_features),
                                                     float(scale), ctypes.byref(h)), "rt_weights_upload_device")
        self.synchronize()
        return DeviceTernaryWeights(self, h, t.shape[0], int(in_features), scale)

    def pack_ternary_weights(self, weights, scale: float = 1.0) -> DeviceTernaryWeights:
        """{-1,0,+1} [N, K] -> device weights.  src/rotor/gpu_ternary.py:112-136 (which
        returned host bytes in a w+1 code); here the rotor code is uploaded once."""
        W = np.asarray(weights)
        if W.ndim != 2:
            raise ValueError("pack_ternary_weights expects a 2-D [out, in] matrix")
        return self.upload(pack_rotor_rows(W), W.shape[1], scale)

    # -- compute ------------------------------------------------------------------
    def quantize_rows(self, x):
        """Per-token absmax int8: x [M, K] -> (q int8 [M, K], s fp32 [M]) device tensors."""
        torch = _torch()
        xt = self._dev(x, torch.float32)
        M, K = xt.shape
        q = torch.empty((M, K), dtype=torch.int8, device=self.device)
        s = torch.empty((M,), dtype=torch.float32, device=self.device)
        self._bind_stream()
        _hip.check(self.lib.rt_quantize_rows(self.ctx, xt.data_ptr(), M, K, q.data_ptr(), s.data_ptr()),
                   "rt_quantize_rows")
        return q, s

    def linear_i32(self, w: DeviceTernaryWeights, q):
        """Exact int32 accumulators q [M, K] int8 x W^T -> [M, N] (device tensor)."""
        torch = _torch()
        qt = self._dev(q, torch.int8)
        if qt.ndim != 2 or qt.shape[1] != w.in_features:
            raise ValueError(f"q of shape {tuple(qt.shape)} does not match K={w.in_features}")
        acc = torch.empty((qt.shape[0], w.out_features), dtype=torch.int32, device=self.device)
        self._bind_stream()
        _hip.check(self.lib.rt_linear_i32(self.ctx, w.handle, qt.data_ptr(), qt.shape[0], acc.data_ptr()),
                   "rt_linear_i32")
        return acc

    def linear_device(self, w: DeviceTernaryWeights, x, row_scale=None, out=None):
        """W2A8 ternary linear on device tensors: x [M, K] fp32 -> y [M, N] fp32."""
        torch = _torch()
        xt = self._dev(x, torch.float32)
        if xt.ndim != 2 or xt.shape[1] != w.in_features:
            raise ValueError(f"x of shape {tuple(xt.shape)} does not match K={w.in_features}")
        M = xt.shape[0]
        y = out if out is not None else torch.empty((M, w.out_features), dtype=torch.float32, device=self.device)
        self._bind_stream()
        if row_scale is None:
            _hip.check(self.lib.rt_linear_f32(self.ctx, w.handle, xt.data_ptr(), M, y.data_ptr()), "rt_linear_f32")
        else:
            rs = self._dev(row_scale, torch.float32).reshape(-1)
            if rs.numel() != w.out_features:
                raise ValueError("row scales must have out_features entries")
            _hip.check(self.lib.rt_linear_f32_rowscale(self.ctx, w.handle, xt.data_ptr(), M, rs.data_ptr(),
                                                       y.data_ptr()), "rt_linear_f32_rowscale")
        return y

    def linear(self, w: DeviceTernaryWeights, x):
        """x [M, K] numpy -> numpy y [M, N]; torch in -> torch (device) out."""
        torch = _torch()
        y = self.linear_device(w, x)
        if isinstance(x, torch.Tensor):
            return y
        return y.cpu().numpy()

    def ternary_matmul(self, packed_weights, scales, input_vec, in_dim: int, out_dim: int) -> np.ndarray:
        """Reference duck type (src/rotor/gpu_ternary.py:138-202): one token, per-row
        scales, numpy in and out.  ``packed_weights`` is what pack_ternary_weights
        returned."""
        if not isinstance(packed_weights, DeviceTernaryWeights):
            raise TypeError("packed_weights must come from HIPTernaryOps.pack_ternary_weights")
        if packed_weights.shape != (out_dim, in_dim):
            raise ValueError(f"weights are {packed_weights.shape}, call asked for ({out_dim}, {in_dim})")
        x = np.asarray(input_vec, dtype=np.float32).reshape(1, in_dim)
        y = self.linear_device(packed_weights, x, row_scale=np.asarray(scales, dtype=np.float32))
        return y.cpu().numpy().reshape(out_dim)

    def plan(self, weights, xs, ys) -> LinearPlan:
        """Prepare one launch of len(weights) linears: ys[g] = W_g(xs[g]); device tensors,
        all xs with the same number of rows.  Equal xs tensors share one quantisation."""
        G = len(weights)
        if not (G == len(xs) == len(ys)) or G == 0:
            raise ValueError("plan needs equal, non-zero numbers of weights, inputs and outputs")
        M = xs[0].shape[0]
        for w, x, y in zip(weights, xs, ys):
            if x.shape != (M, w.in_features) or y.shape != (M, w.out_features):
                raise ValueError("plan: tensor shapes do not match the weights")
            if not (x.is_contiguous() and y.is_contiguous()) or x.device != self.device or y.device != self.device:
                raise ValueError("plan: tensors must be contiguous and on the backend's device")
        P = ctypes.c_void_p
        wa = (P * G)(*[w.handle for w in weights])
        xa = (P * G)(*[x.data_ptr() for x in xs])
        ya = (P * G)(*[y.data_ptr() for y in ys])
        h = ctypes.c_void_p()
        _hip.check(self.lib.rt_plan_create(self.ctx, G, wa, xa, M, ya, ctypes.byref(h)), "rt_plan_create")
        return LinearPlan(self, h, (list(weights), list(xs), list(ys)))

    # -- reusable quantised activations ------------------------------------------
    def activations(self, capacity: int, in_features: int) -> DeviceActivations:
        h = ctypes.c_void_p()
        _hip.check(self.lib.rt_act_create(self.ctx, int(capacity), int(in_features), ctypes.byref(h)), "rt_act_create")
        return DeviceActivations(self, h, int(capacity), int(in_features))

    def _check_rows(self, t, act, name):
        if t.ndim != 2 or t.shape[1] != act.in_features or t.shape[0] > act.capacity:
            raise ValueError(f"{name} of shape {tuple(t.shape)} does not fit activations "
                             f"[{act.capacity}, {act.in_features}]")

    def act_quantize(self, x, act: DeviceActivations):
        """act <- per-token int8 of x [M, K] (device)."""
        xt = self._dev(x, _torch().float32)
        self._check_rows(xt, act, "x")
        self._bind_stream()
        _hip.check(self.lib.rt_act_quantize(self.ctx, xt.data_ptr(), xt.shape[0], act.handle), "rt_act_quantize")
        act.tokens = xt.shape[0]
        return act

    def act_rmsnorm_quantize(self, x, norm_w, act: DeviceActivations, eps: float = 1e-6, h_out=None):
        """act <- int8 of RMSNorm(x) * norm_w (fused); optional fp32 h_out [M, K]."""
        torch = _torch()
        xt = self._dev(x, torch.float32)
        wt = self._dev(norm_w, torch.float32).reshape(-1)
        self._check_rows(xt, act, "x")
        if wt.numel() != act.in_features:
            raise ValueError("norm weight must have in_features entries")
        self._bind_stream()
        _hip.check(self.lib.rt_act_rmsnorm_quantize(self.ctx, xt.data_ptr(), wt.data_ptr(), float(eps), xt.shape[0],
                                                    act.handle, h_out.data_ptr() if h_out is not None else None),
                   "rt_act_rmsnorm_quantize")
        act.tokens = xt.shape[0]
        return act

    def act_relu2_mul_quantize(self, gate, up, act: DeviceActivations, a_out=None):
        """act <- int8 of relu(gate)^2 * up (fused); optional fp32 a_out [M, K]."""
        torch = _torch()
        g = self._dev(gate, torch.float32)
        u = self._dev(up, torch.float32)
        self._check_rows(g, act, "gate")
        if u.shape != g.shape:
            raise ValueError("gate and up must have the same shape")
        self._bind_stream()
        _hip.check(self.lib.rt_act_relu2_mul_quantize(self.ctx, g.data_ptr(), u.data_ptr(), g.shape[0], act.handle,
                                                      a_out.data_ptr() if a_out is not None else None),
                   "rt_act_relu2_mul_quantize")
        act.tokens = g.shape[0]
        return act

    def act_relu2_mul_norm_quantize(self, gate, up, norm_w, act: DeviceActivations, eps: float = 1e-6, a_out=None):
        """act <- int8 of RMSNorm(relu(gate)^2 * up) * norm_w (fused)."""
        torch = _torch()
        g = self._dev(gate, torch.float32)
        u = self._dev(up, torch.float32)
        wt = self._dev(norm_w, torch.float32).reshape(-1)
        self._check_rows(g, act, "gate")
        if u.shape != g.shape or wt.numel() != act.in_features:
            raise ValueError("gate, up and norm weight shapes do not match")
        self._bind_stream()
        _hip.check(self.lib.rt_act_relu2_mul_norm_quantize(self.ctx, g.data_ptr(), u.data_ptr(), wt.data_ptr(),
                                                           float(eps), g.shape[0], act.handle,
                                                           a_out.data_ptr() if a_out is not None else None),
                   "rt_act_relu2_mul_norm_quantize")
        act.tokens = g.shape[0]
        return act

    def linear_act(self, w: DeviceTernaryWeights, act: DeviceActivations, out=None, residual=None):
        """y [M, N] fp32 = W2A8 linear of the activations held (+ residual [M, N])."""
        torch = _torch()
        if act.in_features != w.in_features:
            raise ValueError("activations and weights disagree on in_features")
        y = out if out is not None else torch.empty((act.tokens, w.out_features), dtype=torch.float32,
                                                    device=self.device)
        self._bind_stream()
        res = residual.data_ptr() if residual is not None else None
        _hip.check(self.lib.rt_linear_act_f32(self.ctx, w.handle, act.handle, res, y.data_ptr()), "rt_linear_act_f32")
        return y

    def plan_act(self, weights, acts, M: int, ys) -> LinearPlan:
        """One launch of len(weights) linears over caller-filled activations."""
        G = len(weights)
        if not (G == len(acts) == len(ys)) or G == 0:
            raise ValueError("plan_act needs equal, non-zero numbers of weights, activations and outputs")
        for w, a, y in zip(weights, acts, ys):
            if a.in_features != w.in_features or tuple(y.shape) != (M, w.out_features) or not y.is_contiguous():
                raise ValueError("plan_act: shapes do not match")
        P = ctypes.c_void_p
        wa = (P * G)(*[w.handle for w in weights])
        aa = (P * G)(*[a.handle for a in acts])
        ya = (P * G)(*[y.data_ptr() for y in ys])
        h = ctypes.c_void_p()
        _hip.check(self.lib.rt_plan_create_act(self.ctx, G, wa, aa, int(M), ya, ctypes.byref(h)), "rt_plan_create_act")
        return LinearPlan(self, h, (list(weights), list(acts), list(ys)))

    def plan_act_gate_up(self, w_gu, scales, act, M: int, a) -> LinearPlan:
        """Gate and up for M > 64 tokens over caller-filled activations in one GEMM launch
        (rt_plan_create_act_gate_up) on the matrix of interleave_gate_up: a fp32 [M, F] =
        relu(g)^2 * u, the values act_relu2_mul_quantize forms from separate g and u."""
        torch = _torch()
        N, K = w_gu.out_features, w_gu.in_features
        if act.in_features != K or a.dtype != torch.float32 or tuple(a.shape) != (M, N // 2) or not a.is_contiguous():
            raise ValueError("plan_act_gate_up: shapes do not match")
        h = ctypes.c_void_p()
        s_gate, s_up = scales
        _hip.check(self.lib.rt_plan_create_act_gate_up(self.ctx, w_gu.handle, float(s_gate), float(s_up), act.handle,
                                                       int(M), a.data_ptr(), ctypes.byref(h)),
                   "rt_plan_create_act_gate_up")
        return LinearPlan(self, h, (w_gu, act, a))

    def plan_fused(self, weights, mode: int, x, aux=None, aux2=None, eps: float = 1e-6, ys=None, residuals=None,
                   attn_head_dim: int = 0, attn_max_len: int = 0):
        """One-token plan whose single launch quantises its input row in the prologue:
        mode = _hip.SRC_QUANT / SRC_RMSNORM / SRC_RELU2MUL / SRC_RELU2MUL_NORM; x, aux, aux2
        device fp32 [K]; ys[g] fp32 [N_g] outputs (+ residuals[g])."""
        G = len(weights)
        if G == 0 or len(ys) != G or (residuals is not None and len(residuals) != G):
            raise ValueError("plan_fused: mismatched argument lists")
        K = weights[0].in_features
        for w, y in zip(weights, ys):
            if w.in_features != K or y.numel() != w.out_features or not y.is_contiguous():
                raise ValueError("plan_fused: shapes do not match")
        self._check_src(mode, K, x, aux, aux2, "plan_fused")
        if mode == _hip.SRC_ATTN_NORM:
            need = self.lib.rt_attention_decode_workspace(K // max(attn_head_dim, 1), attn_head_dim, attn_max_len)
            if attn_head_dim <= 0 or x.numel() * x.element_size() < need:
                raise ValueError("plan_fused: attention partials buffer too small")
        src = _hip.RtSrc(int(mode), x.data_ptr(), aux.data_ptr() if aux is not None else None,
                         aux2.data_ptr() if aux2 is not None else None, float(eps), int(attn_head_dim),
                         int(attn_max_len))
        P = ctypes.c_void_p
        wa = (P * G)(*[w.handle for w in weights])
        ya = (P * G)(*[y.data_ptr() for y in ys])
        ra = (P * G)(*[r.data_ptr() if r is not None else None for r in residuals]) if residuals is not None else None
        h = ctypes.c_void_p()
        _hip.check(self.lib.rt_plan_create_fused(self.ctx, G, wa, ctypes.byref(src), ya, ra, ctypes.byref(h)),
                   "rt_plan_create_fused")
        return LinearPlan(self, h, (list(weights), [x, aux, aux2], list(ys), list(residuals or [])))

    def _check_src(self, mode, K, x, aux, aux2, who):
        for t in ((x if mode != _hip.SRC_ATTN_NORM else None), aux,
                  (aux2 if mode != _hip.SRC_RMSNORM_SSQ else None)):
            if t is not None and (t.numel() < K or not t.is_contiguous() or t.device != self.device):
                raise ValueError(f"{who}: source tensors must be contiguous device tensors of >= K elements")
        if mode == _hip.SRC_RMSNORM_SSQ:
            t = aux2
            if (t is None or t.dtype != _torch().float64 or t.numel() < K // 32 or not t.is_contiguous()
                    or t.device != self.device):
                raise ValueError(f"{who}: RMSNORM_SSQ needs aux2 = float64 device partial sums [K/32]")

    def interleave_gate_up(self, w_gate, w_up):
        """The matrix rt_plan_create_gate_up runs: gate and up [F, K] interleaved in groups
        of 32 rows (rows 64 j .. 64 j + 31 = gate rows 32 j .., the next 32 = up rows 32 j ..),
        uploaded once; returns (matrix, (gate scale, up scale))."""
        F, K = w_gate.out_features, w_gate.in_features
        if (w_up.out_features, w_up.in_features) != (F, K) or F % 32:
            raise ValueError("interleave_gate_up: gate and up must have the same shape with F % 32 == 0")
        g, u = w_gate.download(), w_up.download()
        gu = np.stack([g.reshape(F // 32, 32, -1), u.reshape(F // 32, 32, -1)], axis=1).reshape(2 * F, -1)
        return self.upload(gu, K, 1.0), (w_gate.scale, w_up.scale)

    def plan_gate_up(self, w_gu, scales, mode: int, x, aux=None, aux2=None, eps: float = 1e-6, a=None, ssq=None,
                     g_out=None, u_out=None):
        """One-token gate/up plan of the gated FFN (rt_plan_create_gate_up) on the matrix of
        interleave_gate_up: a[i] = relu(g_i)^2 * u_i (fp32 [F]) and ssq[j] (float64 [F/32]) =
        sum of a^2 over outputs 32 j .. 32 j + 31, the input of an SRC_RMSNORM_SSQ plan."""
        torch = _torch()
        N, K = w_gu.out_features, w_gu.in_features
        F = N // 2
        if N % 64:
            raise ValueError("plan_gate_up: the interleaved matrix needs N % 64 == 0")
        self._check_src(mode, K, x, aux, aux2, "plan_gate_up")
        if a is None or a.numel() < F or a.dtype != torch.float32 or not a.is_contiguous():
            raise ValueError("plan_gate_up: a must be a contiguous float32 device tensor of F elements")
        if ssq is None or ssq.numel() < F // 32 or ssq.dtype != torch.float64 or not ssq.is_contiguous():
            raise ValueError("plan_gate_up: ssq must be a contiguous float64 device tensor of F/32 elements")
        for t in (g_out, u_out):
            if t is not None and (t.numel() < F or t.dtype != torch.float32 or not t.is_contiguous()):
                raise ValueError("plan_gate_up: g_out / u_out must be float32 device tensors of F elements")
        ptr = lambda t: t.data_ptr() if t is not None else None
        src = _hip.RtSrc(int(mode), x.data_ptr(), ptr(aux), ptr(aux2), float(eps), 0, 0)
        h = ctypes.c_void_p()
        s_gate, s_up = scales
        _hip.check(self.lib.rt_plan_create_gate_up(self.ctx, w_gu.handle, float(s_gate), float(s_up), ctypes.byref(src),
                                                   a.data_ptr(), ssq.data_ptr(), ptr(g_out), ptr(u_out),
                                                   ctypes.byref(h)), "rt_plan_create_gate_up")
        return LinearPlan(self, h, ([w_gu], [x, aux, aux2], [a, ssq], [g_out, u_out]))

    def __del__(self):
        try:
            if getattr(self, "ctx", None):
                self.lib.rt_ctx_destroy(self.ctx)
                self.ctx = None
        except Exception:
            pass


__all__ = ["HIPTernaryOps", "DeviceTernaryWeights", "DeviceActivations", "LinearPlan", "unpack_rotor_rows"]
