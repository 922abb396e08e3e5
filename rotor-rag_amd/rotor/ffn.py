"""Ternary FFN block of the benchmark configuration (BitNet-2B shape):
RMSNorm(d_model) -> gate & up ternary linears (d_model -> d_ff) -> relu(gate)^2 * up ->
ternary down linear (d_ff -> d_model).

It is the caller of the ternary linear that the reference's GatedFFN.forward is
(src/rotor/transformer.py:320-341: gate_proj/up_proj on the same input, elementwise
activation, down_proj), with the configuration's relu^2 activation and no sub-norm.

On the GPU the block never leaves the device.  One token (decode) is two launches when
d_model and d_ff are multiples of 64 and d_ff <= 8192:
  1. gate/up pair plan over a copy of gate and up interleaved in 32-row groups: RMSNorm +
     int8 quantiser in the prologue, relu^2(gate) * up in the epilogue (rt_plan_create_gate_up)
  2. down plan quantising that row in its prologue            (rt_plan_create_fused)
Otherwise, and for several tokens, four:
  1. RMSNorm fused with the per-token int8 quantiser          (rt_act_rmsnorm_quantize)
  2. gate and up in one GEMV/GEMM launch on the shared int8 x (rt_plan_create_act)
  3. relu^2(gate) * up fused with the quantiser               (rt_act_relu2_mul_quantize)
  4. down on the int8 activations                             (rt_linear_act_f32)
Both give the same bits.  No call allocates device memory after the first forward at a
given token count (and, for one token, input buffer), so a forward can be captured in a
HIP graph.
"""
from __future__ import annotations

import numpy as np

from .transformer import RMSNorm, TernaryLinear


class TernaryFFNBlock:
    def __init__(self, d_model: int, d_ff: int, use_gpu: bool = True, eps: float = 1e-6, max_tokens: int = 64):
        self.d_model, self.d_ff, self.eps = d_model, d_ff, eps
        self.use_gpu = use_gpu
        self.max_tokens = max_tokens
        self.norm = RMSNorm(d_model, eps)
        self.gate_proj = TernaryLinear(d_model, d_ff, use_gpu)
        self.up_proj = TernaryLinear(d_model, d_ff, use_gpu)
        self.down_proj = TernaryLinear(d_ff, d_model, use_gpu)
        self.gpu = self.gate_proj.gpu
        self._state = {}   # token count -> (plan, g, u, y)
        self._acts = None
        self._norm_w_dev = None
        self._gu = None      # interleaved gate/up copy for the one-token path
        self._pair = None    # (input pointer, gate/up plan, down plan, y)
        self._xin = None     # forward()'s device copy of its input
        self.pair_ok = d_model % 64 == 0 and d_ff % 64 == 0 and d_ff <= 8192

    def load(self, norm_weight, gate, up, down):
        """gate/up/down: (rotor bytes [out, ceil(in/4)], scale) each."""
        self.norm.weight = np.asarray(norm_weight, dtype=np.float32)
        self.gate_proj.load_from_bitnet(*gate)
        self.up_proj.load_from_bitnet(*up)
        self.down_proj.load_from_bitnet(*down)
        self._state.clear()
        self._gu = self._pair = None
        if self.use_gpu:
            import torch

            self._norm_w_dev = torch.from_numpy(self.norm.weight.copy()).to(self.gpu.device)
            self._acts = (self.gpu.activations(self.max_tokens, self.d_model),
                          self.gpu.activations(self.max_tokens, self.d_ff))

    def _buffers(self, M):
        st = self._state.get(M)
        if st is None:
            import torch

            dev = self.gpu.device
            g = torch.empty((M, self.d_ff), dtype=torch.float32, device=dev)
            u = torch.empty((M, self.d_ff), dtype=torch.float32, device=dev)
            y = torch.empty((M, self.d_model), dtype=torch.float32, device=dev)
            act_h = self._acts[0]
            plan = self.gpu.plan_act([self.gate_proj.gpu_packed_weights, self.up_proj.gpu_packed_weights],
                                     [act_h, act_h], M, [g, u])
            st = self._state[M] = (plan, g, u, y)
        return st

    def _pair_plans(self, x):
        """One token: the gate/up pair plan and the down plan.  Plans hold the input
        pointer, so they are rebuilt when x is another buffer."""
        if self._pair is None or self._pair[0] != x.data_ptr():
            import torch

            from . import _hip

            hip, dev = self.gpu, self.gpu.device
            if self._gu is None:
                self._gu = hip.interleave_gate_up(self.gate_proj.gpu_packed_weights, self.up_proj.gpu_packed_weights)
            w_gu, scales = self._gu
            a = torch.empty(self.d_ff, dtype=torch.float32, device=dev)
            ssq = torch.empty(self.d_ff // 32, dtype=torch.float64, device=dev)
            y = torch.empty((1, self.d_model), dtype=torch.float32, device=dev)
            gu = hip.plan_gate_up(w_gu, scales, _hip.SRC_RMSNORM, x.reshape(-1), self._norm_w_dev, eps=self.eps,
                                  a=a, ssq=ssq)
            down = hip.plan_fused([self.down_proj.gpu_packed_weights], _hip.SRC_QUANT, a, ys=[y.reshape(-1)])
            self._pair = (x.data_ptr(), gu, down, y)
        return self._pair

    def launches(self, M: int) -> int:
        """Kernel launches of one forward over M tokens."""
        return 2 if M == 1 and self.pair_ok else 4

    def forward_device(self, x):
        """x: device tensor [M, d_model] fp32 -> device tensor [M, d_model] (reused buffer)."""
        M = x.shape[0]
        if M > self.max_tokens:
            raise ValueError(f"{M} tokens exceed max_tokens={self.max_tokens}")
        if M == 1 and self.pair_ok:
            if not x.is_contiguous():
                raise ValueError("x must be contiguous")
            _, gu, down, y = self._pair_plans(x)
            gu.run()
            down.run()
            return y
        plan, g, u, y = self._buffers(M)
        act_h, act_a = self._acts
        hip = self.gpu
        hip.act_rmsnorm_quantize(x, self._norm_w_dev, act_h, self.eps)
        act_h.tokens = M
        plan.gemv()
        hip.act_relu2_mul_quantize(g, u, act_a)
        hip.linear_act(self.down_proj.gpu_packed_weights, act_a, out=y)
        return y

    def forward(self, x):
        """x [..., d_model] (numpy or torch) -> same leading shape, d_model."""
        if self.use_gpu:
            import torch

            shape = tuple(x.shape)
            xt = x if isinstance(x, torch.Tensor) else torch.from_numpy(np.ascontiguousarray(x, np.float32))
            xt = xt.to(self.gpu.device, torch.float32).reshape(-1, self.d_model)
            if self._xin is None:
                self._xin = torch.empty((self.max_tokens, self.d_model), dtype=torch.float32, device=self.gpu.device)
            xin = self._xin[:xt.shape[0]]
            xin.copy_(xt)  # one input buffer, so the one-token plans are built once
            y = self.forward_device(xin).clone().reshape(shape)
            return y if isinstance(x, torch.Tensor) else y.cpu().numpy()
        h = self.norm.forward(np.asarray(x, np.float32))
        g = self.gate_proj.forward(h)
        u = self.up_proj.forward(h)
        a = np.maximum(g, 0) ** 2 * u
        return self.down_proj.forward(a.astype(np.float32))
