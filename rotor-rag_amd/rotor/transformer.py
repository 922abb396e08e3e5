"""Ternary layers with the reference's Python surface (src/rotor/transformer.py).

``TernaryLinear(in_features, out_features, use_gpu=False)``, ``.load_from_bitnet(
packed_weights, scale)`` and ``.forward(x)`` keep the reference's names, arguments,
shapes and return types (src/rotor/transformer.py:50,77,111).

With ``use_gpu=True`` the layer runs on MI355X through the HIP library: the rotor
bytes go to the device once at load time and ``forward`` is one W2A8 launch
(per-token int8 activations, exact int32 accumulation, fp32 output) for the whole
[batch*seq, K] input.  If the HIP backend cannot be created, or a call fails, the
layer raises -- it never falls back to the CPU (the reference does so silently,
src/rotor/transformer.py:74-75,145-147).

With ``use_gpu=False`` it computes the reference's CPU formula
``np.dot(x, W_i8.T) * scale`` (src/rotor/transformer.py:150) on fp32 x.
"""
from __future__ import annotations

import numpy as np

from .format import rotor_rows_to_planes, unpack_rotor_rows


class RMSNorm:
    """x / sqrt(mean(x^2) + eps) * weight (src/rotor/transformer.py:17-36)."""

    def __init__(self, dim: int, eps: float = 1e-6):
        self.eps = eps
        self.weight = np.ones(dim, dtype=np.float32)

    def forward(self, x: np.ndarray) -> np.ndarray:
        norm = np.sqrt(np.mean(x ** 2, axis=-1, keepdims=True) + self.eps)
        return (x / norm) * self.weight


class TernaryLinear:
    """Linear layer with ternary weights in the rotor format (src/rotor/transformer.py:39-171)."""

    def __init__(self, in_features: int, out_features: int, use_gpu: bool = False):
        self.in_features = in_features
        self.out_features = out_features
        self.use_gpu = use_gpu
        self.scale = 1.0
        self.weight_shape = (out_features, in_features)
        self._packed = None          # rotor bytes [out, ceil(in/4)] (host)
        self._planes = None          # (bit0, bit1), built on first access
        self._weights_cache = None   # int8 [out, in], built on first access
        self.gpu = None
        self.gpu_packed_weights = None
        self.gpu_scales = None
        if use_gpu:
            from .gpu_layers import get_gpu, last_error

            self.gpu = get_gpu()
            if self.gpu is None:
                raise RuntimeError(f"TernaryLinear(use_gpu=True): HIP backend unavailable: {last_error()}")

    # Reference attributes, materialised lazily (the reference fills them eagerly at
    # load time, src/rotor/transformer.py:95-103; on the GPU path they are not needed).
    @property
    def bit0(self):
        return self._get_planes()[0]

    @property
    def bit1(self):
        return self._get_planes()[1]

    def _get_planes(self):
        if self._planes is None:
            if self._packed is None:
                n = (self.in_features * self.out_features + 7) // 8
                return np.zeros(n, np.uint8), np.zeros(n, np.uint8)
            b0, b1 = rotor_rows_to_planes(self._packed, self.in_features)
            self._planes = (b0.reshape(-1), b1.reshape(-1))
        return self._planes

    @property
    def weights_cache(self):
        if self._weights_cache is None and self._packed is not None:
            self._weights_cache = unpack_rotor_rows(self._packed, self.in_features)
        return self._weights_cache

    @weights_cache.setter
    def weights_cache(self, value):
        self._weights_cache = None if value is None else np.asarray(value, dtype=np.int8)

    def load_from_bitnet(self, packed_weights: np.ndarray, scale: float = 1.0):
        """Load rotor/BitNet bytes [out_features, ceil(in_features/4)] (uint8) and a
        per-tensor scale (src/rotor/transformer.py:77-109)."""
        p = np.ascontiguousarray(packed_weights, dtype=np.uint8)
        if p.ndim != 2 or p.shape[0] != self.out_features or p.shape[1] * 4 < self.in_features:
            raise ValueError(f"packed weights of shape {p.shape} do not fit "
                             f"[{self.out_features}, {(self.in_features + 3) // 4}]")
        p = np.ascontiguousarray(p[:, : (self.in_features + 3) // 4])
        self.scale = float(scale)
        self._packed = p
        self._planes = None
        self._weights_cache = None
        if self.gpu is not None and self.use_gpu:
            self.gpu_packed_weights = self.gpu.upload(p, self.in_features, self.scale)
            self.gpu_scales = np.full(self.out_features, self.scale, dtype=np.float32)

    def forward(self, x):
        """y = x @ W.T * scale for x [batch, seq, in] or [seq, in] (src/rotor/transformer.py:111-155).

        GPU mode also accepts a torch tensor (on the GPU or not) and then returns a
        device tensor; numpy in gives numpy out.
        """
        shape = tuple(x.shape)
        if shape[-1] != self.in_features:
            raise ValueError(f"input has {shape[-1]} features, layer expects {self.in_features}")
        x2 = x.reshape(-1, self.in_features)
        if self.use_gpu:
            if self.gpu_packed_weights is None:
                raise RuntimeError("TernaryLinear: weights not loaded")
            y = self.gpu.linear(self.gpu_packed_weights, x2)
        else:
            y = np.dot(x2, self.weights_cache.T) * self.scale
        return y.reshape(shape[:-1] + (self.out_features,))

    __call__ = forward
