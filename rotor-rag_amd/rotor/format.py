"""Host-side handling of the rotor 2-bit weight format (product code).

Code: value = bit0 - bit1; a 2-bit field f = 2*bit0 + bit1 per element, element j of
a byte in bits (2j+1, 2j): 00 -> 0, 10 -> +1, 01 -> -1, 11 -> 0 (reserved).
Layout per src/rotor/core.py:75-110; decode rule per native/c/rotor_core.c:240-256.
Matrices are row-major [N][ceil(K/4)] bytes, rows packed independently, which is the
shape of the BitNet tensors handed to TernaryLinear.load_from_bitnet
(src/rotor/transformer.py:77-92).
"""
from __future__ import annotations

import numpy as np


def pack_rotor_rows(W) -> np.ndarray:
    """Ternary W [N, K] (any int/float dtype holding -1/0/+1) -> rotor bytes [N, ceil(K/4)]."""
    W = np.asarray(W)
    if W.ndim != 2:
        raise ValueError(f"expected a 2-D weight matrix, got shape {W.shape}")
    N, K = W.shape
    Kp = (K + 3) // 4 * 4
    f = np.zeros((N, Kp), dtype=np.uint8)
    f[:, :K] = np.where(W > 0, 2, np.where(W < 0, 1, 0)).astype(np.uint8)
    f = f.reshape(N, Kp // 4, 4)
    return (f[..., 0] | (f[..., 1] << 2) | (f[..., 2] << 4) | (f[..., 3] << 6)).astype(np.uint8)


def unpack_rotor_rows(packed, K: int) -> np.ndarray:
    """Rotor bytes [N, Kb] -> int8 [N, K]."""
    p = np.asarray(packed, dtype=np.uint8)
    N, Kb = p.shape
    if K > 4 * Kb:
        raise ValueError(f"K={K} exceeds the {4 * Kb} elements held by {Kb} bytes per row")
    out = np.empty((N, Kb, 4), dtype=np.int8)
    for j in range(4):
        f = (p >> (2 * j)) & 3
        out[..., j] = (f >> 1).astype(np.int8) - (f & 1).astype(np.int8)
    return np.ascontiguousarray(out.reshape(N, Kb * 4)[:, :K])


def rotor_rows_to_planes(packed, K: int):
    """Rotor bytes [N, Kb] -> LSB-first bit planes (bit0, bit1) [N, ceil(K/8)], the
    storage of the reference TernaryLinear (src/rotor/transformer.py:55-58,92-96)."""
    w = unpack_rotor_rows(packed, K)
    b0 = np.packbits((w == 1).astype(np.uint8), axis=1, bitorder="little")
    b1 = np.packbits((w == -1).astype(np.uint8), axis=1, bitorder="little")
    return b0, b1
