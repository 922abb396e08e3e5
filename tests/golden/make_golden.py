"""Write the golden fixtures of the rotor format from the reference's own C core.

Run in the build container (where /root/reference exists):
    make -C oracle            # compiles the reference's native/c/rotor_core.c -> oracle/_ref/
    python tests/golden/make_golden.py

Outputs (data only, committed):
  ref_core_vectors.npz  inputs and outputs of the reference C functions
                        bitnet_to_rotor, rotor_unpack_weights (native/c/rotor_core.c:202-299),
                        rotor_pack / rotor_unpack (:38-75) and rotor_encode / rotor_decode (:25-36)
  kats.json             known-answer vectors quoted from the reference's tests and docs
"""
from __future__ import annotations

import ctypes
import json
from pathlib import Path

import numpy as np

HERE = Path(__file__).resolve().parent
REF_LIB = HERE.parent.parent / "oracle" / "_ref" / "librotor_core.so"

# Known answers stated by the reference (file:line of the statement).
KATS = {
    "encode": {  # tests/test_core.py:23-30
        "values": [1, -1, 0, 1, -1, 0, 0, 1],
        "bit0": [1, 0, 0, 1, 0, 0, 0, 1],
        "bit1": [0, 1, 0, 0, 1, 0, 0, 0],
        "source": "tests/test_core.py:23-30",
    },
    "pack": {  # tests/test_core.py:90-98 packs these 8 values to 2 bytes; bytes from src/rotor/core.py:99-108
        "values": [1, -1, 0, 1, -1, 0, 1, 0],
        "packed": [0x86, 0x21],
        "source": "tests/test_core.py:90-98; src/rotor/core.py:99-108",
    },
    "bytes": [  # single bytes and their 4 decoded weights (LSB-first fields)
        {"byte": 0x24, "weights": [0, -1, 1, 0], "bit0": 0b0100, "bit1": 0b0010,
         "source": "src/rotor/bitnet.py:95,345-354 (0b00_10_01_00 -> [0,-1,+1,0])"},
        {"byte": 0x12, "weights": [1, 0, -1, 0],
         "source": "src/rotor/bitnet.py:172-176 (0b00_01_00_10 <-> [+1,0,-1,0]); tests/debug_bitnet_format.py:20-27"},
        {"byte": 0x86, "weights": [1, -1, 0, 1], "source": "tests/test_optimized_model.py:45-83 bytes, LSB-first reading"},
        {"byte": 0x68, "weights": [0, 1, 1, -1], "source": "tests/test_optimized_model.py:45-83 bytes, LSB-first reading"},
        {"byte": 0x81, "weights": [-1, 0, 0, 1], "source": "tests/test_optimized_model.py:45-83 bytes, LSB-first reading"},
        {"byte": 0x60, "weights": [0, 0, 1, -1], "source": "examples/test_fast_conversion.py:39-41 / src/rotor/bitnet_fast.py:179"},
        {"byte": 0x80, "weights": [0, 0, 0, 1], "source": "examples/test_fast_conversion.py:39-41 / src/rotor/bitnet_fast.py:179"},
    ],
    "quant": {  # closed form of src/rotor/quantization.py:137-149 on a row with max|x| = 127 (s = 1)
        "x": [127.0, 0.5, 1.5, 2.5, -0.5, -1.5, 3.49, -126.5],
        "q": [127, 0, 2, 2, 0, -2, 3, -126],
        "s": 1.0,
        "source": "src/rotor/quantization.py:137-149 (round half to even, clip [-128,127])",
    },
    "sign_matmul": {  # tests/test_core.py:132-159 (off-path sign-activation GEMV; kept for the C baseline)
        "W": [[1, -1, 0, 1], [0, 1, -1, 0], [1, 0, 1, -1]],
        "x": [0.5, -0.3, 0.8, -0.2],
        "y": [1, -2, 3],
        "source": "tests/test_core.py:132-159",
    },
}


def _u8(a):
    return a.ctypes.data_as(ctypes.POINTER(ctypes.c_uint8))


def main():
    lib = ctypes.CDLL(str(REF_LIB))
    sz = ctypes.c_size_t
    lib.bitnet_to_rotor.argtypes = [ctypes.c_void_p, sz, sz, ctypes.c_void_p, ctypes.c_void_p]
    lib.rotor_unpack_weights.argtypes = [ctypes.c_void_p, ctypes.c_void_p, sz, sz, ctypes.c_void_p]
    lib.rotor_pack.argtypes = [ctypes.c_void_p, ctypes.c_void_p, sz, ctypes.c_void_p]
    lib.rotor_unpack.argtypes = [ctypes.c_void_p, sz, ctypes.c_void_p, ctypes.c_void_p]
    lib.rotor_encode.argtypes = [ctypes.c_void_p, sz, ctypes.c_void_p, ctypes.c_void_p]
    for f in (lib.bitnet_to_rotor, lib.rotor_unpack_weights, lib.rotor_pack, lib.rotor_unpack, lib.rotor_encode):
        f.restype = None

    rng = np.random.default_rng(20251201)
    out = {}
    cases = {
        "all_bytes": (np.arange(256, dtype=np.uint8).reshape(1, 256), 1024),
        "ragged": (rng.integers(0, 256, size=(37, 13), dtype=np.uint8), 50),
        "square": (rng.integers(0, 256, size=(64, 160), dtype=np.uint8), 640),
    }
    for name, (src, cols) in cases.items():
        src = np.ascontiguousarray(src)
        rows = src.shape[0]
        ob = (cols + 7) // 8
        b0 = np.zeros((rows, ob), np.uint8)
        b1 = np.zeros((rows, ob), np.uint8)
        lib.bitnet_to_rotor(src.ctypes.data, rows, cols, b0.ctypes.data, b1.ctypes.data)
        w = np.zeros((rows, cols), np.int8)
        lib.rotor_unpack_weights(b0.ctypes.data, b1.ctypes.data, rows, cols, w.ctypes.data)
        out[f"{name}_src"] = src
        out[f"{name}_cols"] = np.array(cols)
        out[f"{name}_bit0"] = b0
        out[f"{name}_bit1"] = b1
        out[f"{name}_w"] = w

    vals = rng.choice(np.array([-1, 0, 1], np.int8), size=4000)
    e0 = np.zeros(4000, np.uint8)
    e1 = np.zeros(4000, np.uint8)
    lib.rotor_encode(vals.ctypes.data, 4000, e0.ctypes.data, e1.ctypes.data)
    packed = np.zeros(1000, np.uint8)
    lib.rotor_pack(e0.ctypes.data, e1.ctypes.data, 4000, packed.ctypes.data)
    u0 = np.zeros(4000, np.uint8)
    u1 = np.zeros(4000, np.uint8)
    lib.rotor_unpack(packed.ctypes.data, 4000, u0.ctypes.data, u1.ctypes.data)
    out.update(enc_values=vals, enc_bit0=e0, enc_bit1=e1, enc_packed=packed, unp_bit0=u0, unp_bit1=u1)

    np.savez_compressed(HERE / "ref_core_vectors.npz", **out)
    (HERE / "kats.json").write_text(json.dumps(KATS, indent=1) + "\n")
    print("wrote", HERE / "ref_core_vectors.npz", "and", HERE / "kats.json")


if __name__ == "__main__":
    main()
