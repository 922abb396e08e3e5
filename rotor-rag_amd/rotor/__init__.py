"""rotor - MI355X-native ternary linear path with the rotor-RAG Python surface.

Modules mirror the reference package ``src/rotor`` for the hot path only:
``transformer`` (TernaryLinear, RMSNorm), ``gpu_layers`` (get_gpu), ``gpu_ternary``
(the HIP backend over the ctypes C ABI in ``_hip``) and ``format`` (rotor bytes).
"""
__version__ = "0.1.0"
