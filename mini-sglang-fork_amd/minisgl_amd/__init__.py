"""MI355X-native W8A8 int8 linear + fused-MoE path for mini-sglang.

Drop-in layer classes (``layers``), an MoE backend plugin (``moe``) and the
HIP kernels behind them (``kernel``, a ctypes binding of libmw8.so).
"""

__version__ = "0.1.0"
