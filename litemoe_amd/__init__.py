"""litemoe_amd: the MoE decode/prefill hot path of LiteMoE, MI355X (gfx950) native.

The host API mirrors LiteMoE's engine (``Granite.forward``, ``KVCache``,
``Engine.generate``, ``capture_decode``, ``OutputRing``); the compute is a
C-ABI library of hand-written HIP kernels (``include/litemoe_amd.h``),
loaded with ctypes by :mod:`litemoe_amd._lib`.
"""
__version__ = "0.1.0"
