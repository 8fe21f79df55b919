"""p0pc0rn_amd - MI355X (gfx950) int4 quantized-matmul hot path of p0pc0rn.

The product is the C-ABI library libp0pc0rn_hip.so (include/p0pc0rn.h) and its Node host (p0pc0rn_amd/js). This
Python package holds the build driver (p0pc0rn_amd.build) and a ctypes mirror of the C ABI (p0pc0rn_amd.capi).
"""
__version__ = "0.1.0"
