"""det_amd: det's quantized-linear path (W4/W6/W8 x int8 GEMM, activation quantization) on MI355X.

The product is the C-ABI library det_amd/libdet_hip.so (declared in include/det_hip.h); `det_amd.ffi` binds it
with ctypes for Python callers (tests, bench).  There is no CPU fallback: importing the bindings without the
built library raises.
"""
