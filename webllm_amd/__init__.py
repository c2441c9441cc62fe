"""webllm_amd: MI355X-native GPTQ int4 quantized linears (the hot path of intplusplus/webllm).

The GPU work lives in libqlinear.so (webllm_amd/csrc, C ABI in include/qlinear.h); this package
is the Python host side of that ABI. Nothing here computes on the CPU in place of the library.
"""
from . import qlinear  # noqa: F401

__all__ = ["qlinear"]
