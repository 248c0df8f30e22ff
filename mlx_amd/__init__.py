"""mlx_amd: MI355X-native (gfx950) backend plugin for Lux GPU Core's
group-wise affine quantized matmul.

The product is the shared library mlx_amd/lib/libluxgpu_backend_hip.so (HIP
kernels + the plugin C ABI), with the core-side selection library
mlx_amd/lib/libluxgpu_quant_core.so.  This package holds its sources (csrc/), the
build (build.py), and a Python mirror of the reference's plugin loader and
vtable calls (abi.py, loader.py, runtime.py).
"""
import os

PLUGIN_PATH = os.path.join(os.path.dirname(os.path.abspath(__file__)), "lib",
                           "libluxgpu_backend_hip.so")
# core-side selection and the public quantized op (include/lux_quant_core.h)
CORE_PATH = os.path.join(os.path.dirname(PLUGIN_PATH), "libluxgpu_quant_core.so")


def plugin_built() -> bool:
    return os.path.exists(PLUGIN_PATH)
