"""mlx_amd: MI355X-native (gfx950) backend plugin for Lux GPU Core's
group-wise affine quantized matmul.

The product is the shared library mlx_amd/lib/libluxgpu_backend_hip.so (HIP
kernels + the plugin C ABI).  This package holds its sources (csrc/), the
build (build.py), and a Python mirror of the reference's plugin loader and
vtable calls (abi.py, loader.py, runtime.py).
"""
import os

PLUGIN_PATH = os.path.join(os.path.dirname(os.path.abspath(__file__)), "lib",
                           "libluxgpu_backend_hip.so")


def plugin_built() -> bool:
    return os.path.exists(PLUGIN_PATH)
