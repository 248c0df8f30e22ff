"""The drop-in boundary, on the CPU: ABI layout, exported symbols, loader
behaviour (reference src/plugin_loader.hpp) including its failure paths,
forced with fake plugins.  No GPU calls."""
import ctypes
import os
import re
import subprocess

import numpy as np
import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
INCLUDE = os.path.join(ROOT, "include")
FAKE_SRC = os.path.join(ROOT, "tests", "fake_plugins", "fake_plugin.c")
LAYOUT_SRC = os.path.join(ROOT, "tests", "fake_plugins", "abi_layout.c")
REF_INCLUDE = "/root/reference/include"


def _run(cmd, **kw):
    r = subprocess.run(cmd, capture_output=True, text=True, **kw)
    assert r.returncode == 0, f"{cmd}\n{r.stdout}\n{r.stderr}"
    return r.stdout


PLUGIN_HEADERS = ("lux_gpu_backend_abi.h", "lux_gpu_quant_backend.h")
CORE_HEADERS = ("lux_quant_core.h",)


def declared_symbols(headers=PLUGIN_HEADERS):
    """Functions the given public headers declare with default visibility."""
    syms = set()
    for h in headers:
        txt = open(os.path.join(INCLUDE, h)).read()
        syms |= set(re.findall(r'visibility\("default"\)\)\)\s+[\w ]+?\**\s*\**(\w+)\s*\(', txt))
    return syms


def test_headers_compile_and_layout_asserts_hold(tmp_path):
    for h in PLUGIN_HEADERS + CORE_HEADERS:
        src = tmp_path / "t.c"
        src.write_text(f'#include "{INCLUDE}/{h}"\nint main(void){{return 0;}}\n')
        _run(["gcc", "-std=c11", "-Wall", "-Werror", "-fsyntax-only", str(src)])
        _run(["g++", "-std=c++17", "-Wall", "-Werror", "-fsyntax-only", "-x", "c++", str(src)])


def _layout(tmp_path, ref: bool):
    exe = tmp_path / ("layout_ref" if ref else "layout")
    cmd = ["gcc", "-std=c11", "-O0", LAYOUT_SRC, "-o", str(exe)]
    if ref:
        cmd[1:1] = ["-DUSE_REF", f"-I{REF_INCLUDE}"]
    _run(cmd)
    return [int(v) for v in _run([str(exe)]).split()]


def test_abi_layout_matches_ctypes_mirror(tmp_path):
    from mlx_amd import abi
    got = _layout(tmp_path, ref=False)
    names = [f[0] for f in abi.BackendVtbl._fields_]
    assert len(names) == 61
    assert got[:61] == [getattr(abi.BackendVtbl, n).offset for n in names]
    assert got[61:] == [ctypes.sizeof(abi.BackendVtbl), ctypes.sizeof(abi.BackendDesc),
                        abi.BackendDesc.vtbl.offset, ctypes.sizeof(abi.DeviceInfo), abi.ABI_VERSION]


@pytest.mark.skipif(not os.path.isdir(REF_INCLUDE), reason="reference headers not mounted")
def test_abi_layout_identical_to_reference_header(tmp_path):
    """Same slot offsets, struct sizes and ABI version as the reference's
    include/lux/gpu/backend_plugin.h."""
    assert _layout(tmp_path, ref=False) == _layout(tmp_path, ref=True)


def test_plugin_exports_exactly_the_declared_symbols():
    import mlx_amd
    assert mlx_amd.plugin_built(), "run __graft_entry__.build() first"
    out = _run(["nm", "-D", "--defined-only", mlx_amd.PLUGIN_PATH])
    exported = {l.split()[-1] for l in out.splitlines() if " T " in l}
    declared = declared_symbols()
    assert declared == {"lux_gpu_backend_init", "lux_gpu_backend_quant_init", "lux_gpu_quantized_matmul_noalloc",
                        "lux_gpu_quantized_matmul_kernel_name"}
    assert declared <= exported
    # nothing else leaks from the plugin (hidden visibility)
    assert {s for s in exported if s.startswith("lux")} == declared
    # and the library loads; its symbols resolve through dlsym
    lib = ctypes.CDLL(mlx_amd.PLUGIN_PATH, mode=os.RTLD_NOW | os.RTLD_LOCAL)
    for s in declared:
        assert getattr(lib, s) is not None


def test_core_library_exports_exactly_the_declared_symbols():
    import mlx_amd
    assert os.path.exists(mlx_amd.CORE_PATH), "run __graft_entry__.build() first"
    out = _run(["nm", "-D", "--defined-only", mlx_amd.CORE_PATH])
    exported = {l.split()[-1] for l in out.splitlines() if " T " in l}
    declared = declared_symbols(CORE_HEADERS)
    assert len(declared) == 12 and "lux_tensor_quantized_matmul" in declared
    assert {s for s in exported if s.startswith("lux")} == declared
    lib = ctypes.CDLL(mlx_amd.CORE_PATH, mode=os.RTLD_NOW | os.RTLD_LOCAL)
    for s in declared:
        assert getattr(lib, s) is not None


def test_quant_extension_table_without_gpu():
    """The extension table is static: usable for introspection without a device."""
    import mlx_amd
    from mlx_amd import abi
    lib = ctypes.CDLL(mlx_amd.PLUGIN_PATH, mode=os.RTLD_NOW | os.RTLD_LOCAL)
    qinit = abi.QUANT_INIT_FN(("lux_gpu_backend_quant_init", lib))
    p = ctypes.POINTER(abi.QuantVtbl)()
    assert qinit(ctypes.byref(p))
    q = p.contents
    assert q.ext_version == abi.QUANT_EXT_VERSION
    assert q.struct_size == ctypes.sizeof(abi.QuantVtbl)
    # kernel selection is pure host logic
    assert q.select_kernel(1, 4096, 14336, 64, 4, abi.FLOAT16, abi.FLOAT16) == abi.KERNEL_GEMV
    assert q.select_kernel(2048, 4096, 4096, 64, 4, abi.BFLOAT16, abi.BFLOAT16) == abi.KERNEL_GEMM
    assert q.select_kernel(2048, 4096, 4096, 64, 4, abi.FLOAT32, abi.FLOAT32) == abi.KERNEL_GEMV
    # K not a multiple of 256, and f32 scales at group 32 with 8-bit codes
    # where the register-W GEMM does not apply (K % 1024 != 0), stay on the
    # GEMV; with K % 1024 == 0 that GEMM takes them
    assert q.select_kernel(2048, 4160, 4096, 64, 4, abi.BFLOAT16, abi.BFLOAT16) == abi.KERNEL_GEMV
    assert q.select_kernel(2048, 4352, 4096, 32, 8, abi.BFLOAT16, abi.FLOAT32) == abi.KERNEL_GEMV
    assert q.select_kernel(2048, 4096, 4096, 32, 8, abi.BFLOAT16, abi.FLOAT32) == abi.KERNEL_GEMM
    assert q.select_kernel(2048, 4096, 4096, 32, 4, abi.BFLOAT16, abi.FLOAT32) == abi.KERNEL_GEMM
    # the GEMV/GEMM crossover: M = 16 for 4/8-bit codes with K % 1024 == 0
    # and 16-bit x (the GEMV's MFMA kernels), else M = 8
    if not os.environ.get("LUX_HIP_GEMV_MAX_M"):
        for bits in (4, 8):
            assert q.select_kernel(16, 4096, 14336, 64, bits, abi.FLOAT16, abi.FLOAT16) == abi.KERNEL_GEMV
            assert q.select_kernel(17, 4096, 14336, 64, bits, abi.FLOAT16, abi.FLOAT16) == abi.KERNEL_GEMM
        for bits in (3, 6):
            assert q.select_kernel(8, 4096, 11008, 64, bits, abi.FLOAT16, abi.FLOAT16) == abi.KERNEL_GEMV
            assert q.select_kernel(9, 4096, 11008, 64, bits, abi.FLOAT16, abi.FLOAT16) == abi.KERNEL_GEMM
        assert q.select_kernel(12, 3328, 4096, 64, 4, abi.BFLOAT16, abi.BFLOAT16) == abi.KERNEL_GEMM
    # NULL context / buffers are rejected before any device work
    assert q.op_quantized_matmul(None, None, None, None, None, None, 1, 64, 1, 64, 4, 1, 1, 1) == \
        abi.ERR_INVALID_ARGUMENT
    assert q.op_dequantize(None, None, None, None, None, 1, 64, 64, 4, 1, 1) == abi.ERR_INVALID_ARGUMENT


def _kernel_name_fn():
    import mlx_amd
    lib = ctypes.CDLL(mlx_amd.PLUGIN_PATH, mode=os.RTLD_NOW | os.RTLD_LOCAL)
    f = lib.lux_gpu_quantized_matmul_kernel_name
    f.restype = ctypes.c_char_p
    f.argtypes = [ctypes.c_int] * 9
    return lambda *shape, kernel=0: (lambda r: None if r is None else r.decode())(f(*shape, kernel))


@pytest.mark.skipif(bool(os.environ.get("LUX_HIP_GEMV_MAX_M") or os.environ.get("LUX_HIP_GEMM_RW")),
                    reason="selection overridden by the environment")
def test_auto_kernel_for_every_baseline_config():
    """The kernel AUTO launches for each BASELINE configuration (a dry run of
    the dispatch: host logic only), so a change of selection shows here."""
    from mlx_amd import abi
    name = _kernel_name_fn()
    F32, F16, BF16 = abi.FLOAT32, abi.FLOAT16, abi.BFLOAT16
    # (M, K, N, group, bits, x, scales/biases, out) -> kernel
    configs = {
        # c0: the CPU-backend GEMV case, all fp32
        (1, 4096, 4096, 64, 4, F32, F32, F32): "qgemv_line_kernel",
        # c1: decode, M = 1 / 4 / 8
        (1, 4096, 14336, 64, 4, F16, F16, F16): "qgemv_line_kernel",
        (4, 4096, 14336, 64, 4, F16, F16, F16): "qgemv_q4_kernel",
        (8, 4096, 14336, 64, 4, F16, F16, F16): "qgemv_q4_kernel",
        # c2: 8-bit, group 128, at the GEMV/GEMM crossover
        (32, 8192, 8192, 128, 8, BF16, BF16, BF16): "qgemm_small_kernel",
        # c3: prefill GEMM at both N
        (2048, 4096, 4096, 64, 4, BF16, BF16, BF16): "qgemm_rw_kernel",
        (2048, 4096, 14336, 64, 4, BF16, BF16, BF16): "qgemm_rw_kernel",
        # c4: 3- and 6-bit codes at M = 1 and 64
        (1, 4096, 11008, 64, 3, F16, F16, F16): "qgemv_line_kernel",
        (1, 4096, 11008, 64, 6, F16, F16, F16): "qgemv_line_kernel",
        (64, 4096, 11008, 64, 3, F16, F16, F16): "qgemm_small_kernel",
        (64, 4096, 11008, 64, 6, F16, F16, F16): "qgemm_small_kernel",
    }
    for shape, want in configs.items():
        assert name(*shape) == want, shape
    # GEMV and GEMM choices of the same configs
    assert name(1, 4096, 14336, 64, 4, F16, F16, F16, kernel=abi.KERNEL_GEMM) == "qgemm_kernel"
    assert name(2048, 4096, 4096, 64, 4, BF16, BF16, BF16, kernel=abi.KERNEL_GEMV) == "qgemv_stream_kernel"
    # errors and empty shapes
    assert name(1, 100, 4096, 64, 4, F16, F16, F16) is None
    assert name(2048, 4096, 4096, 64, 4, F32, F32, F32, kernel=abi.KERNEL_GEMM) is None
    assert name(0, 4096, 4096, 64, 4, F16, F16, F16) == ""


@pytest.mark.skipif(bool(os.environ.get("LUX_HIP_GEMV_MAX_M") or os.environ.get("LUX_HIP_GEMM_RW")),
                    reason="selection overridden by the environment")
def test_every_kernel_family_is_chosen_somewhere():
    """Each kernel of the plugin is AUTO's choice for a class of shapes (none
    is dead code); one representative shape per kernel.  (The row-run GEMV,
    qgemv_kernel, was retired once no shape picked it.)"""
    from mlx_amd import abi
    name = _kernel_name_fn()
    F32, F16, BF16 = abi.FLOAT32, abi.FLOAT16, abi.BFLOAT16
    families = {
        "qgemv_line_kernel": (1, 4096, 14336, 64, 4, F16),       # M = 1, K up to 16384
        "qgemv_split_kernel": (1, 14336, 4096, 64, 4, F16),      # M = 1 down projections, K > 8192
        "qgemv_stream_kernel": (2, 4096, 14336, 64, 3, F16),     # M = 2..8, 3/5/6-bit codes
        "qgemv_line_kernel#f32": (16, 4096, 11008, 64, 3, F32),   # f32 x, 3/5/6-bit codes: one row per launch
        "qgemv_mx_kernel": (4, 4096, 14336, 64, 8, F16),         # M = 2..4, 8-bit codes
        "qgemv_q4_kernel": (4, 4096, 14336, 64, 4, F16),         # M = 2..8, 4-bit codes, K = 4096
        "qgemv_dec_kernel": (6, 8192, 8192, 64, 4, F16),         # M = 5..8, 4-bit codes, K = 8192
        "qgemv_mid_kernel": (12, 4096, 14336, 64, 4, F16),       # M = 9..16, 4/8-bit codes
        "qmm_skinny_kernel": (6, 4096, 14336, 64, 8, F16),       # M = 5..8, 8-bit codes, K <= 4096
        "qgemm_small_kernel": (32, 8192, 8192, 128, 8, BF16),    # 8 < M <= 64
        "qgemm_sk_kernel": (32, 4096, 28672, 64, 4, BF16),       # 8 < M <= 64, wide N
        "qgemm_rw_kernel": (2048, 4096, 4096, 64, 4, BF16),      # M > 64, 4/8-bit, K % 1024 == 0
        "qgemm_kernel": (2048, 4096, 11008, 64, 3, BF16),        # M > 64, other widths or K
        "qmm_generic_kernel": (1, 96, 256, 32, 4, F16),          # K % 64 != 0
    }
    for want, (M, K, N, gs, bits, xd) in families.items():
        want = want.split("#")[0]
        assert name(M, K, N, gs, bits, xd, xd, xd) == want, (want, M, K, N, gs, bits, xd)


# ------------------------------------------------------------- loader ------

def _fake(tmp_path, name, *defs, subdir="p"):
    d = tmp_path / subdir
    d.mkdir(exist_ok=True)
    so = d / f"libluxgpu_backend_{name}.so"
    _run(["gcc", "-std=c11", "-shared", "-fPIC", f'-DFAKE_NAME="{name}"', *defs, FAKE_SRC,
          "-o", str(so)])
    return d, so


def test_loader_accepts_good_plugin_and_orders_paths(tmp_path):
    from mlx_amd.loader import PluginLoader
    d1, _ = _fake(tmp_path, "metal", subdir="a")
    env = {"LUX_GPU_BACKEND_PATH": f"/nonexistent:{d1}"}
    L = PluginLoader(env)
    # the last entry of the variable is searched first (reference :135-141)
    assert L.search_paths[0] == str(d1) and L.search_paths[1] == "/nonexistent"
    assert L.load_backend("metal")
    b = L.get_backend("metal")
    assert b.available and b.desc.abi_version == 2 and b.quant is None
    assert L.available_backends() == ["cpu", "metal"]
    assert L.get_best_backend() is b
    assert not L.load_backend("webgpu")


def test_loader_init_false_means_unavailable(tmp_path):
    from mlx_amd.loader import PluginLoader
    d, so = _fake(tmp_path, "cuda", "-DFAKE_INIT_FALSE")
    L = PluginLoader({"LUX_GPU_BACKEND_PATH": str(d)})
    assert not L.load_backend_from_path(str(so))
    assert L.get_backend("cuda") is None and L.available_backends() == ["cpu"]


def test_loader_rejects_abi_mismatch(tmp_path, capfd):
    from mlx_amd.loader import PluginLoader
    d, so = _fake(tmp_path, "webgpu", "-DFAKE_ABI=1")
    L = PluginLoader({"LUX_GPU_BACKEND_PATH": str(d)})
    assert not L.load_backend("webgpu")
    assert "has ABI version 1, expected 2" in capfd.readouterr().err
    assert L.backends == {}


def test_context_failure_is_reported(tmp_path):
    from mlx_amd import runtime
    from mlx_amd.loader import PluginLoader
    d, _ = _fake(tmp_path, "metal", "-DFAKE_NULL_CTX")
    L = PluginLoader({"LUX_GPU_BACKEND_PATH": str(d)})
    assert L.load_backend("metal")
    b = L.get_backend("metal")
    b.quant = object()  # the fake has no extension; only create_context matters here
    with pytest.raises(RuntimeError, match="create_context"):
        runtime.Context(0, backend=b)


def test_lux_backend_selection(tmp_path):
    from mlx_amd.loader import PluginLoader
    d, _ = _fake(tmp_path, "metal")
    _fake(tmp_path, "cuda")
    env = {"LUX_GPU_BACKEND_PATH": str(d)}
    assert PluginLoader(dict(env, LUX_BACKEND="cuda")).select().name == "cuda"
    assert PluginLoader(dict(env)).select().name == "metal"          # priority order
    assert PluginLoader(dict(env, LUX_BACKEND="cpu")).select() is None
    assert PluginLoader(dict(env, LUX_BACKEND="webgpu")).select() is None


def test_hip_plugin_without_gpu_reports_unavailable():
    """On a machine with no gfx950 device the plugin's init returns false, the
    loader registers it unavailable, and the runtime refuses to run (no CPU
    fallback)."""
    import torch  # noqa: F401  (only to know whether a GPU is visible)
    if torch.cuda.is_available():
        pytest.skip("a GPU is visible")
    from mlx_amd import runtime
    from mlx_amd.loader import PluginLoader
    L = PluginLoader({})
    assert not L.load_backend("hip")
    runtime._backend = None
    with pytest.raises(RuntimeError, match="unavailable"):
        runtime.get_backend("hip")


def test_reference_loader_loads_plugins(tmp_path):
    """The reference's own PluginLoader (compiled from its header into
    oracle/_ref) accepts a plugin built against this project's ABI header."""
    probe = os.path.join(ROOT, "oracle", "_ref", "ref_loader_probe")
    if not os.path.exists(probe):
        pytest.skip("oracle/_ref not built")
    import json
    d, _ = _fake(tmp_path, "metal")
    out = json.loads(_run([probe, "metal"], env=dict(os.environ, LUX_GPU_BACKEND_PATH=str(d))))
    assert out["loaded"] and out["available"] and out["abi_version"] == 2
    assert out["backend_name"] == "metal" and out["context"]
    d2, _ = _fake(tmp_path, "cuda", "-DFAKE_ABI=1", subdir="q")
    out = json.loads(_run([probe, "cuda"], env=dict(os.environ, LUX_GPU_BACKEND_PATH=str(d2))))
    assert not out["available"]
