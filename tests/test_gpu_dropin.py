"""The drop-in, end to end on the GPU: the REFERENCE's own plugin loader
(src/plugin_loader.hpp, compiled from its header into oracle/_ref by
oracle/Makefile) finds libluxgpu_backend_hip.so by name through
LUX_GPU_BACKEND_PATH, checks its ABI, creates a context on the MI355X and --
through the additive quant table it looks up beside the init symbol -- runs
the reference's dense-matmul known answer [[1,2],[3,4]] x [[5,6],[7,8]] =
[[19,22],[43,50]] (test/test_core.cpp:95-117) as a 4-bit quantized matmul
with scale 1 and bias 0."""
import json
import os
import subprocess

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))


@pytest.mark.gpu
def test_reference_loader_runs_the_hip_plugin():
    import mlx_amd
    probe = os.path.join(ROOT, "oracle", "_ref", "ref_loader_probe")
    if not os.path.exists(probe):
        pytest.skip("oracle/_ref not built (the reference sources were absent when it was built)")
    assert os.path.exists(mlx_amd.PLUGIN_PATH), "plugin not built"
    env = dict(os.environ, LUX_GPU_BACKEND_PATH=os.path.dirname(mlx_amd.PLUGIN_PATH))
    print(f"[case] reference loader probe: hip from {env['LUX_GPU_BACKEND_PATH']}", flush=True)
    r = subprocess.run([probe, "hip"], env=env, capture_output=True, text=True, timeout=120)
    assert r.returncode == 0, r.stderr
    out = json.loads(r.stdout.strip().splitlines()[-1])
    print(out)
    assert out["loaded"] and out["available"]
    assert out["abi_version"] == 2 and out["backend_name"] == "hip"
    assert out["context"]
    assert out["qmm_rc"] == 0 and out["copy_rc"] == 0
    assert out["y"] == [19, 22, 43, 50]
