"""Runs the C++ adapter's known-answer program (tests/cpp/test_layerops_hip.cpp,
built by `make -C mimir-framework_amd kat`) on the GPU: the reference's own
KATs through the drop-in C++ signatures."""
import os
import subprocess

import pytest

pytestmark = pytest.mark.gpu

REPO = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
KAT = os.path.join(REPO, "mimir-framework_amd", "lib", "test_layerops_hip")


def test_cpp_adapter_kats():
    assert os.path.exists(KAT), f"{KAT} not built (make -C mimir-framework_amd kat)"
    print("running", KAT, flush=True)
    p = subprocess.run([KAT], capture_output=True, text=True, timeout=100)
    assert p.returncode == 0, p.stdout + p.stderr


REF_PROG = os.path.join(REPO, "oracle", "_ref", "test_device_model_ref")


@pytest.mark.skipif(not os.path.exists(REF_PROG), reason="oracle/_ref/test_device_model_ref not built")
def test_device_model_on_the_reference_layer():
    """tests/cpp/test_device_model_ref.cpp: DeviceModel<Layer> on the
    reference's own Layer and Model, beside Model::forwardPassNamed /
    backwardPass, including Tests/test_runtime_residual_merge.cpp."""
    print("running", REF_PROG, flush=True)
    p = subprocess.run([REF_PROG], capture_output=True, text=True, timeout=100)
    assert p.returncode == 0, (p.stdout + p.stderr)[-4000:]
    assert "all checks passed" in p.stdout
