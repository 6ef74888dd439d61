"""The JavaScript host (elffuss-engine_amd/js) on the CPU: runs tests/js/shim_cpu.js
under node (no device calls)."""
import os
import shutil
import subprocess

import pytest

HERE = os.path.dirname(os.path.abspath(__file__))


@pytest.mark.skipif(shutil.which("node") is None, reason="node is not installed")
def test_js_shim_cpu(eff):
    r = subprocess.run(["node", os.path.join(HERE, "js", "shim_cpu.js")], capture_output=True, text=True, timeout=120)
    assert r.returncode == 0, r.stdout + r.stderr
    assert "shim_cpu ok" in r.stdout


@pytest.mark.skipif(shutil.which("node") is None, reason="node is not installed")
def test_js_sampler_cpu(eff):
    """sample() against closed forms and its distributions; the candidate step
    against sample() over the whole vector (tests/js/shim_muestreo.js)."""
    r = subprocess.run(["node", os.path.join(HERE, "js", "shim_muestreo.js")], capture_output=True, text=True,
                       timeout=300)
    assert r.returncode == 0, r.stdout + r.stderr
    assert "shim_muestreo ok" in r.stdout
