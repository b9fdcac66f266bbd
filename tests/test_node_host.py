"""The Node host layer without a GPU: tests/node/host_cpu.js checks the mask
state, the parameter packer and the addon's host helpers against the
reference's behaviour and messages."""
import os
import shutil
import subprocess

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
ADDON = os.path.join(ROOT, "shared_amd", "js", "sas_napi.node")


@pytest.mark.skipif(shutil.which("node") is None, reason="node is not installed")
def test_node_host_cpu():
    if not os.path.exists(ADDON):
        pytest.fail("the N-API addon is not built (python -m shared_amd.build)")
    import torch
    if torch.cuda.is_available():
        pytest.skip("a HIP device is present: the no-device checks do not apply")
    proc = subprocess.run(["node", os.path.join(ROOT, "tests", "node", "host_cpu.js")], stdout=subprocess.PIPE,
                          stderr=subprocess.STDOUT, text=True, timeout=120)
    print(proc.stdout)
    assert proc.returncode == 0, proc.stdout[-3000:]
    assert proc.stdout.strip().endswith("all ok")


def test_addon_exports():
    if shutil.which("node") is None:
        pytest.skip("node is not installed")
    js = ("const a=require(process.argv[1]);"
          "console.log(Object.keys(a).sort().join(','))")
    out = subprocess.run(["node", "-e", js, ADDON], stdout=subprocess.PIPE, stderr=subprocess.STDOUT, text=True,
                         timeout=60)
    assert out.returncode == 0, out.stdout
    names = set(out.stdout.strip().split(","))
    for fn in ("create", "destroy", "reserve", "alloc", "free", "copy", "synchronize", "sample", "sampleAsync",
               "verify", "verifyAsync", "clampParams", "maskFromIds", "pcgUniform", "version"):
        assert fn in names, fn
