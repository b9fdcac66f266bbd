"""Build the native parts in-tree.

* ``libshared_amd_sampler.so``: the HIP kernels and the C ABI, for gfx950.
* ``js/sas_napi.node``: the N-API addon that exposes the C ABI to Node.
* ``libsas_probe.so``: measurement probes for bench.py (the streaming
  bound of the sampling kernels); the sampling library never loads it.

Run ``python -m shared_amd.build`` (or ``__graft_entry__.build()``).
"""
from __future__ import annotations

import os
import shutil
import subprocess
import sys

PKG = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(PKG)
CSRC = os.path.join(PKG, "csrc")
INCLUDE = os.path.join(ROOT, "include")
LIB = os.path.join(PKG, "libshared_amd_sampler.so")
NAPI = os.path.join(PKG, "js", "sas_napi.node")
PROBE = os.path.join(PKG, "libsas_probe.so")
HIP_SOURCES = ["capi.hip", "sample_kernel.hip", "verify_kernel.hip", "lmhead_kernel.hip"]
PROBE_SOURCES = ["probe_kernel.hip"]

# -ffp-contract=off: the double-precision tail must round like a JS engine.
# -packed-fp32-ops: packed FP32 instructions are kept out of the code.
HIPCC_FLAGS = [
    "--offload-arch=gfx950", "-O3", "-std=c++17", "-fPIC", "-shared",
    "-ffp-contract=off", "-fno-fast-math",
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    "-Wall", "-Wno-unused-command-line-argument",
]


def _hipcc() -> str:
    for cand in (os.environ.get("HIPCC"), "/opt/rocm/bin/hipcc", shutil.which("hipcc")):
        if cand and os.path.exists(cand):
            return cand
    raise RuntimeError("hipcc not found: the HIP library cannot be built")


def _run(cmd: list[str]) -> None:
    proc = subprocess.run(cmd, stdout=subprocess.PIPE, stderr=subprocess.STDOUT, text=True)
    out = "\n".join(l for l in proc.stdout.splitlines() if "packed-fp32-ops" not in l)
    if proc.returncode != 0:
        raise RuntimeError(f"build failed ({proc.returncode}): {' '.join(cmd)}\n{out}")


def build_hip(out: str = LIB, sources: list[str] = HIP_SOURCES) -> str:
    srcs = [os.path.join(CSRC, s) for s in sources]
    tmp = out + ".tmp"
    _run([_hipcc(), *HIPCC_FLAGS, "-I", INCLUDE, "-I", CSRC, *srcs, "-o", tmp])
    os.replace(tmp, out)
    return out


def build_napi(out: str = NAPI) -> str | None:
    """Build the Node addon; returns None when Node's headers are absent."""
    inc = "/usr/include/node"
    src = os.path.join(CSRC, "napi_addon.cc")
    if not os.path.exists(os.path.join(inc, "node_api.h")) or not os.path.exists(src):
        return None
    tmp = out + ".tmp"
    _run(["g++", "-O2", "-std=c++17", "-fPIC", "-shared", "-Wall", "-I", inc, "-I", INCLUDE,
          src, "-o", tmp, "-L", PKG, "-lshared_amd_sampler", "-Wl,-rpath,$ORIGIN/.."])
    os.replace(tmp, out)
    return out


def build_probe(out: str = PROBE) -> str:
    return build_hip(out, PROBE_SOURCES)


def build_all() -> None:
    build_hip()
    build_probe()
    build_napi()


if __name__ == "__main__":
    build_all()
    print("built", LIB, NAPI if os.path.exists(NAPI) else "(no node addon)", file=sys.stderr)
