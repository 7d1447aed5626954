"""Build the in-tree native libraries of the pb_amd package.

* ``pb_amd/libpbmoe.so``       — the gfx950 HIP kernels + C ABI (include/pbmoe.h)
* ``pb_amd/libpbmoe_synth.so`` — host seeded generator (no HIP dependency)

hipcc cross-compiles gfx950 code objects without a GPU present.  All HIP code
is compiled with packed-fp32 instructions disabled.
"""
from __future__ import annotations

import os
import subprocess
import sys
from concurrent.futures import ThreadPoolExecutor

HERE = os.path.dirname(os.path.abspath(__file__))
CSRC = os.path.join(HERE, "csrc")
ROOT = os.path.dirname(HERE)
HIPCC = os.environ.get("HIPCC", "/opt/rocm/bin/hipcc")
ARCH = "gfx950"

HIP_SOURCES = ["pbmoe_kernels.hip", "pbmoe_decode.hip", "pbmoe_prefill.hip", "pbmoe_attn.hip",
               "pbmoe_abi.cpp", "pbmoe_pack.cpp"]
HIP_FLAGS = [
    f"--offload-arch={ARCH}", "-O3", "-std=c++17", "-fPIC", "-shared",
    "-fvisibility=hidden", "-Wall", "-Wno-unused-function",
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    f"-I{os.path.join(ROOT, 'include')}",
]


def _run(cmd: list[str]) -> None:
    proc = subprocess.run(cmd, stdout=subprocess.PIPE, stderr=subprocess.STDOUT, text=True)
    # hipcc's host pass warns that it does not know the packed-fp32 feature
    lines = [l for l in proc.stdout.splitlines() if "packed-fp32-ops" not in l]
    if lines:
        print("\n".join(lines), file=sys.stderr)
    if proc.returncode != 0:
        raise RuntimeError(f"build failed ({proc.returncode}): {' '.join(cmd)}")


def build_synth() -> str:
    out = os.path.join(HERE, "libpbmoe_synth.so")
    _run(["gcc", "-O3", "-mfma", "-std=c11", "-fPIC", "-shared", "-fopenmp", "-ffp-contract=off",
          "-Wall", "-o", out, os.path.join(CSRC, "synth_host.c"), "-lm"])
    return out


def build_hip() -> str:
    """Each source compiles to its own object (host code + gfx950 code
    object) in parallel; one link makes the shared library."""
    out = os.path.join(HERE, "libpbmoe.so")
    tmp = out + ".tmp"
    objdir = os.path.join(ROOT, "_build")
    os.makedirs(objdir, exist_ok=True)
    compile_flags = [f for f in HIP_FLAGS if f != "-shared"]
    jobs = []
    for s in HIP_SOURCES:
        obj = os.path.join(objdir, s.rsplit(".", 1)[0] + ".o")
        jobs.append(([HIPCC, *compile_flags, "-c", "-o", obj, os.path.join(CSRC, s)], obj))
    workers = max(1, min(len(jobs), os.cpu_count() or 1, 8))
    with ThreadPoolExecutor(workers) as pool:
        list(pool.map(lambda j: _run(j[0]), jobs))
    _run([HIPCC, f"--offload-arch={ARCH}", "-shared", "-fPIC", "-o", tmp, *[o for _, o in jobs]])
    os.replace(tmp, out)
    return out


def build_all() -> None:
    build_synth()
    build_hip()


if __name__ == "__main__":
    build_all()
