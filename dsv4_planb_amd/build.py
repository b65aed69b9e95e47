"""Build ``libsas_hip.so`` (gfx950) in-tree with hipcc.

The library holds the HIP kernels, the C ABI of ``include/sas.h`` and the host
restatement of the reference metadata scheduler.  ``libsas_probe.so`` holds the
on-box peak probes the benchmark rates the kernels against.  The outputs land
next to this file so they travel with the source tree.
"""

from __future__ import annotations

import os
import shutil
import subprocess
import sys

HERE = os.path.dirname(os.path.abspath(__file__))
CSRC = os.path.join(HERE, "csrc")
LIB = os.path.join(HERE, "libsas_hip.so")
PROBE_LIB = os.path.join(HERE, "libsas_probe.so")  # on-box peak probes (benchmark only)
OBJ_DIR = os.path.join(HERE, "_build")

HIPCC = os.environ.get("HIPCC", "/opt/rocm/bin/hipcc")
ARCH = os.environ.get("SAS_OFFLOAD_ARCH", "gfx950")
# Packed FP32 instructions are disabled for all device code.
DEVICE_FLAGS = ["-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops"]
COMMON = ["-O3", "-std=c++17", "-fPIC", "-Wall", "-Wno-unused-function"]


def _run(cmd, verbose):
    if verbose:
        print(" ".join(cmd), flush=True)
    r = subprocess.run(cmd, capture_output=True, text=True)
    out = "\n".join(l for l in (r.stdout + r.stderr).splitlines()
                    if "packed-fp32-ops' is not a recognized feature" not in l)
    if r.returncode != 0:
        raise RuntimeError(f"build step failed ({r.returncode}): {' '.join(cmd)}\n{out}")
    if verbose and out.strip():
        print(out)


def build(verbose: bool = False) -> str:
    """Compile every source and link ``libsas_hip.so``; returns its path."""
    if shutil.which(HIPCC) is None and not os.path.exists(HIPCC):
        raise RuntimeError(f"hipcc not found at {HIPCC}")
    os.makedirs(OBJ_DIR, exist_ok=True)
    o_hip = os.path.join(OBJ_DIR, "sas_capi.o")
    o_meta = os.path.join(OBJ_DIR, "sas_metadata.o")
    _run([HIPCC, f"--offload-arch={ARCH}", *COMMON, *DEVICE_FLAGS, "-c",
          os.path.join(CSRC, "sas_capi.hip"), "-o", o_hip], verbose)
    _run(["g++", *COMMON, "-c", os.path.join(CSRC, "sas_metadata.cpp"), "-o", o_meta], verbose)
    tmp = LIB + ".tmp"
    _run([HIPCC, f"--offload-arch={ARCH}", "-shared", "-fPIC", o_hip, o_meta, "-o", tmp], verbose)
    os.replace(tmp, LIB)
    tmp = PROBE_LIB + ".tmp"
    _run([HIPCC, f"--offload-arch={ARCH}", *COMMON, *DEVICE_FLAGS, "-shared",
          os.path.join(CSRC, "sas_probe.hip"), "-o", tmp], verbose)
    os.replace(tmp, PROBE_LIB)
    return LIB


if __name__ == "__main__":
    print(build(verbose="-v" in sys.argv))
