"""Build recipe for libinfurnace_hip.so (gfx950 only).

``python -m infurnace_amd.build`` compiles every ``csrc/*.hip`` with hipcc for
gfx950 into ``_build/`` and links ``infurnace_amd/libinfurnace_hip.so`` in
place (git-ignored; it travels to the GPU box with the source tree).

Packed fp32 VALU forms are switched off for device code
(``-target-feature -packed-fp32-ops``); hipcc's host pass warns that it does
not know the feature, which is harmless.
"""
from __future__ import annotations

import concurrent.futures as cf
import glob
import os
import subprocess
import sys

PKG = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(PKG)
CSRC = os.path.join(PKG, "csrc")
BUILD_DIR = os.path.join(ROOT, "_build")
LIB_PATH = os.path.join(PKG, "libinfurnace_hip.so")
ARCH = "gfx950"

HIPCC = os.environ.get("HIPCC", "/opt/rocm/bin/hipcc")
DEVICE_FLAGS = [
    f"--offload-arch={ARCH}",
    "-O3",
    "-std=c++17",
    "-fPIC",
    "-Wall",
    "-Wno-unused-function",
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
]


# Per-source extras for the prefill kernel.  It rescales its fp32 accumulators with VALU work
# inside the key loop; with the accumulators in AGPRs the compiler copies all of them to VGPRs and
# back every iteration, so its MFMAs are selected in the VGPR form.  Its maxima run over scores
# that are never NaN for finite inputs (masked keys are -inf), so fmaxf needs no NaN-quieting of
# its operands.  The precondition -- finite queries and K/V -- is part of the documented interface
# (the header's layout notes); with a NaN or Inf among the inputs the prefill output is unspecified.
# The one-launch shared-prefix decode, which runs the prefill body on some of its workgroups, is in
# the same file and shares both.
FILE_FLAGS = {
    "paged_prefill_wide.hip": ["-mllvm", "-amdgpu-mfma-vgpr-form", "-fno-honor-nans"],
    # The whole-row decode kernel's first nine arguments (plan, pool, tables, query, sizes, grid) are
    # preloaded into scalar registers at dispatch, so its first loads (the step plan) do not wait
    # for the kernel-argument loads.
    "paged_decode_rows.hip": ["-mllvm", "-amdgpu-kernarg-preload-count=9"],
}


def _compile(src: str) -> str:
    obj = os.path.join(BUILD_DIR, os.path.basename(src) + ".o")
    extra = FILE_FLAGS.get(os.path.basename(src), [])
    cmd = [HIPCC, *DEVICE_FLAGS, *extra, "-c", src, "-o", obj]
    r = subprocess.run(cmd, capture_output=True, text=True)
    # the only accepted diagnostic noise is the host pass not knowing the gfx feature
    noise = "'-packed-fp32-ops' is not a recognized feature for this target (ignoring feature)"
    err = "\n".join(ln for ln in r.stderr.splitlines() if noise not in ln)
    if r.returncode != 0:
        raise RuntimeError(f"hipcc failed for {src}:\n{err}")
    if err.strip():
        sys.stderr.write(err + "\n")
    return obj


def sources() -> list[str]:
    return sorted(glob.glob(os.path.join(CSRC, "*.hip")))


def build(jobs: int = 8) -> str:
    """Compile all HIP sources for gfx950 and link the shared library; returns its path."""
    os.makedirs(BUILD_DIR, exist_ok=True)
    srcs = sources()
    with cf.ThreadPoolExecutor(max_workers=max(1, min(jobs, len(srcs)))) as ex:
        objs = list(ex.map(_compile, srcs))
    tmp = LIB_PATH + ".tmp"
    cmd = [HIPCC, f"--offload-arch={ARCH}", "-shared", "-fPIC", "-o", tmp, *objs]
    subprocess.run(cmd, check=True)
    # A kernel whose host-side launch stub was not emitted links as an undefined symbol and only fails
    # when the library is loaded; refuse such a library here.
    nm = subprocess.run(["nm", "-u", tmp], capture_output=True, text=True)
    missing = [ln.split()[-1] for ln in nm.stdout.splitlines() if "_ZN3ifn" in ln]
    if missing:
        os.remove(tmp)
        raise RuntimeError(f"{len(missing)} undefined library symbols, e.g. {missing[0]}")
    os.replace(tmp, LIB_PATH)
    return LIB_PATH


if __name__ == "__main__":
    print(build())
