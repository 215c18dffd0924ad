"""Build the gfx950 C-ABI library ``lib/libgdn_mi355x.so`` with hipcc.

Usage: ``python v100-attention-lab_amd/build.py`` (or ``build()`` from
Python).  The library is built in-tree so that it travels with the source
tree; nothing is installed.
"""

from __future__ import annotations

import os
import shutil
import subprocess
import sys
import time

PKG_DIR = os.path.dirname(os.path.abspath(__file__))
REPO_DIR = os.path.dirname(PKG_DIR)
CSRC = os.path.join(PKG_DIR, "csrc")
# One translation unit per q/k/v dtype, the host API, the input
# preparation and the backward, compiled in parallel.
SOURCES = ["gdn_fwd_api.hip", "gdn_fwd_f16.hip", "gdn_fwd_bf16.hip", "gdn_fwd_f32.hip",
           "gdn_fwd_c64.hip", "gdn_fwd_scan32.hip", "gdn_prep.hip", "gdn_bwd.hip"]
OBJ_DIR = os.path.join(PKG_DIR, "_build")
INCLUDE = os.path.join(REPO_DIR, "include")
LIB_DIR = os.path.join(PKG_DIR, "lib")
LIB_NAME = "libgdn_mi355x.so"
LIB_PATH = os.path.join(LIB_DIR, LIB_NAME)
# The same sources with -DGDN_PHASE_STAMPS: the 32-row scan and record kernels
# sum s_memtime windows of their MFMA phases (bench.py --phase-stamps reads
# them).  A measurement build only; the product never loads it.
STAMPS_LIB_PATH = os.path.join(LIB_DIR, "libgdn_mi355x_stamps.so")

ARCH = "gfx950"

HIPCC_FLAGS = [
    f"--offload-arch={ARCH}",
    "-O3",
    "-std=c++17",
    "-fPIC",
    # No packed-fp32 VALU (v_pk_*_f32) anywhere in device code.
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    "-Wno-unused-command-line-argument",
]


# Per-source flags.  The scan kernels keep their MFMA accumulators (the
# carried state) in arch VGPRs: with the AGPR form every iteration would copy
# the state through v_accvgpr_read / write on its serial path.
SOURCE_FLAGS = {
    "gdn_fwd_scan32.hip": ["-mllvm", "-amdgpu-mfma-vgpr-form"],
}


def hipcc() -> str:
    exe = shutil.which("hipcc") or "/opt/rocm/bin/hipcc"
    if not os.path.exists(exe):
        raise RuntimeError("hipcc not found; the ROCm toolchain is required to build")
    return exe


def _filtered(stderr: str) -> str:
    # hipcc's host pass does not know the packed-fp32 feature and says so;
    # that note is expected and filtered.
    noise = "is not a recognized feature for this target"
    return "\n".join(l for l in stderr.splitlines() if noise not in l)


def build(verbose: bool = True, extra_flags=None, phase_stamps: bool = False) -> str:
    """Compile the HIP sources into ``lib/libgdn_mi355x.so`` (or, with
    ``phase_stamps``, the measurement build ``lib/libgdn_mi355x_stamps.so``);
    returns its path."""
    obj_dir = OBJ_DIR + ("_stamps" if phase_stamps else "")
    lib_path = STAMPS_LIB_PATH if phase_stamps else LIB_PATH
    extra_flags = list(extra_flags or []) + (["-DGDN_PHASE_STAMPS"] if phase_stamps else [])
    os.makedirs(LIB_DIR, exist_ok=True)
    os.makedirs(obj_dir, exist_ok=True)
    t0 = time.time()
    procs = []
    objs = []
    for src in SOURCES:
        obj = os.path.join(obj_dir, os.path.splitext(src)[0] + ".o")
        cmd = [hipcc(), *HIPCC_FLAGS, *SOURCE_FLAGS.get(src, []), *(extra_flags or []),
               f"-I{INCLUDE}", "-c", os.path.join(CSRC, src), "-o", obj]
        if verbose:
            print("[build]", " ".join(cmd), flush=True)
        procs.append((src, subprocess.Popen(cmd, stdout=subprocess.PIPE, stderr=subprocess.PIPE,
                                            text=True)))
        objs.append(obj)
    failed = []
    for src, pr in procs:
        out, err = pr.communicate()
        err = _filtered(err)
        if pr.returncode != 0:
            failed.append(f"{src} ({pr.returncode}):\n{err}")
        elif verbose and err.strip():
            print(err, file=sys.stderr)
    if failed:
        raise RuntimeError("hipcc failed:\n" + "\n".join(failed))
    tmp = lib_path + ".tmp"
    link = [hipcc(), f"--offload-arch={ARCH}", "-shared", "-fPIC", *objs, "-o", tmp]
    res = subprocess.run(link, capture_output=True, text=True)
    if res.returncode != 0:
        raise RuntimeError(f"link failed ({res.returncode}):\n{_filtered(res.stderr)}")
    os.replace(tmp, lib_path)
    if verbose:
        print(f"[build] {lib_path} ({time.time() - t0:.1f} s)", flush=True)
    return lib_path


if __name__ == "__main__":
    build(phase_stamps="--phase-stamps" in sys.argv[1:])
