"""Builds ``libinfrared_amd.so`` (the gfx950 kernels + C ABI) in-tree with hipcc.

Run ``python -m infrared_amd.build`` (or ``__graft_entry__.build()``). Every
``csrc/*.hip`` / ``csrc/*.cpp`` file compiles to an object under ``_build/``
in parallel, then one shared library is linked next to this file, where the
loader in ``infrared_amd._lib`` looks for it.
"""

from __future__ import annotations

import concurrent.futures as cf
import glob
import os
import shutil
import subprocess
import sys

PKG_DIR = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(PKG_DIR)
CSRC = os.path.join(PKG_DIR, "csrc")
INCLUDE = os.path.join(ROOT, "include")
BUILD_DIR = os.path.join(PKG_DIR, "_build")
LIB_NAME = "libinfrared_amd.so"
LIB_PATH = os.path.join(PKG_DIR, LIB_NAME)
ARCH = "gfx950"

# -packed-fp32-ops: no v_pk_{add,mul,fma}_f32 in device code (fp32 math is
# scalar VALU or MFMA only).
DEVICE_FLAGS = ["-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops"]
COMMON_FLAGS = [
    "-O3",
    "-std=c++17",
    "-fPIC",
    f"--offload-arch={ARCH}",
    "-Wall",
    "-Wno-unused-function",
    "-Wno-unused-command-line-argument",
    f"-I{INCLUDE}",
    f"-I{CSRC}",
]


# Per-source extras. The prefill kernel's max reductions never see a NaN from
# its own arithmetic (masked scores are -inf), so fmaxf needs no NaN quieting.
# The planned decode's six leading scalar arguments (the plan and the offsets
# of its first reads) are preloaded into SGPRs; kernels whose first argument is
# an aggregate preload nothing. A code object built so starts with a 256-byte
# block that loads those arguments the ordinary way, for firmware that does
# not preload.
FILE_FLAGS = {
    "paged_prefill.hip": ["-fno-honor-nans"],
    "paged_decode_planned.hip": ["-mllvm", "-amdgpu-kernarg-preload-count=6"],
}


def hipcc() -> str:
    path = shutil.which("hipcc") or "/opt/rocm/bin/hipcc"
    if not os.path.exists(path):
        raise RuntimeError("hipcc not found: the ROCm toolchain is required to build infrared_amd")
    return path


def sources() -> list[str]:
    return sorted(glob.glob(os.path.join(CSRC, "*.hip")) + glob.glob(os.path.join(CSRC, "*.cpp")))


def _compile(src: str, extra: list[str]) -> str:
    obj = os.path.join(BUILD_DIR, os.path.basename(src) + ".o")
    own = FILE_FLAGS.get(os.path.basename(src), [])
    cmd = [hipcc(), "-x", "hip", *COMMON_FLAGS, *DEVICE_FLAGS, *own, *extra, "-c", src, "-o", obj]
    res = subprocess.run(cmd, capture_output=True, text=True)
    # hipcc's host pass does not know the device-only target feature; that
    # warning is expected and dropped, anything else is shown.
    noise = ("packed-fp32-ops", "is not a recognized feature for this target")
    msg = "\n".join(
        line for line in (res.stdout + res.stderr).splitlines() if not any(n in line for n in noise)
    ).strip()
    if res.returncode != 0:
        raise RuntimeError(f"hipcc failed for {os.path.basename(src)}:\n{msg}")
    if msg:
        print(msg, file=sys.stderr)
    return obj


def build(verbose: bool = False, extra_flags: list[str] | None = None) -> str:
    """Compiles every source and links the shared library; returns its path."""
    os.makedirs(BUILD_DIR, exist_ok=True)
    extra = list(extra_flags or [])
    srcs = sources()
    with cf.ThreadPoolExecutor(max_workers=min(8, len(srcs))) as ex:
        objs = list(ex.map(lambda s: _compile(s, extra), srcs))
    tmp = LIB_PATH + ".tmp"
    cmd = [hipcc(), "-shared", "-fPIC", f"--offload-arch={ARCH}", *objs, "-o", tmp]
    res = subprocess.run(cmd, capture_output=True, text=True)
    if res.returncode != 0:
        raise RuntimeError(f"link failed:\n{res.stdout}{res.stderr}")
    os.replace(tmp, LIB_PATH)
    if verbose:
        print(f"built {LIB_PATH} from {len(srcs)} sources")
    return LIB_PATH


if __name__ == "__main__":
    build(verbose=True)
