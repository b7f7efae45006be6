"""Build libprefixlm.so (gfx950) in-tree with hipcc.

One translation unit, csrc/prefixlm.hip, holds the kernels and the C ABI
declared in include/prefixlm.h. The library links the HIP runtime by its
soname (libamdhip64.so.7), so inside a PyTorch process it binds to the runtime
torch already loaded and shares its streams.
"""
from __future__ import annotations

import os
import shutil
import subprocess
import sys

PKG_DIR = os.path.dirname(os.path.abspath(__file__))
SRC_ROOT = os.path.dirname(PKG_DIR)                    # hrm-text_amd/
REPO_ROOT = os.path.dirname(SRC_ROOT)
CSRC = os.path.join(SRC_ROOT, "csrc")
INCLUDE = os.path.join(REPO_ROOT, "include")
LIB_NAME = "libprefixlm.so"
LIB_PATH = os.path.join(PKG_DIR, LIB_NAME)

HIP_FLAGS = [
    "--offload-arch=gfx950",
    "-O3",
    "-std=c++17",
    "-fPIC",
    "-shared",
    "-munsafe-fp-atomics",
    # no packed fp32 arithmetic in device code
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    "-Wno-unused-command-line-argument",
]


def hipcc() -> str:
    for cand in (os.environ.get("HIPCC"), "/opt/rocm/bin/hipcc", shutil.which("hipcc")):
        if cand and os.path.exists(cand):
            return cand
    raise RuntimeError("hipcc not found (looked at $HIPCC, /opt/rocm/bin/hipcc, PATH)")


def build(verbose: bool = False, extra_flags=()) -> str:
    """Compile csrc/prefixlm.hip into prefixlm/libprefixlm.so; returns the path."""
    src = os.path.join(CSRC, "prefixlm.hip")
    tmp = LIB_PATH + ".tmp"
    cmd = [hipcc(), *HIP_FLAGS, *extra_flags, f"-I{INCLUDE}", f"-I{CSRC}", src, "-o", tmp]
    if verbose:
        print(" ".join(cmd), file=sys.stderr)
    proc = subprocess.run(cmd, capture_output=True, text=True)
    # the host pass does not know the device-only target feature; drop that note
    err = "\n".join(l for l in proc.stderr.splitlines() if "not a recognized feature" not in l)
    if proc.returncode != 0:
        raise RuntimeError(f"hipcc failed ({proc.returncode}):\n{err}")
    if verbose and err.strip():
        print(err, file=sys.stderr)
    os.replace(tmp, LIB_PATH)
    return LIB_PATH


if __name__ == "__main__":
    print(build(verbose=True))
