"""Build the HIP library ``lucid_amd/liblucid_amd.so`` for gfx950 (in-tree).

Usage: ``python -m lucid_amd.build``.  hipcc cross-compiles without a GPU.
"""
from __future__ import annotations

import os
import subprocess
import sys

HERE = os.path.dirname(os.path.abspath(__file__))
CSRC = os.path.join(HERE, "csrc")
ARCH = os.environ.get("LUCID_OFFLOAD_ARCH", "gfx950")

# Every HIP translation unit is compiled with packed-fp32 instructions disabled.  Host code
# gets hidden symbol visibility: each library exports only the extern "C" entry points its
# header declares, so two libraries loaded into one process (RTLD_GLOBAL included) never
# bind each other's internal helpers or their static state.
HIPCC_FLAGS = [
    f"--offload-arch={ARCH}", "-O3", "-std=c++17", "-shared", "-fPIC",
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    "-Xarch_host", "-fvisibility=hidden", "-Xarch_host", "-fvisibility-inlines-hidden",
]

TARGETS = {
    "liblucid_amd.so": ["lucid_capi.hip"],
    "liblucid_path.so": ["path_capi.hip"],
}


def build(verbose: bool = False) -> list[str]:
    hipcc = os.environ.get("HIPCC", "/opt/rocm/bin/hipcc")
    built = []
    for out, srcs in TARGETS.items():
        dst = os.path.join(HERE, out)
        tmp = dst + ".tmp"
        cmd = [hipcc, *HIPCC_FLAGS, "-o", tmp, *[os.path.join(CSRC, s) for s in srcs]]
        if verbose:
            print(" ".join(cmd), flush=True)
        res = subprocess.run(cmd, capture_output=True, text=True)
        if res.returncode != 0:
            raise RuntimeError(f"hipcc failed for {out}:\n{res.stderr}")
        os.replace(tmp, dst)
        built.append(dst)
    return built


if __name__ == "__main__":
    for p in build(verbose="-v" in sys.argv):
        print("built", p)
