"""Build the gfx950 attention library and its Node.js N-API addon, in-tree.

    python supra2-img-web_amd/build.py          # both
    python supra2-img-web_amd/build.py lib      # libsupra_attn.so only

Outputs (git-ignored, shipped with the tree):
    supra2-img-web_amd/lib/libsupra_attn.so   HIP kernels + C ABI (include/supra_attn.h)
    supra2-img-web_amd/lib/supra_attn.node    N-API addon over the C ABI (rpath $ORIGIN)
"""

from __future__ import annotations

import os
import shutil
import subprocess
import sys

PKG = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(PKG)
CSRC = os.path.join(PKG, "csrc")
LIBDIR = os.path.join(PKG, "lib")
INCLUDE = os.path.join(ROOT, "include")
LIB = os.path.join(LIBDIR, "libsupra_attn.so")
ADDON = os.path.join(LIBDIR, "supra_attn.node")

HIP_SOURCES = ["api.hip", "flash_mfma.hip", "flash_small.hip", "flash_small16.hip", "wide_mfma.hip", "generic.hip", "linear_mfma.hip", "groupnorm.hip",
               "safetensors.hip", "weights.hip"]
ARCH = "gfx950"
# Packed FP32 instructions are kept out of the device code (they are emitted from plain float
# code at -O3 otherwise); the host pass warns that it does not know the feature.
# MFMA accumulators are kept in ordinary VGPRs: with the AGPR form the compiler copies the
# score and output tiles between register files around every softmax step.
HIP_FLAGS = [
    f"--offload-arch={ARCH}",
    "-O3",
    "-std=c++17",
    "-fPIC",
    "-Wall",
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    "-mllvm", "-amdgpu-mfma-vgpr-form",
]
NODE_INCLUDE = "/usr/include/node"


def _hipcc() -> str:
    for cand in (os.environ.get("HIPCC"), "/opt/rocm/bin/hipcc", shutil.which("hipcc")):
        if cand and os.path.exists(cand):
            return cand
    raise RuntimeError("hipcc not found (set HIPCC or install ROCm)")


def _run(cmd: list[str]) -> None:
    res = subprocess.run(cmd, stdout=subprocess.PIPE, stderr=subprocess.STDOUT, text=True)
    lines = [ln for ln in res.stdout.splitlines() if "packed-fp32-ops' is not a recognized feature" not in ln]
    if res.returncode != 0:
        raise RuntimeError("build failed (%d): %s\n%s" % (res.returncode, " ".join(cmd), "\n".join(lines)))
    if lines:
        sys.stderr.write("\n".join(lines) + "\n")


def build_lib() -> str:
    """Compiles each source to an object in parallel (one hipcc process per file), then links."""
    from concurrent.futures import ThreadPoolExecutor

    os.makedirs(LIBDIR, exist_ok=True)
    objdir = os.path.join(LIBDIR, "obj")
    os.makedirs(objdir, exist_ok=True)
    objs = [os.path.join(objdir, os.path.splitext(s)[0] + ".o") for s in HIP_SOURCES]
    jobs = max(1, min(len(HIP_SOURCES), int(os.environ.get("MAX_JOBS", os.cpu_count() or 4))))
    with ThreadPoolExecutor(max_workers=jobs) as ex:
        for f in [ex.submit(_run, [_hipcc(), *HIP_FLAGS, "-c", f"-I{INCLUDE}", os.path.join(CSRC, s), "-o", o])
                  for s, o in zip(HIP_SOURCES, objs)]:
            f.result()
    tmp = LIB + ".tmp"
    _run([_hipcc(), f"--offload-arch={ARCH}", "-fPIC", "-shared", *objs, "-o", tmp])
    os.replace(tmp, LIB)
    return LIB


def build_addon() -> str | None:
    """The N-API addon; skipped (returns None) when the Node headers are absent."""
    if not os.path.exists(os.path.join(NODE_INCLUDE, "node_api.h")):
        sys.stderr.write("node_api.h not found; N-API addon not built\n")
        return None
    os.makedirs(LIBDIR, exist_ok=True)
    tmp = ADDON + ".tmp"
    _run([
        "gcc", "-O2", "-std=c11", "-fPIC", "-shared", "-Wall", "-Wextra",
        f"-I{NODE_INCLUDE}", f"-I{INCLUDE}", "-DNAPI_VERSION=8", "-DNODE_GYP_MODULE_NAME=supra_attn",
        os.path.join(CSRC, "napi_addon.c"),
        f"-L{LIBDIR}", "-lsupra_attn", "-Wl,-rpath,$ORIGIN",
        "-o", tmp,
    ])
    os.replace(tmp, ADDON)
    return ADDON


def build(addon: bool = True) -> None:
    build_lib()
    if addon:
        build_addon()


if __name__ == "__main__":
    what = sys.argv[1] if len(sys.argv) > 1 else "all"
    if what == "lib":
        print(build_lib())
    elif what == "addon":
        print(build_addon())
    else:
        build()
        print(LIB)
        print(ADDON)
