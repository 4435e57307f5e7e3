"""Build libnovaq.so in-tree for gfx950 with hipcc.

Run ``python -m novann_amd._build`` (or call :func:`build`).  Every call
recompiles all sources; objects go to ``novann_amd/_build/`` and the shared
library to ``novann_amd/libnovaq.so``.
"""
from __future__ import annotations

import concurrent.futures as cf
import json
import os
import re
import subprocess
import sys

PKG = os.path.dirname(os.path.abspath(__file__))
CSRC = os.path.join(PKG, "csrc")
OBJ_DIR = os.path.join(PKG, "_build")
LIB = os.path.join(PKG, "libnovaq.so")
ARCH = "gfx950"

HIPCC = os.environ.get("HIPCC", "/opt/rocm/bin/hipcc")
# No fast-math and no flush-to-zero: the casts are bit-exact and rely on IEEE
# fp32 arithmetic with denormals.  Packed fp32 instructions are disabled.
HIP_FLAGS = [
    f"--offload-arch={ARCH}", "-O3", "-std=c++17", "-fPIC",
    "-fno-gpu-rdc", "-ffp-contract=off",
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    "-Wall", "-Wno-unused-function",
]


# The compiler's per-function resource remarks, kept beside the objects as
# kernel_resources.json: a test checks that no device function was outlined
# (a kernel's barrier inside a called function) and that nothing spills.
RESOURCE_FLAG = "-Rpass-analysis=kernel-resource-usage"
RESOURCES = os.path.join(OBJ_DIR, "kernel_resources.json")
_FIELDS = {"VGPRs": "vgprs", "AGPRs": "agprs", "ScratchSize [bytes/lane]": "scratch",
           "Occupancy [waves/SIMD]": "occupancy", "SGPRs Spill": "sgpr_spill",
           "VGPRs Spill": "vgpr_spill", "LDS Size [bytes/block]": "lds"}


def sources() -> list[str]:
    return sorted(os.path.join(CSRC, f) for f in os.listdir(CSRC) if f.endswith(".hip"))


def _resources(text: str) -> dict:
    """Function name -> resource fields, from the compiler's remarks."""
    res, cur = {}, None
    for line in text.splitlines():
        if "kernel-resource-usage" not in line or "remark:" not in line:
            continue
        body = line.split("remark:", 1)[1].replace("[-Rpass-analysis=kernel-resource-usage]", "")
        body = body.strip()
        if body.startswith("Function Name:"):
            cur = body.split(":", 1)[1].strip()
            res[cur] = {}
            continue
        m = re.match(r"(.+?):\s*(\d+)$", body)
        if cur and m and m.group(1) in _FIELDS:
            res[cur][_FIELDS[m.group(1)]] = int(m.group(2))
    return res


def _compile(src: str) -> tuple[str, dict]:
    obj = os.path.join(OBJ_DIR, os.path.basename(src)[:-4] + ".o")
    cmd = [HIPCC, *HIP_FLAGS, RESOURCE_FLAG, "-c", src, "-o", obj]
    r = subprocess.run(cmd, capture_output=True, text=True)
    text = r.stdout + r.stderr
    # drop the remarks (and the source excerpts they quote) and the host
    # pass's note about the device-only feature flag
    out = "\n".join(l for l in text.splitlines()
                    if "packed-fp32-ops" not in l and "kernel-resource-usage" not in l
                    and not l.startswith("In file included from")
                    and not re.match(r"^\s*(\d+ \||\|)", l))
    if r.returncode != 0:
        raise RuntimeError(f"hipcc failed for {src}:\n{out}")
    if out.strip():
        print(out, file=sys.stderr)
    return obj, _resources(text)


def build(verbose: bool = False) -> str:
    os.makedirs(OBJ_DIR, exist_ok=True)
    srcs = sources()
    with cf.ThreadPoolExecutor(max_workers=min(8, len(srcs))) as ex:
        done = list(ex.map(_compile, srcs))
    objs = [o for o, _ in done]
    res = {}
    for (_, r), src in zip(done, srcs):
        for name, fields in r.items():
            res[name] = dict(fields, source=os.path.basename(src))
    with open(RESOURCES, "w") as f:
        json.dump(res, f, indent=1, sort_keys=True)
    tmp = LIB + ".tmp"
    cmd = [HIPCC, f"--offload-arch={ARCH}", "-shared", "-fPIC", "-o", tmp, *objs]
    r = subprocess.run(cmd, capture_output=True, text=True)
    if r.returncode != 0:
        raise RuntimeError(f"link failed:\n{r.stdout}{r.stderr}")
    os.replace(tmp, LIB)
    if verbose:
        print(f"built {LIB}")
    return LIB


if __name__ == "__main__":
    build(verbose=True)
