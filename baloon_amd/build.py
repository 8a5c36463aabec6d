"""Build libixgdn.so (HIP, gfx950) in-tree with hipcc.

    python -m baloon_amd.build           # compile every csrc/*.hip and link the library

Each translation unit is compiled for gfx950 only, with packed-FP32 instruction selection
disabled (-packed-fp32-ops), and with kernel resource-usage remarks captured to
``_build/resource_usage.txt`` (one line per kernel: ``name=... VGPRs=.. AGPRs=.. ScratchSize=..
Occupancy=.. SGPRsSpill=.. VGPRsSpill=.. LDSSize=..``) so tests can assert that no hot kernel
spills to scratch and report SGPR spills, which land in VGPR lanes (v_writelane/v_readlane).
"""
from __future__ import annotations

import concurrent.futures as cf
import os
import re
import subprocess
import sys

PKG = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(PKG)
CSRC = os.path.join(PKG, "csrc")
INCLUDE = os.path.join(ROOT, "include")
BUILD = os.path.join(PKG, "_build")
LIB = os.path.join(PKG, "libixgdn.so")
RESOURCE_REPORT = os.path.join(BUILD, "resource_usage.txt")

HIPCC = os.environ.get("HIPCC", "/opt/rocm/bin/hipcc")
ARCH = "gfx950"
FLAGS = [
    f"--offload-arch={ARCH}", "-O3", "-std=c++17", "-fPIC", "-Wall",
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    "-I", INCLUDE, "-I", CSRC,
]


# Per-file additions. The decode kernels' atomics are single-lane group counters whose
# results are used only at the end of a workgroup; the atomic optimizer would expand each
# into a wave scan that broadcasts the result right away, waiting out the atomic's round
# trip (and every load in flight) in the middle of the state stream.
FILE_FLAGS = {
    "gdn_decode.hip": ["-mllvm", "-amdgpu-atomic-optimizer-strategy=None"],
}


def sources():
    return sorted(os.path.join(CSRC, f) for f in os.listdir(CSRC) if f.endswith(".hip"))


def _compile(src: str) -> tuple[str, str]:
    obj = os.path.join(BUILD, os.path.basename(src) + ".o")
    cmd = [HIPCC, *FLAGS, *FILE_FLAGS.get(os.path.basename(src), []), "-Rpass-analysis=kernel-resource-usage",
           "-c", src, "-o", obj]
    r = subprocess.run(cmd, capture_output=True, text=True)
    if r.returncode != 0:
        raise RuntimeError(f"hipcc failed for {src}:\n{r.stderr}")
    return obj, r.stderr


def _resource_summary(remarks: str) -> str:
    """Condense -Rpass-analysis=kernel-resource-usage remarks to one line per kernel."""
    lines, cur = [], None
    for ln in remarks.splitlines():
        m = re.search(r"remark:\s+(Function Name|VGPRs|AGPRs|ScratchSize \[bytes/lane\]|Occupancy \[waves/SIMD\]|"
                      r"VGPRs Spill|SGPRs Spill|LDS Size \[bytes/block\]):\s*(\S+)", ln)
        if not m:
            continue
        key, val = m.group(1), m.group(2)
        if key == "Function Name":
            cur = {"name": val}
            lines.append(cur)
        elif cur is not None:
            cur[key.split(" [")[0].replace(" ", "")] = val      # e.g. "SGPRs Spill" -> SGPRsSpill
    out = []
    for d in lines:
        out.append(" ".join(f"{k}={v}" for k, v in d.items()))
    return "\n".join(out) + "\n"


def build(verbose: bool = False) -> str:
    os.makedirs(BUILD, exist_ok=True)
    srcs = sources()
    with cf.ThreadPoolExecutor(max_workers=min(8, len(srcs))) as ex:
        results = list(ex.map(_compile, srcs))
    objs = [o for o, _ in results]
    remarks = "".join(r for _, r in results)
    with open(RESOURCE_REPORT, "w") as f:
        f.write(_resource_summary(remarks))
    tmp = LIB + ".tmp"
    r = subprocess.run([HIPCC, f"--offload-arch={ARCH}", "-shared", "-fPIC", "-o", tmp, *objs],
                       capture_output=True, text=True)
    if r.returncode != 0:
        raise RuntimeError(f"link failed:\n{r.stderr}")
    os.replace(tmp, LIB)
    if verbose:
        print(open(RESOURCE_REPORT).read(), end="")
        print(f"built {LIB}")
    return LIB


if __name__ == "__main__":
    build(verbose=True)
    sys.exit(0)
