"""Build libntlowbit.so (the gfx950 kernels and their C-ABI) in-tree.

Each csrc/*.hip file is compiled to an object in parallel with hipcc for
gfx950 only, then linked into nano-train_amd/lowbit/libntlowbit.so next to the
Python package that loads it.  Packed-FP32 instruction selection is disabled
for all device code (-Xclang -target-feature -Xclang -packed-fp32-ops).  The
compiler's per-kernel resource report (registers, scratch, occupancy) is kept
in _build/kernel_resources.json for the register checks in the tests.
"""

from __future__ import annotations

import concurrent.futures as cf
import json
import os
import re
import subprocess
import sys

HERE = os.path.dirname(os.path.abspath(__file__))
CSRC = os.path.join(HERE, "csrc")
OBJ_DIR = os.path.join(HERE, "_build")
RESOURCES = os.path.join(OBJ_DIR, "kernel_resources.json")
LIB = os.path.join(HERE, "lowbit", "libntlowbit.so")
HIPCC = os.environ.get("HIPCC", "/opt/rocm/bin/hipcc")
ARCH = "gfx950"

COMMON = [
    f"--offload-arch={ARCH}",
    "-O3",
    "-std=c++17",
    "-fPIC",
    "-Wall",
    "-Wno-unused-function",
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
]


def sources():
    return sorted(os.path.join(CSRC, f) for f in os.listdir(CSRC) if f.endswith(".hip"))


_REMARK = re.compile(r"remark: +(.+?): (\S+) \[-Rpass-analysis=kernel-resource-usage\]")


def _resources(stderr: str) -> dict:
    """{kernel: {field: value}} from the kernel-resource-usage remarks."""
    out, cur = {}, None
    for line in stderr.splitlines():
        m = _REMARK.search(line)
        if not m:
            continue
        key, val = m.group(1).strip(), m.group(2)
        if key == "Function Name":
            cur = out.setdefault(val, {})
        elif cur is not None:
            cur[key] = int(val) if val.isdigit() else val
    return out


def _compile(src: str):
    obj = os.path.join(OBJ_DIR, os.path.basename(src) + ".o")
    cmd = [HIPCC, *COMMON, "-Rpass-analysis=kernel-resource-usage", "-c", src, "-o", obj]
    res = subprocess.run(cmd, capture_output=True, text=True)
    noise = ("packed-fp32-ops", "kernel-resource-usage")
    lines = res.stderr.splitlines()
    # a remark is followed by the source line and caret it points at
    keep, skip = [], 0
    for l in lines:
        if skip:
            skip -= 1
            continue
        if "kernel-resource-usage" in l:
            skip = 2 if "Function Name" in l else 0
            continue
        if any(n in l for n in noise) or not l.strip():
            continue
        keep.append(l)
    err = "\n".join(keep)
    if res.returncode != 0:
        raise RuntimeError(f"hipcc failed for {src}:\n{err}")
    if err:
        sys.stderr.write(err + "\n")
    return obj, _resources(res.stderr)


def build(verbose: bool = False) -> str:
    os.makedirs(OBJ_DIR, exist_ok=True)
    srcs = sources()
    with cf.ThreadPoolExecutor(max_workers=min(8, len(srcs))) as ex:
        done = list(ex.map(_compile, srcs))
    objs = [o for o, _ in done]
    resources = {}
    for _, r in done:
        resources.update(r)
    with open(RESOURCES, "w") as fh:
        json.dump(resources, fh, indent=0, sort_keys=True)
    tmp = LIB + ".tmp"
    cmd = [HIPCC, f"--offload-arch={ARCH}", "-shared", "-fPIC", "-o", tmp, *objs]
    subprocess.run(cmd, check=True)
    os.replace(tmp, LIB)
    if verbose:
        print(f"built {LIB}")
    return LIB


if __name__ == "__main__":
    build(verbose=True)
