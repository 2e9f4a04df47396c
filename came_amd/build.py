"""Build libcame8.so (HIP, gfx950) in-tree with hipcc.

    python -m came_amd.build          # or: import came_amd.build; came_amd.build.build()

Flags that matter for results:
  -ffp-contract=off                        no implicit fused multiply-adds; the kernels
                                           call fmaf exactly where torch's CPU kernels fuse
  -fhip-fp32-correctly-rounded-divide-sqrt IEEE division and square root
  -Xclang -target-feature -Xclang -packed-fp32-ops
                                           no packed fp32 instructions in device code
"""
from __future__ import annotations

import os
import shutil
import subprocess
import sys
from concurrent.futures import ThreadPoolExecutor

HERE = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(HERE)
CSRC = os.path.join(HERE, "csrc")
OUT_DIR = os.path.join(HERE, "lib")
OUT = os.path.join(OUT_DIR, "libcame8.so")
ARCH = os.environ.get("CAME8_OFFLOAD_ARCH", "gfx950")

HIPCC_FLAGS = [
    f"--offload-arch={ARCH}",
    "-O3",
    "-std=c++17",
    "-fPIC",
    "-ffp-contract=off",
    "-fhip-fp32-correctly-rounded-divide-sqrt",
    "-fno-gpu-flush-denormals-to-zero",
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    "-Wall",
    "-Wno-unused-function",
]

# translation units: the host code with the flat-pass kernels, and one per band-pass family
UNITS = [("came8", "came8.hip", [])] + [
    (f"band_{t.lower()}_p{p}", "came8_band.hip", [f"-DCAME8_BAND_TYPE={t}", f"-DCAME8_BAND_PASS={p}"])
    for t in ("F32", "BF16", "F16") for p in (1, 2)
]


def hipcc() -> str:
    for cand in (shutil.which("hipcc"), "/opt/rocm/bin/hipcc"):
        if cand and os.path.exists(cand):
            return cand
    raise RuntimeError("hipcc not found")


def _run(cmd: list[str]) -> tuple[int, str]:
    res = subprocess.run(cmd, capture_output=True, text=True)
    noise = "packed-fp32-ops"  # hipcc's host pass does not know the device feature
    return res.returncode, "\n".join(l for l in res.stderr.splitlines() if noise not in l)


def build(verbose: bool = True, jobs: int | None = None) -> str:
    """Compile the HIP sources under came_amd/csrc into came_amd/lib/libcame8.so (always recompiles).

    The translation units compile in parallel (``jobs`` processes, default: the CPU count, at most
    the number of units), then link into one shared library."""
    os.makedirs(OUT_DIR, exist_ok=True)
    cc = hipcc()
    inc = ["-I", os.path.join(ROOT, "include"), "-I", CSRC]
    objs, cmds = [], []
    for name, src, defs in UNITS:
        obj = os.path.join(OUT_DIR, f"{name}.o")
        objs.append(obj)
        cmds.append([cc, *HIPCC_FLAGS, *defs, *inc, "-c", "-o", obj, os.path.join(CSRC, src)])
    jobs = jobs or min(len(cmds), os.cpu_count() or 1)
    if verbose:
        print(f"[came_amd.build] {len(cmds)} units, {jobs} parallel: {' '.join(cmds[0])}", flush=True)
    with ThreadPoolExecutor(max_workers=jobs) as ex:
        results = list(ex.map(_run, cmds))
    for (name, _, _), (rc, errs) in zip(UNITS, results):
        if rc != 0:
            raise RuntimeError(f"hipcc failed on {name} ({rc}):\n{errs}")
        if verbose and errs.strip():
            print(errs, file=sys.stderr)
    tmp = OUT + ".tmp"
    rc, errs = _run([cc, f"--offload-arch={ARCH}", "-shared", "-fPIC", "-o", tmp, *objs])
    if rc != 0:
        raise RuntimeError(f"link failed ({rc}):\n{errs}")
    for o in objs:
        os.remove(o)
    os.replace(tmp, OUT)
    return OUT


if __name__ == "__main__":
    print(build())
