"""Build recipe for libmsda_hip.so (the HIP kernels + C ABI) for gfx950.

    python msda-triton_amd/build.py            # compile every source, link
    python msda-triton_amd/build.py --asm      # also write gfx950 ISA listings to _build/

Sources are compiled in parallel with hipcc into objects under
msda-triton_amd/_build/, then linked into
msda-triton_amd/msda_triton_amd/libmsda_hip.so, which the Python package
loads with ctypes.  Cross-compiling needs no GPU.
"""

from __future__ import annotations

import argparse
import os
import shutil
import subprocess
import sys
from concurrent.futures import ThreadPoolExecutor
from pathlib import Path

HERE = Path(__file__).resolve().parent
CSRC = HERE / "csrc"
BUILD = HERE / "_build"
OUT = HERE / "msda_triton_amd" / "libmsda_hip.so"
ARCH = "gfx950"

SOURCES = [
    "msda_capi.hip", "msda_forward.hip", "msda_backward.hip", "msda_backward_priv.hip",
    "msda_backward_owner.hip", "msda_backward_binned.hip", "msda_proj.hip",
]

# -packed-fp32-ops off: keep v_pk_{add,mul,fma}_f32 out of the device code.
DEVICE_FLAGS = [
    f"--offload-arch={ARCH}",
    "-O3",
    "-std=c++17",
    "-fPIC",
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    "-Wall",
    "-Wno-unused-function",
]


def hipcc() -> str:
    for cand in (os.environ.get("HIPCC"), "/opt/rocm/bin/hipcc", shutil.which("hipcc")):
        if cand and Path(cand).exists():
            return cand
    raise RuntimeError("hipcc not found (ROCm is required to build libmsda_hip.so)")


def _run(cmd: list[str]) -> None:
    res = subprocess.run(cmd, capture_output=True, text=True)
    # The host pass warns that it does not know the packed-fp32 feature; drop it.
    err = "\n".join(
        ln for ln in res.stderr.splitlines() if "packed-fp32-ops" not in ln
    ).strip()
    if res.returncode != 0:
        raise RuntimeError(f"command failed: {' '.join(cmd)}\n{err}")
    if err:
        print(err, file=sys.stderr)


def build(asm: bool = False, jobs: int | None = None) -> Path:
    cc = hipcc()
    BUILD.mkdir(exist_ok=True)
    objs = []
    cmds = []
    for src in SOURCES:
        obj = BUILD / (Path(src).stem + ".o")
        objs.append(obj)
        cmds.append([cc, *DEVICE_FLAGS, "-c", str(CSRC / src), "-o", str(obj)])
        if asm:
            cmds.append([cc, *DEVICE_FLAGS, "--cuda-device-only", "-S", str(CSRC / src),
                         "-o", str(BUILD / (Path(src).stem + f".{ARCH}.s"))])
    with ThreadPoolExecutor(max_workers=jobs or min(8, len(cmds))) as ex:
        list(ex.map(_run, cmds))
    tmp = OUT.with_suffix(".so.tmp")
    _run([cc, f"--offload-arch={ARCH}", "-shared", "-fPIC", *map(str, objs), "-o", str(tmp)])
    os.replace(tmp, OUT)
    return OUT


if __name__ == "__main__":
    ap = argparse.ArgumentParser(description=__doc__.splitlines()[0])
    ap.add_argument("--asm", action="store_true", help="also emit gfx950 ISA listings")
    ap.add_argument("-j", "--jobs", type=int, default=None)
    args = ap.parse_args()
    print(build(asm=args.asm, jobs=args.jobs))
