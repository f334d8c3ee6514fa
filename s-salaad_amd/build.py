"""Build the gfx950 HIP library `ssalaad_amd/libssalaad_amd.so` in-tree.

Every source under csrc/ is compiled with hipcc for gfx950 only and linked into
one shared library exporting the C ABI declared in include/ssalaad_amd.h. The
library is linked against the HIP runtime that PyTorch ships, so a process that
imports torch first holds a single libamdhip64.

With --checked, the same sources are built with SSL_DEVICE_CHECKS=1 into
`ssalaad_amd/libssalaad_amd_checked.so`: the kernels re-check every index they
read from plans and records and report a bad one in the call's status word
(ssl_device_checks). Load it with SSALAAD_AMD_LIB=<its path>.

Usage: python s-salaad_amd/build.py [-v] [--checked]
"""

from __future__ import annotations

import os
import shutil
import subprocess
import sys
import time
from concurrent.futures import ThreadPoolExecutor
from pathlib import Path

HERE = Path(__file__).resolve().parent
CSRC = HERE / "csrc"
OUT = HERE / "ssalaad_amd" / "libssalaad_amd.so"
OUT_CHECKED = HERE / "ssalaad_amd" / "libssalaad_amd_checked.so"
BUILD_DIR = HERE / "_build"
ARCH = "gfx950"


def _hipcc() -> str:
    rocm = os.environ.get("ROCM_PATH", "/opt/rocm")
    for cand in (Path(rocm) / "bin" / "hipcc", shutil.which("hipcc")):
        if cand and Path(cand).exists():
            return str(cand)
    raise RuntimeError("hipcc not found; the HIP library cannot be built")


def _torch_lib() -> str | None:
    try:
        import importlib.util

        spec = importlib.util.find_spec("torch")
        if spec and spec.origin:
            lib = Path(spec.origin).parent / "lib"
            if (lib / "libamdhip64.so").exists():
                return str(lib)
    except Exception:
        pass
    return None


COMMON_FLAGS = [
    "-O3",
    "-std=c++17",
    f"--offload-arch={ARCH}",
    "-fPIC",
    "-mcode-object-version=5",
    # Packed-fp32 VALU instructions are kept out of every kernel.
    "-Xclang",
    "-target-feature",
    "-Xclang",
    "-packed-fp32-ops",
    # One-lane ticket atomics stay one-lane: the wave-aggregating atomic
    # rewrite broadcasts the result and so waits for it at once, stalling the
    # wave's first loads behind a device round trip.
    "-mllvm",
    "-amdgpu-atomic-optimizer-strategy=None",
    "-Wall",
    "-Wno-unused-function",
    "-I",
    str(HERE.parent / "include"),
]


def build(verbose: bool = False, jobs: int = 8, checked: bool = False) -> Path:
    hipcc = _hipcc()
    out = OUT_CHECKED if checked else OUT
    build_dir = BUILD_DIR / "checked" if checked else BUILD_DIR
    build_dir.mkdir(parents=True, exist_ok=True)
    flags = COMMON_FLAGS + (["-DSSL_DEVICE_CHECKS=1"] if checked else [])
    sources = sorted(CSRC.glob("*.hip")) + sorted(CSRC.glob("*.cpp"))
    if not sources:
        raise RuntimeError("no sources under csrc/")

    def compile_one(src: Path) -> Path:
        obj = build_dir / (src.name + ".o")
        cmd = [hipcc, *flags, "-c", str(src), "-o", str(obj)]
        if src.suffix == ".cpp":
            cmd[1:1] = ["-x", "hip"]
        t0 = time.time()
        res = subprocess.run(cmd, capture_output=True, text=True)
        # hipcc's host pass reports the device-only feature flag; drop that line.
        err = "\n".join(
            ln for ln in res.stderr.splitlines() if "packed-fp32-ops" not in ln
        )
        if res.returncode != 0:
            raise RuntimeError(f"hipcc failed for {src.name}:\n{err}")
        if verbose:
            print(f"[build] {src.name}: {time.time() - t0:.1f}s")
            if err.strip():
                print(err)
        return obj

    with ThreadPoolExecutor(max_workers=max(1, min(jobs, len(sources)))) as ex:
        objs = list(ex.map(compile_one, sources))

    tmp = out.with_name(out.name + ".tmp")
    link = [hipcc, f"--offload-arch={ARCH}", "-shared", "-fPIC", *map(str, objs), "-o", str(tmp)]
    tlib = _torch_lib()
    if tlib:
        link[1:1] = [f"-L{tlib}", f"-Wl,-rpath,{tlib}"]
    res = subprocess.run(link, capture_output=True, text=True)
    if res.returncode != 0:
        raise RuntimeError(f"link failed:\n{res.stderr}")
    os.replace(tmp, out)
    if verbose:
        print(f"[build] wrote {out}")
    return out


if __name__ == "__main__":
    build(verbose="-v" in sys.argv, checked="--checked" in sys.argv)
