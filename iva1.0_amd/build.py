"""Builds libivakv.so (the gfx950 HIP kernels behind the C ABI in include/ivakv.h).

One hipcc invocation compiles every ``csrc/*.hip`` translation unit for gfx950
and links them into ``libivakv.so`` next to this file.  The library is written
to a temporary name first and renamed, so a concurrent reader never maps a
half-written file.
"""
from __future__ import annotations

import os
import shutil
import subprocess
from pathlib import Path

PKG_DIR = Path(__file__).resolve().parent
REPO_ROOT = PKG_DIR.parent
CSRC = PKG_DIR / "csrc"
INCLUDE = REPO_ROOT / "include"
LIB_NAME = "libivakv.so"
LIB_PATH = PKG_DIR / LIB_NAME
OFFLOAD_ARCH = "gfx950"

# Packed-FP32 VALU ops (v_pk_fma_f32 and friends) are disabled for device code;
# the host pass prints a harmless "not a recognized feature" warning for it.
DEVICE_FLAGS = ["-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops"]


def hipcc_path() -> str:
    for cand in (os.environ.get("HIPCC"), shutil.which("hipcc"), "/opt/rocm/bin/hipcc"):
        if cand and Path(cand).exists():
            return cand
    raise RuntimeError("hipcc not found: set HIPCC or install ROCm")


def sources() -> list[Path]:
    return sorted(CSRC.glob("*.hip"))


CEILING_SRC = PKG_DIR / "bench_kernels" / "ivakv_ceiling.hip"
CEILING_LIB = PKG_DIR / "libivakv_ceiling.so"


def build(verbose: bool = False) -> Path:
    """Compiles all HIP sources into ``libivakv.so`` (and the read-ceiling kernels of
    ``bench.py --workload ceiling`` into ``libivakv_ceiling.so``); returns the main path."""
    srcs = sources()
    if not srcs:
        raise RuntimeError(f"no HIP sources under {CSRC}")
    _compile(srcs, LIB_PATH, verbose)
    _compile([CEILING_SRC], CEILING_LIB, verbose)
    return LIB_PATH


def _compile(srcs, lib_path: Path, verbose: bool) -> None:
    tmp = lib_path.with_name(lib_path.name + f".tmp{os.getpid()}")
    cmd = [
        hipcc_path(),
        f"--offload-arch={OFFLOAD_ARCH}",
        "-O3",
        "-std=c++17",
        "-fPIC",
        "-shared",
        "-Wall",
        "-Wno-unused-command-line-argument",
        f"-I{INCLUDE}",
        f"-I{CSRC}",
        *DEVICE_FLAGS,
        "-o",
        str(tmp),
        *[str(s) for s in srcs],
    ]
    if verbose:
        print(" ".join(cmd), flush=True)
    proc = subprocess.run(cmd, capture_output=True, text=True)
    if proc.returncode != 0:
        tmp.unlink(missing_ok=True)
        raise RuntimeError(f"hipcc failed ({proc.returncode}):\n{proc.stdout}\n{proc.stderr}")
    os.replace(tmp, lib_path)


def kernel_resource_usage(srcs=None) -> dict:
    """Per-kernel register and scratch figures of every gfx950 kernel instantiation, from
    the compiler's ``-Rpass-analysis=kernel-resource-usage`` remarks (device-only
    compiles of each source, in parallel, into a temporary directory).  Returns
    ``{mangled kernel name: {"VGPRs", "AGPRs", "ScratchSize", "Occupancy"}}``."""
    import re
    import tempfile
    srcs = sources() if srcs is None else srcs
    keys = ("VGPRs", "AGPRs", "ScratchSize", "Occupancy")
    out: dict = {}
    with tempfile.TemporaryDirectory() as tmp:
        procs = []
        for i, src in enumerate(srcs):
            cmd = [hipcc_path(), f"--offload-arch={OFFLOAD_ARCH}", "-O3", "-std=c++17", "-c",
                   "--cuda-device-only", "-Rpass-analysis=kernel-resource-usage",
                   f"-I{INCLUDE}", f"-I{CSRC}", *DEVICE_FLAGS, "-o", str(Path(tmp) / f"{i}.o"),
                   str(src)]
            procs.append((src, subprocess.Popen(cmd, stdout=subprocess.PIPE,
                                                stderr=subprocess.PIPE, text=True)))
        for src, proc in procs:
            _, err = proc.communicate()
            if proc.returncode != 0:
                raise RuntimeError(f"hipcc failed on {src.name}:\n{err[-2000:]}")
            cur = None
            for line in err.splitlines():
                m = re.search(r"Function Name: (\S+)", line)
                if m:
                    cur = m.group(1)
                    out[cur] = {}
                    continue
                m = re.search(r"remark:\s+(\w+)(?: \[[^\]]*\])?: (\d+)", line)
                if m and cur and m.group(1) in keys:
                    out[cur][m.group(1)] = int(m.group(2))
    return out


if __name__ == "__main__":
    print(build(verbose=True))
