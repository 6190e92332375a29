"""Build libmoeoffload.so (all HIP kernels + the C ABI) for gfx950, in-tree.

    python drama3-offloading_amd/build.py [--jobs N] [--asm] [--asan-host]

Each csrc/*.hip is compiled to an object with hipcc, then linked into one
shared library next to this file.  The library links the HIP runtime by its
soname, so a process that has already imported torch resolves it to torch's
own runtime (one HIP runtime per process).  `--asm` also writes the gfx950
assembly of each source into _build/ for inspection.

`--asan-host` instead builds _build/asan/libmoeoffload.so with the host code
(the coded-pool encoder, every precondition path) under AddressSanitizer and
the device code as usual, for the CPU tests:

    MOE_OFFLOAD_LIB=drama3-offloading_amd/_build/asan/libmoeoffload.so \
    LD_PRELOAD=$(/opt/rocm/llvm/bin/clang -print-file-name=libclang_rt.asan-x86_64.so) \
    ASAN_OPTIONS=detect_leaks=0 python -m pytest tests -m "not gpu"

Every build also links libmoeoffload_marks.so: the same objects with
moe_gemv.hip compiled under MOE_PHASE_MARKS, whose decode GEMV launches
record per-wave phase marks (the bench's `--probe gemvphases` loads it in
place of the product library).
"""
from __future__ import annotations

import argparse
import concurrent.futures as cf
import os
import shutil
import subprocess
import sys
from pathlib import Path

HERE = Path(__file__).resolve().parent
CSRC = HERE / "csrc"
BUILD = HERE / "_build"
LIB = HERE / "libmoeoffload.so"
MARKS_LIB = HERE / "libmoeoffload_marks.so"
ARCH = "gfx950"

HIPCC = os.environ.get("HIPCC") or shutil.which("hipcc") or "/opt/rocm/bin/hipcc"

# -packed-fp32-ops: keep hipcc from emitting v_pk_{add,mul,fma}_f32, which
# have given silently wrong results on this hardware.  The host pass warns
# that it does not know the feature; that warning is harmless.
DEVICE_FLAGS = [
    f"--offload-arch={ARCH}", "-O3", "-std=c++17", "-fPIC",
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    "-Wall", "-Wno-unused-function",
]


def sources() -> list[Path]:
    return sorted(CSRC.glob("*.hip"))


def _run(cmd: list[str]) -> None:
    proc = subprocess.run(cmd, stdout=subprocess.PIPE, stderr=subprocess.STDOUT, text=True)
    out = "\n".join(l for l in proc.stdout.splitlines()
                    if "packed-fp32-ops' is not a recognized feature" not in l)
    if proc.returncode != 0:
        raise RuntimeError(f"command failed ({proc.returncode}): {' '.join(cmd)}\n{out}")
    if out.strip():
        print(out, file=sys.stderr)


# host-only AddressSanitizer: each -fsanitize= goes to the host pass alone
ASAN_HOST_FLAGS = ["-g", "-Xarch_host", "-fsanitize=address",
                   "-Xarch_host", "-fno-omit-frame-pointer"]


def compile_one(src: Path, asm: bool, out_dir: Path = BUILD, extra=()) -> Path:
    obj = out_dir / (src.stem + ".o")
    _run([HIPCC, *DEVICE_FLAGS, *extra, "-c", str(src), "-o", str(obj)])
    if asm:
        _run([HIPCC, *DEVICE_FLAGS, "--cuda-device-only", "-S", str(src),
              "-o", str(BUILD / (src.stem + ".s"))])
    return obj


def build(jobs: int = 8, asm: bool = False, asan_host: bool = False) -> Path:
    if not Path(HIPCC).exists() and shutil.which(HIPCC) is None:
        raise RuntimeError(f"hipcc not found ({HIPCC})")
    out_dir = BUILD / "asan" if asan_host else BUILD
    out_dir.mkdir(parents=True, exist_ok=True)
    lib = out_dir / LIB.name if asan_host else LIB
    extra = ASAN_HOST_FLAGS if asan_host else []
    srcs = sources()
    with cf.ThreadPoolExecutor(max_workers=max(1, jobs)) as ex:
        objs = list(ex.map(lambda s: compile_one(s, asm and not asan_host, out_dir, extra),
                           srcs))
    link_extra = ["-Xarch_host", "-fsanitize=address", "-Xarch_host", "-shared-libasan"] \
        if asan_host else []
    tmp = lib.with_suffix(".so.tmp")
    _run([HIPCC, f"--offload-arch={ARCH}", "-shared", "-fPIC", *link_extra, "-o", str(tmp),
          *map(str, objs), "-ldl"])
    os.replace(tmp, lib)
    if not asan_host:
        build_marks(objs)
    return lib


def build_marks(objs: list[Path]) -> Path:
    """libmoeoffload_marks.so: `objs` with moe_gemv's object rebuilt under
    MOE_PHASE_MARKS (the decode GEMV launches record phase marks)."""
    marks_dir = BUILD / "marks"
    marks_dir.mkdir(parents=True, exist_ok=True)
    marked = compile_one(CSRC / "moe_gemv.hip", False, marks_dir, ["-DMOE_PHASE_MARKS"])
    rest = [o for o in objs if o.name != marked.name]
    tmp = MARKS_LIB.with_suffix(".so.tmp")
    _run([HIPCC, f"--offload-arch={ARCH}", "-shared", "-fPIC", "-o", str(tmp),
          *map(str, rest), str(marked), "-ldl"])
    os.replace(tmp, MARKS_LIB)
    return MARKS_LIB


def main() -> None:
    ap = argparse.ArgumentParser()
    ap.add_argument("--jobs", type=int, default=min(8, os.cpu_count() or 1))
    ap.add_argument("--asm", action="store_true")
    ap.add_argument("--asan-host", action="store_true",
                    help="host code under AddressSanitizer, into _build/asan/")
    args = ap.parse_args()
    lib = build(args.jobs, args.asm, args.asan_host)
    print(lib)


if __name__ == "__main__":
    main()
