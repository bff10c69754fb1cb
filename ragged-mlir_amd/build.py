"""Build libragged_hip.so (gfx950 kernels + C ABI) into the ragged package.

    python ragged-mlir_amd/build.py [--jobs N]

Each translation unit under csrc/ is compiled by hipcc for gfx950 in
parallel, then linked into ragged/libragged_hip.so. The sha256 of the sources
and the public header is embedded (rg_build_info) and written beside the
library as libragged_hip.so.sha256 so that artifacts record exactly which
build they bind to. Packed FP32 instructions are disabled for all device code.
"""
from __future__ import annotations

import argparse
from concurrent.futures import ThreadPoolExecutor
import hashlib
import os
from pathlib import Path
import shutil
import subprocess
import sys

ROOT = Path(__file__).resolve().parent
CSRC = ROOT / "csrc"
INCLUDE = ROOT.parent / "include"
BUILD = ROOT / "_build"
LIBRARY = ROOT / "ragged" / "libragged_hip.so"
UNITS = ("inst_softmax.hip", "inst_sum.hip", "inst_max.hip", "kernels_common.hip", "abi.hip")
ARCH = "gfx950"
FLAGS = ["-O3", "-std=c++17", "-fPIC", "-Wall", "-Wno-unused-function",
         "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops"]


def hipcc() -> str:
    for candidate in (os.environ.get("HIPCC"), shutil.which("hipcc"), "/opt/rocm/bin/hipcc"):
        if candidate and Path(candidate).exists():
            return candidate
    raise RuntimeError("hipcc not found; install ROCm or set HIPCC")


def source_digest() -> str:
    digest = hashlib.sha256()
    for path in sorted(CSRC.glob("*")) + sorted(INCLUDE.glob("*.h")):
        if path.is_file():
            digest.update(path.name.encode())
            digest.update(path.read_bytes())
    return digest.hexdigest()


def _run(command: list[str]) -> None:
    result = subprocess.run(command, capture_output=True, text=True)
    noise = ("packed-fp32-ops", "warning: unknown", "warnings generated")
    messages = [line for line in (result.stdout + result.stderr).splitlines()
                if line.strip() and not any(n in line for n in noise)]
    if result.returncode:
        raise RuntimeError(f"{' '.join(command)} failed:\n" + "\n".join(messages))
    if messages:
        print("\n".join(messages), file=sys.stderr)


def build(jobs: int | None = None, verbose: bool = True) -> Path:
    compiler = hipcc()
    digest = source_digest()
    BUILD.mkdir(parents=True, exist_ok=True)
    defines = [f"-DRG_SOURCE_DIGEST=\"{digest[:16]}\""]
    objects, commands = [], []
    for unit in UNITS:
        obj = BUILD / (unit + ".o")
        objects.append(obj)
        commands.append([compiler, f"--offload-arch={ARCH}", *FLAGS, *defines, "-I", str(INCLUDE),
                         "-c", str(CSRC / unit), "-o", str(obj)])
    workers = jobs or min(len(commands), max(1, os.cpu_count() or 1))
    with ThreadPoolExecutor(max_workers=workers) as pool:
        list(pool.map(_run, commands))
    temporary = LIBRARY.with_suffix(".so.tmp")
    _run([compiler, f"--offload-arch={ARCH}", "-shared", "-fPIC", *map(str, objects), "-o", str(temporary)])
    os.replace(temporary, LIBRARY)
    library_digest = hashlib.sha256(LIBRARY.read_bytes()).hexdigest()
    LIBRARY.with_name(LIBRARY.name + ".sha256").write_text(library_digest + "\n")
    if verbose:
        print(f"built {LIBRARY} (sources {digest[:16]}, library {library_digest[:16]})")
    return LIBRARY


def main(argv=None) -> int:
    parser = argparse.ArgumentParser(description=__doc__)
    parser.add_argument("--jobs", type=int)
    args = parser.parse_args(argv)
    build(args.jobs)
    return 0


if __name__ == "__main__":
    raise SystemExit(main())
