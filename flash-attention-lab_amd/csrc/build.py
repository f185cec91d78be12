"""Builds the gfx950 C-ABI library, flash_lab/libflash_lab_hip.so, with hipcc.

    python flash-attention-lab_amd/csrc/build.py [-v]

Each .hip file is compiled to an object in csrc/_build (in parallel), then linked into one shared
library next to the Python package, which loads it with ctypes. No CMake, no torch extension
machinery: the library has a plain C ABI (include/flash_lab_hip.h).
"""

from __future__ import annotations

import argparse
import concurrent.futures
import datetime
import hashlib
import json
import os
import shutil
import subprocess
import sys
from pathlib import Path

CSRC = Path(__file__).resolve().parent
PKG_ROOT = CSRC.parent
REPO = PKG_ROOT.parent
INCLUDE = REPO / "include"
BUILD_DIR = CSRC / "_build"
OUTPUT = PKG_ROOT / "flash_lab" / "libflash_lab_hip.so"

SOURCES = ("abi.hip", "prefill_fwd.hip", "prefill_pp.hip", "prefill_causal.hip", "decode.hip",
           "decode_mfma.hip", "smoke.hip")
ARCH = "gfx950"
FLAGS = (
    f"--offload-arch={ARCH}",
    "-O3",
    "-std=c++17",
    "-fPIC",
    # Packed fp32 VALU forms are kept out of the device code on purpose.
    "-Xclang",
    "-target-feature",
    "-Xclang",
    "-packed-fp32-ops",
    "-Wall",
    "-Wno-unused-function",
)


def hipcc() -> str:
    found = shutil.which("hipcc") or "/opt/rocm/bin/hipcc"
    if not Path(found).exists():
        raise RuntimeError("hipcc not found (is ROCm installed under /opt/rocm?)")
    return found


def _run(cmd: list[str], verbose: bool) -> None:
    if verbose:
        print(" ".join(cmd), flush=True)
    proc = subprocess.run(cmd, capture_output=True, text=True)
    # hipcc's host pass warns that it does not know the device-only feature; that is expected.
    noise = "is not a recognized feature for this target"
    err = "\n".join(line for line in proc.stderr.splitlines() if noise not in line)
    if proc.returncode != 0:
        raise RuntimeError(f"command failed ({proc.returncode}): {' '.join(cmd)}\n{err}")
    if verbose and err.strip():
        print(err, file=sys.stderr)


def build(
    verbose: bool = False,
    jobs: int | None = None,
    defines: tuple[str, ...] = (),
    output: Path | None = None,
) -> Path:
    """Compiles every source and links the library (OUTPUT unless `output` is given); always
    rebuilds. `defines` are NAME=VALUE preprocessor settings of the kernels' tuning knobs."""
    compiler = hipcc()
    output = Path(output) if output is not None else OUTPUT
    build_dir = BUILD_DIR if output == OUTPUT else output.parent / f"_build_{output.stem}"
    build_dir.mkdir(parents=True, exist_ok=True)
    includes = [f"-I{INCLUDE}", f"-I{CSRC}"]
    macro_flags = [f"-D{d}" for d in defines]
    objects = []
    commands = []
    for src in SOURCES:
        obj = build_dir / (Path(src).stem + ".o")
        objects.append(obj)
        commands.append(
            [compiler, *FLAGS, *macro_flags, *includes, "-c", str(CSRC / src), "-o", str(obj)]
        )
    workers = jobs or min(len(commands), os.cpu_count() or 1)
    with concurrent.futures.ThreadPoolExecutor(max_workers=workers) as pool:
        for fut in [pool.submit(_run, cmd, verbose) for cmd in commands]:
            fut.result()
    tmp = output.with_suffix(".so.tmp")
    _run([compiler, f"--offload-arch={ARCH}", "-shared", "-fPIC", *map(str, objects), "-o", str(tmp)],
         verbose)
    os.replace(tmp, output)
    write_build_record(output, compiler, defines)
    return output


def _git(*args: str) -> str | None:
    try:
        proc = subprocess.run(["git", "-C", str(REPO), *args], capture_output=True, text=True,
                              timeout=10)
    except (OSError, subprocess.TimeoutExpired):
        return None
    return proc.stdout.strip() if proc.returncode == 0 else None


def write_build_record(output: Path, compiler: str, defines: tuple[str, ...]) -> Path:
    """<library>.build.json beside the library: the source it was built from (git HEAD and whether
    the tree differed from it, plus a hash of the kernel sources and the header), the compiler
    and the flags. It travels with the library, so a benchmark run on another machine, where
    the checkout has no git metadata, can still say what it ran."""
    digest = hashlib.sha256()
    for path in sorted([*CSRC.glob("*.hip"), *CSRC.glob("*.hpp"), *INCLUDE.glob("*.h")]):
        digest.update(path.name.encode())
        digest.update(path.read_bytes())
    status = _git("status", "--porcelain", "--", str(CSRC), str(INCLUDE))
    version = subprocess.run([compiler, "--version"], capture_output=True, text=True).stdout
    record = {
        "git_head": _git("rev-parse", "HEAD"),
        "sources_differ_from_head": bool(status) if status is not None else None,
        "sources_sha256": digest.hexdigest(),
        "compiler": version.splitlines()[0] if version else compiler,
        "flags": [*FLAGS, *(f"-D{d}" for d in defines)],
        "built_at": datetime.datetime.now(datetime.timezone.utc).isoformat(timespec="seconds"),
    }
    path = output.with_suffix(".build.json")
    path.write_text(json.dumps(record, indent=1) + "\n")
    return path


def main(argv=None) -> int:
    parser = argparse.ArgumentParser(description=__doc__.splitlines()[0])
    parser.add_argument("-v", "--verbose", action="store_true")
    parser.add_argument("-j", "--jobs", type=int)
    parser.add_argument("-D", "--define", action="append", default=[], help="NAME=VALUE knob")
    parser.add_argument("-o", "--output", type=Path)
    args = parser.parse_args(argv)
    path = build(verbose=args.verbose, jobs=args.jobs, defines=tuple(args.define),
                 output=args.output)
    print(f"built {path}")
    return 0


if __name__ == "__main__":
    raise SystemExit(main())
