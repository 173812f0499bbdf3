"""Build the gfx950 kernel library `libmi355x_kernels.so` in-tree.

One shared library holds every kernel (one gfx950 code object per source
file, linked together) behind the C ABI declared in
`include/mi355x_kernels.h`.  Sources compile in parallel; a source is rebuilt
when it, `common.h` or the public header is newer than its object.

    python torch-mojo-backend_amd/build.py [--force] [-j N]
"""

from __future__ import annotations

import argparse
import os
import shutil
import subprocess
import sys
from concurrent.futures import ThreadPoolExecutor
from pathlib import Path

PKG_DIR = Path(__file__).resolve().parent
REPO = PKG_DIR.parent
CSRC = PKG_DIR / "csrc"
OBJ_DIR = PKG_DIR / "_build"
INCLUDE = REPO / "include"
LIB_NAME = "libmi355x_kernels.so"
LIB_PATH = PKG_DIR / "torch_mojo_backend" / "eager_kernels" / LIB_NAME

ARCH = "gfx950"
# -packed-fp32-ops: keep the compiler from emitting packed f32 VALU ops.
COMMON_FLAGS = [
    f"--offload-arch={ARCH}",
    "-O3",
    "-fPIC",
    "-std=c++17",
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    "-Wno-unused-result",
    f"-I{INCLUDE}",
    f"-I{CSRC}",
]


def _hash_flags() -> list[str]:
    """The flags the digest covers (paths excluded: the tree may move)."""
    return [f for f in COMMON_FLAGS if not f.startswith("-I")]


def _source_hash() -> str:
    import importlib.util

    spec = importlib.util.spec_from_file_location("_mi355x_srchash", PKG_DIR / "torch_mojo_backend" / "_srchash.py")
    mod = importlib.util.module_from_spec(spec)
    spec.loader.exec_module(mod)
    return mod.source_hash(_hash_flags())


def hipcc() -> str:
    for cand in (os.environ.get("HIPCC"), "/opt/rocm/bin/hipcc", shutil.which("hipcc")):
        if cand and Path(cand).exists():
            return cand
    raise RuntimeError("hipcc not found: the gfx950 kernel library cannot be built")


def _deps_mtime() -> float:
    deps = [CSRC / "common.h", INCLUDE / "mi355x_kernels.h"]
    deps += list(CSRC.glob("*.h"))
    return max(p.stat().st_mtime for p in deps if p.exists())


def _compile(src: Path, force: bool, defines: tuple[str, ...] = ()) -> Path:
    obj = OBJ_DIR / (src.stem + ".o")
    if (
        not force
        and not defines
        and obj.exists()
        and obj.stat().st_mtime >= max(src.stat().st_mtime, _deps_mtime())
    ):
        return obj
    cmd = [hipcc(), *COMMON_FLAGS, *defines, "-c", str(src), "-o", str(obj)]
    proc = subprocess.run(cmd, capture_output=True, text=True)
    if proc.returncode != 0:
        raise RuntimeError(f"compiling {src.name} failed:\n{proc.stderr}")
    return obj


def build(force: bool = True, jobs: int | None = None) -> Path:
    """Compile every csrc/*.hip for gfx950 and link the shared library."""
    OBJ_DIR.mkdir(exist_ok=True)
    sources = sorted(CSRC.glob("*.hip"))
    if not sources:
        raise RuntimeError(f"no HIP sources under {CSRC}")
    jobs = jobs or min(8, os.cpu_count() or 4)
    # runtime.hip carries the source digest, so it is rebuilt every time
    digest = (f'-DMI355X_SOURCE_HASH="{_source_hash()}"',)
    with ThreadPoolExecutor(max_workers=jobs) as pool:
        objs = list(pool.map(lambda s: _compile(s, force, digest if s.name == "runtime.hip" else ()), sources))
    tmp = LIB_PATH.with_suffix(".so.tmp")
    cmd = [hipcc(), f"--offload-arch={ARCH}", "-shared", "-fPIC", "-o", str(tmp), *map(str, objs)]
    proc = subprocess.run(cmd, capture_output=True, text=True)
    if proc.returncode != 0:
        raise RuntimeError(f"linking {LIB_NAME} failed:\n{proc.stderr}")
    os.replace(tmp, LIB_PATH)
    return LIB_PATH


def main() -> int:
    ap = argparse.ArgumentParser()
    ap.add_argument("--force", action="store_true", help="rebuild every object")
    ap.add_argument("-j", type=int, default=None)
    args = ap.parse_args()
    path = build(force=args.force, jobs=args.j)
    print(path)
    return 0


if __name__ == "__main__":
    sys.exit(main())
