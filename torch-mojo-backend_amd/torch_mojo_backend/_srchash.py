"""Digest of the kernel library's sources.

build.py compiles it into the library (`mi355x_source_hash()`); the loader
recomputes it from the sources beside the package and refuses a library
built from other sources, so a stale prebuilt .so cannot load silently.
This module imports nothing from the package (build.py loads it by path).
"""

from __future__ import annotations

import hashlib
from pathlib import Path

PKG_DIR = Path(__file__).resolve().parents[1]  # torch-mojo-backend_amd/
CSRC = PKG_DIR / "csrc"
INCLUDE = PKG_DIR.parent / "include"


def source_files() -> list[Path]:
    files = list(CSRC.glob("*.hip")) + list(CSRC.glob("*.h")) + list(INCLUDE.glob("*.h"))
    return sorted(files, key=lambda f: (f.parent.name, f.name))


def source_hash(flags: list[str] | tuple[str, ...] = ()) -> str | None:
    """sha256 (first 16 hex digits) over the sources' names and bytes and
    the compile flags; None when the sources are not present."""
    files = source_files()
    if not files:
        return None
    h = hashlib.sha256()
    for f in files:
        h.update(f"{f.parent.name}/{f.name}\0".encode())
        h.update(f.read_bytes())
        h.update(b"\0")
    h.update(" ".join(flags).encode())
    return h.hexdigest()[:16]
