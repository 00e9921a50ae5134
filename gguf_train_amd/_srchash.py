"""Fingerprint of the sources libgt_attn.so is built from.

The build compiles the fingerprint into the library (gt_source_hash) and the loader compares it
with the sources next to it, so a library built from other sources than the tree it sits in is
refused instead of silently run.  Inputs: every csrc/*.hip, *.cpp, *.h and *.py (source
generators) file and include/gt_attn.h, by name and content, in sorted order.
"""

from __future__ import annotations

import hashlib
from pathlib import Path

PKG_DIR = Path(__file__).resolve().parent


def source_files(pkg_dir: Path = PKG_DIR) -> list[Path]:
    csrc = pkg_dir / "csrc"
    files = [p for pat in ("*.hip", "*.cpp", "*.h", "*.py") for p in csrc.glob(pat)]
    files.append(pkg_dir.parent / "include" / "gt_attn.h")
    return sorted(files, key=lambda p: p.name)


def source_hash(pkg_dir: Path = PKG_DIR) -> str | None:
    """Hex SHA-256 over the sources, or None when they are not present (an installed library)."""
    files = source_files(pkg_dir)
    if not all(p.is_file() for p in files) or len(files) < 2:
        return None
    h = hashlib.sha256()
    for p in files:
        h.update(p.name.encode() + b"\0")
        h.update(p.read_bytes())
        h.update(b"\0")
    return h.hexdigest()
