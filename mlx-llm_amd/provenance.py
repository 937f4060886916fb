"""Source hash of libmlxq.so: the kernel, host and header sources plus the
build script, so that a library built from other sources (a stale .so
pushed with a newer tree) is detected instead of silently measured."""
from __future__ import annotations

import hashlib
from pathlib import Path

PKG = Path(__file__).resolve().parent
ROOT = PKG.parent


def source_files() -> list[Path]:
    files = [PKG / "build.py"]
    for d, pats in ((PKG / "csrc", ("*.hip", "*.cpp", "*.hpp", "*.h")), (PKG / "host", ("*.cpp", "*.hpp", "*.h")),
                    (ROOT / "include", ("*.h",))):
        for pat in pats:
            files += d.glob(pat)
    return sorted(set(files))


def source_hash() -> str:
    h = hashlib.sha256()
    for f in source_files():
        h.update(str(f.relative_to(ROOT)).encode() + b"\0" + f.read_bytes() + b"\0")
    return h.hexdigest()[:16]


def library_hash(version: str) -> str | None:
    """The src=... field of mlxq_version()."""
    for part in version.split():
        if part.startswith("src="):
            return part[4:]
    return None
