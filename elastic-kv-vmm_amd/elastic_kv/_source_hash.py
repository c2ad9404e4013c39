"""Fingerprint of the native sources.

build_native.py compiles it into libelastic_vmm.so (ekv_source_hash) and the
launch helper module (source_hash()), and the loader compares it with the
sources next to them, so a build from older sources is refused instead of
running stale kernels.
"""

import hashlib
from pathlib import Path

PACKAGE_ROOT = Path(__file__).resolve().parents[1]
HEADER_DIR = PACKAGE_ROOT.parent / "include"


def native_sources():
    """The HIP and C++ sources and headers the library and launch helper are built from, in a fixed order."""
    sources = sorted(path for path in (PACKAGE_ROOT / "csrc").glob("*") if path.suffix in (".hip", ".cpp", ".h"))
    return sources + sorted(HEADER_DIR.glob("*.h"))


def source_hash():
    """32 hex digits of SHA-256 over the names and bytes of native_sources(); None without sources."""
    sources = native_sources()
    if not sources:
        return None
    digest = hashlib.sha256()
    for path in sources:
        digest.update(path.name.encode() + b"\0" + path.read_bytes() + b"\0")
    return digest.hexdigest()[:32]
