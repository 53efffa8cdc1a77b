"""Source identity of the gfx950 library, for detecting a stale build.

The Makefile embeds `clef-build-id:<hash>` in lib/libclef_i4.so, where
<hash> is the first 16 hex digits of the SHA-256 of the concatenated bytes of
csrc/* (sorted by path), ../include/clef_i4.h and the Makefile. This module
computes the same hash from the tree and reads the embedded one from the file
without loading the library (a loaded library cannot be replaced in-process).
"""
from __future__ import annotations

import glob
import hashlib
import os

_HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(_HERE, "lib", "libclef_i4.so")
_TAG = b"clef-build-id:"


def source_id() -> str | None:
    """Hash of the sources, or None when the tree holds no sources."""
    srcs = sorted(glob.glob(os.path.join(_HERE, "csrc", "*")))
    if not srcs:
        return None
    files = srcs + [os.path.join(_HERE, "..", "include", "clef_i4.h"), os.path.join(_HERE, "Makefile")]
    h = hashlib.sha256()
    for f in files:
        with open(f, "rb") as fh:
            h.update(fh.read())
    return h.hexdigest()[:16]


def library_id(path: str = LIB_PATH) -> str | None:
    """The identity embedded in the built library, or None if absent."""
    try:
        with open(path, "rb") as fh:
            data = fh.read()
    except FileNotFoundError:
        return None
    at = data.find(_TAG)
    if at < 0:
        return None
    return data[at + len(_TAG):at + len(_TAG) + 16].decode("ascii", "replace")


def stale() -> str | None:
    """A message when the library is missing or built from other sources."""
    src, built = source_id(), library_id()
    if built is None:
        return f"{LIB_PATH} is not built (or carries no build identity)"
    if src is not None and src != built:
        return f"{LIB_PATH} was built from other sources (library {built}, tree {src})"
    return None
