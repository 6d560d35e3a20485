"""Hash of the sources libfpa.so is built from (csrc/*, include/fpa.h).

build.py bakes it into the library (fpa_source_hash()); the loader recomputes it from the
sources next to the package and refuses a library built from other sources.  No torch import:
build.py uses this module before torch is needed.
"""
import hashlib
import os

PKG = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))  # first-passage-attention_amd/
ROOT = os.path.dirname(PKG)


def source_files():
    csrc = os.path.join(PKG, "csrc")
    files = sorted(os.path.join(csrc, f) for f in os.listdir(csrc)
                   if f.endswith((".hip", ".h", ".hpp", ".cpp")))
    return files + [os.path.join(ROOT, "include", "fpa.h")]


def source_hash():
    """sha256 (first 16 hex digits) over the names and contents of the library's sources, or None
    when they are not present."""
    h = hashlib.sha256()
    try:
        for f in source_files():
            h.update(os.path.basename(f).encode() + b"\0")
            with open(f, "rb") as fh:
                h.update(fh.read())
    except OSError:
        return None
    return h.hexdigest()[:16]
