"""Which code a measurement ran.

Every archived result line (bench.py, the benchmark matrix) carries a stamp:
a short hash of the sources that build the measured path, the same hash as
recorded by build.py when it compiled the library that ran (so a stale build
shows), and the git commit of the tree when the tree has one (the GPU boxes
receive the sources without .git). make_report.py --check compares archived
stamps with the current sources and fails on a mismatch, so archived numbers
cannot silently outlive the kernels they measured.
"""

import glob
import hashlib
import json
import os

PKG_DIR = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
REPO_ROOT = os.path.dirname(PKG_DIR)

# Sources of each measured path, relative to the repository root: the kernels,
# their C ABI header and the host code between the caller and the kernels.
SOURCES = {
    "gqa": ["mla-decode-kernels_amd/csrc/gqa_*.hip", "mla-decode-kernels_amd/csrc/gqa_*.hpp",
            "include/gqa_decode.h", "mla-decode-kernels_amd/python/gqa_decode_ext.cpp"],
    "mla": ["mla-decode-kernels_amd/csrc/mla_decode.hip", "include/mla_decode.h",
            "mla-decode-kernels_amd/python/mla.py"],
}


def source_files(kind, root=REPO_ROOT):
    files = set()
    for pattern in SOURCES[kind]:
        files.update(glob.glob(os.path.join(root, pattern)))
    return sorted(os.path.relpath(f, root) for f in files)


def source_hash(kind, root=REPO_ROOT):
    """First 16 hex digits of SHA-256 over the path's sources (each file's
    relative path, a NUL, its bytes, a NUL), in path order."""
    h = hashlib.sha256()
    for rel in source_files(kind, root):
        h.update(rel.encode() + b"\0")
        with open(os.path.join(root, rel), "rb") as f:
            h.update(f.read())
        h.update(b"\0")
    return h.hexdigest()[:16]


def sidecar_path(lib_path):
    return lib_path + ".sources.json"


def write_sidecar(lib_path, defines=(), root=REPO_ROOT):
    """Record, next to a freshly built library, the source hash of every path
    and the compile-time defines of a variant build."""
    rec = {kind: source_hash(kind, root) for kind in SOURCES}
    rec["defines"] = list(defines)
    with open(sidecar_path(lib_path), "w") as f:
        json.dump(rec, f, sort_keys=True)


def library_defines(lib_path):
    """The compile-time defines the library was built with ([] for the
    shipped build), or None without a record."""
    try:
        with open(sidecar_path(lib_path)) as f:
            return json.load(f).get("defines", [])
    except (OSError, ValueError):
        return None


def library_hash(kind, lib_path):
    """The source hash build.py recorded for the library, or None."""
    try:
        with open(sidecar_path(lib_path)) as f:
            return json.load(f).get(kind)
    except (OSError, ValueError):
        return None


def git_head(root=REPO_ROOT):
    """The commit checked out in `root` (read from .git without running git),
    or None where the tree has no .git."""
    git = os.path.join(root, ".git")
    try:
        with open(os.path.join(git, "HEAD")) as f:
            head = f.read().strip()
        if not head.startswith("ref: "):
            return head
        ref = head[5:]
        ref_file = os.path.join(git, ref)
        if os.path.exists(ref_file):
            with open(ref_file) as f:
                return f.read().strip()
        with open(os.path.join(git, "packed-refs")) as f:
            for line in f:
                parts = line.split()
                if len(parts) == 2 and parts[1] == ref:
                    return parts[0]
    except OSError:
        pass
    return None


def stamp(kind, lib_path):
    """The provenance record of a measurement of path `kind` run with the
    library at lib_path."""
    src = source_hash(kind)
    lib = library_hash(kind, lib_path)
    return {"path": kind, "source_sha16": src, "library_source_sha16": lib,
            "library_matches_sources": lib == src, "library_defines": library_defines(lib_path),
            "git_head": git_head()}
