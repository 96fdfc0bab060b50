"""Builds libbaracuda_kernels.so (every HIP kernel of the package, gfx950 only).

Each ``csrc/*.hip`` translation unit is compiled to an object under
``baracuda_amd/_build/`` in parallel and the objects are linked into
``baracuda_amd/libbaracuda_kernels.so`` (in-tree, so the library travels with
the source tree).  ``python -m baracuda_amd.build`` runs it.
"""
from __future__ import annotations

import concurrent.futures as cf
import hashlib
import os
import shutil
import subprocess
import sys
from pathlib import Path

PKG = Path(__file__).resolve().parent
ROOT = PKG.parent
CSRC = PKG / "csrc"
BUILD = PKG / "_build"
LIB = PKG / "libbaracuda_kernels.so"
# Measurement kernels of bench.py (not product), built beside the library.
PROBES = PKG / "probes"
PROBE_LIB = PKG / "libbaracuda_probes.so"
# Digest of the sources and flags the library was built from, written beside it.
STAMP = PKG / "libbaracuda_kernels.so.srchash"

HIPCC = os.environ.get("HIPCC", shutil.which("hipcc") or "/opt/rocm/bin/hipcc")
ARCH = "gfx950"
# -packed-fp32-ops: hipcc must not emit packed f32 VALU ops (v_pk_*_f32).
# -ffp-contract=off: epilogue arithmetic is evaluated exactly as written, so
# the W8A8 / FP8 dequant products round like the oracle's.
HIP_FLAGS = [
    f"--offload-arch={ARCH}", "-O3", "-std=c++17", "-fPIC",
    "-ffp-contract=off",
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    f"-I{ROOT / 'include'}", f"-I{CSRC}",
]
# Size of the allocation-free u8 RRR entry point's device array, which every
# process that loads the library holds on each GPU it uses (default 64 MiB).
if os.environ.get("BK_NOALLOC_SCRATCH_MIB"):
    HIP_FLAGS.insert(-2, f"-DBARACUDA_U8_RRR_NOALLOC_SCRATCH_BYTES=((size_t){int(os.environ['BK_NOALLOC_SCRATCH_MIB'])}<<20)")


def _compile(src: Path) -> Path:
    obj = BUILD / (src.stem + ".o")
    cmd = [HIPCC, *HIP_FLAGS, "-c", str(src), "-o", str(obj)]
    res = subprocess.run(cmd, capture_output=True, text=True)
    if res.returncode != 0:
        raise RuntimeError(f"hipcc failed for {src.name}:\n{res.stderr}")
    return obj


def source_digest() -> str:
    """SHA-256 over every kernel source, public header and the build flags."""
    h = hashlib.sha256()
    h.update(" ".join(HIP_FLAGS[:-2]).encode())
    files = (sorted(CSRC.glob("*.hip")) + sorted(CSRC.glob("*.hpp")) + sorted((ROOT / "include").glob("*.h"))
             + sorted(PROBES.glob("*.hip")))
    for f in files:
        h.update(f.name.encode())
        h.update(f.read_bytes())
    return h.hexdigest()


def is_stale() -> bool:
    """True when the library is missing or was built from other sources."""
    if not LIB.exists() or not STAMP.exists() or (any(PROBES.glob("*.hip")) and not PROBE_LIB.exists()):
        return True
    return STAMP.read_text().strip() != source_digest()


def ensure_built(verbose: bool = False) -> Path:
    """Build only when the library is missing or stale (source digest differs)."""
    if is_stale():
        build(verbose=verbose)
    return LIB


def _build_probes() -> None:
    """Measurement kernels (probes/*.hip) into their own library, so the
    product library exports exactly what include/baracuda_kernels.h declares."""
    srcs = sorted(PROBES.glob("*.hip"))
    if not srcs:
        return
    tmp = PROBE_LIB.with_suffix(".so.tmp")
    cmd = [HIPCC, *HIP_FLAGS, "-shared", *map(str, srcs), "-o", str(tmp)]
    res = subprocess.run(cmd, capture_output=True, text=True)
    if res.returncode != 0:
        raise RuntimeError(f"hipcc failed for the probes:\n{res.stderr}")
    os.replace(tmp, PROBE_LIB)


def build(verbose: bool = False) -> Path:
    """Compile every kernel source and link the shared library; returns its path."""
    BUILD.mkdir(exist_ok=True)
    digest = source_digest()
    sources = sorted(CSRC.glob("*.hip"))
    with cf.ThreadPoolExecutor(max_workers=min(8, len(sources))) as ex:
        objs = list(ex.map(_compile, sources))
    tmp = LIB.with_suffix(".so.tmp")
    cmd = [HIPCC, f"--offload-arch={ARCH}", "-shared", "-fPIC", *map(str, objs), "-o", str(tmp)]
    res = subprocess.run(cmd, capture_output=True, text=True)
    if res.returncode != 0:
        raise RuntimeError(f"link failed:\n{res.stderr}")
    os.replace(tmp, LIB)
    _build_probes()
    STAMP.write_text(digest + "\n")
    if verbose:
        # stderr: callers such as bench.py keep stdout for their own output
        print(f"built {LIB} from {len(sources)} sources", file=sys.stderr)
    return LIB


if __name__ == "__main__":
    build(verbose=True)
    sys.exit(0)
