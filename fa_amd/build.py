"""Build ``libfa_hip.so`` for gfx950 with hipcc, keyed by a content hash.

The build identity is the SHA-256 of every source and header the library is
compiled from and the compiler command line (the hipcc version is recorded in
the manifest), the pattern of the reference's source-hashed CANN build
(``backends/cce_fa_nk_nz_vector_fp32_v5_sumpack/project/build.py:17-116``):
an up-to-date library is never rebuilt, a stale or partial one always is, and
``build.json`` beside the library records what it was built from. Checking
whether the library is up to date only reads files: it starts no process, so
it is safe inside a process that has already initialised the GPU.

Run as ``python -m fa_amd.build [--force]`` or ``python fa_amd/build.py``.
"""

import argparse
import hashlib
import json
import os
import shutil
import subprocess
import sys
import tempfile
from pathlib import Path

PKG = Path(__file__).resolve().parent
REPO = PKG.parent
CSRC = PKG / "csrc"
INCLUDE = REPO / "include"
LIBDIR = PKG / "_lib"
LIBRARY = LIBDIR / "libfa_hip.so"
MANIFEST = LIBDIR / "build.json"

ARCH = "gfx950"
HIPCC = os.environ.get("HIPCC", "/opt/rocm/bin/hipcc")
# Packed FP32 VALU forms stay disabled for all device code.
FLAGS = (
    f"--offload-arch={ARCH}", "-O3", "-std=c++17", "-shared", "-fPIC",
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
)


def sources():
    return sorted(CSRC.glob("*.hip")) + sorted(INCLUDE.glob("*.h"))


def _hipcc_version():
    try:
        out = subprocess.run([HIPCC, "--version"], capture_output=True, text=True, timeout=120)
        return out.stdout.strip()
    except (OSError, subprocess.SubprocessError):
        return "unavailable"


def identity():
    h = hashlib.sha256()
    for path in sources():
        h.update(str(path.relative_to(REPO)).encode())
        h.update(path.read_bytes())
    h.update(" ".join(FLAGS).encode())
    return h.hexdigest()


def up_to_date():
    if not LIBRARY.is_file() or not MANIFEST.is_file():
        return False
    try:
        manifest = json.loads(MANIFEST.read_text())
    except (OSError, ValueError):
        return False
    return (manifest.get("identity") == identity()
            and manifest.get("sha256") == hashlib.sha256(LIBRARY.read_bytes()).hexdigest())


def build(force=False, verbose=False):
    """Compile the library unless an identical build is already in place."""
    if not force and up_to_date():
        if verbose:
            print(f"up to date: {LIBRARY}")
        return LIBRARY
    LIBDIR.mkdir(exist_ok=True)
    hip_sources = sorted(CSRC.glob("*.hip"))
    ident = identity()
    with tempfile.TemporaryDirectory(dir=LIBDIR) as tmp:
        out = Path(tmp) / LIBRARY.name
        cmd = [HIPCC, *FLAGS, f"-I{INCLUDE}", *map(str, hip_sources), "-o", str(out)]
        if verbose:
            print(" ".join(cmd))
        res = subprocess.run(cmd, capture_output=True, text=True, cwd=tmp)
        if res.returncode != 0:
            sys.stderr.write(res.stdout + res.stderr)
            raise RuntimeError(f"hipcc failed with status {res.returncode}")
        MANIFEST.unlink(missing_ok=True)
        shutil.move(str(out), LIBRARY)
    MANIFEST.write_text(json.dumps({
        "identity": ident,
        "sha256": hashlib.sha256(LIBRARY.read_bytes()).hexdigest(),
        "arch": ARCH,
        "flags": list(FLAGS),
        "hipcc": _hipcc_version(),
        "sources": [str(p.relative_to(REPO)) for p in sources()],
    }, indent=1))
    if verbose:
        print(f"built: {LIBRARY}")
    return LIBRARY


def main(argv=None):
    ap = argparse.ArgumentParser(description=__doc__.splitlines()[0])
    ap.add_argument("--force", action="store_true", help="rebuild even when up to date")
    args = ap.parse_args(argv)
    build(force=args.force, verbose=True)


if __name__ == "__main__":
    main()
