"""Build the gfx950 shared libraries with hipcc, each keyed by a content hash.

Two libraries:

* ``libfa_hip.so`` -- the attention forward and its C ABI
  (``fa_amd/csrc/fa_fwd.hip``, ``include/fa_hip.h``);
* ``libfa_ceiling.so`` -- a measurement kernel that issues nothing but FP16
  MFMAs, for the board's sustained matrix rate
  (``fa_amd/csrc/measure/mfma_ceiling.hip``); never loaded by the attention
  path;
* on request (``--sanitize``), ``libfa_hip_hostsan.so`` -- the attention
  library with its host code (the C ABI's validation, sizing and launch
  set-up) built with AddressSanitizer and UndefinedBehaviorSanitizer; the
  device code is unchanged. Load it with the clang ASan runtime preloaded
  (``LD_PRELOAD=$(hipcc -print-file-name=libclang_rt.asan-x86_64.so)
  ASAN_OPTIONS=detect_leaks=0``) and point the tests at it with
  ``FA_TEST_LIBRARY``.

A library's build identity is the SHA-256 of every source and header it is
compiled from and of the compiler command line (the hipcc version is recorded
in the manifest), the pattern of the reference's source-hashed CANN build
(``backends/cce_fa_nk_nz_vector_fp32_v5_sumpack/project/build.py:17-116``):
an up-to-date library is never rebuilt, a stale or partial one always is, and
a JSON manifest beside the library records what it was built from. Checking
whether a library is up to date only reads files: it starts no process, so it
is safe inside a process that has already initialised the GPU.

Run as ``python -m fa_amd.build [--force]`` or ``python fa_amd/build.py``.
"""

import argparse
import fcntl
import hashlib
import json
import os
import shutil
import subprocess
import sys
import tempfile
from dataclasses import dataclass
from pathlib import Path

PKG = Path(__file__).resolve().parent
REPO = PKG.parent
CSRC = PKG / "csrc"
INCLUDE = REPO / "include"
LIBDIR = PKG / "_lib"

ARCH = "gfx950"
HIPCC = os.environ.get("HIPCC", "/opt/rocm/bin/hipcc")
# Packed FP32 VALU forms stay disabled for all device code.
FLAGS = (
    f"--offload-arch={ARCH}", "-O3", "-std=c++17", "-shared", "-fPIC",
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
)


@dataclass(frozen=True)
class Target:
    name: str          # library file name
    hip: tuple         # HIP sources, relative to CSRC
    headers: tuple     # headers the build depends on, relative to REPO
    flags: tuple = ()  # extra compiler flags of this target

    @property
    def library(self) -> Path:
        return LIBDIR / self.name

    @property
    def manifest(self) -> Path:
        return LIBDIR / (Path(self.name).stem + ".json")

    def sources(self):
        return [CSRC / s for s in self.hip] + [REPO / h for h in self.headers]


ATTENTION = Target("libfa_hip.so", ("fa_fwd.hip",), ("include/fa_hip.h",))
CEILING = Target("libfa_ceiling.so", ("measure/mfma_ceiling.hip",), ())
TARGETS = (ATTENTION, CEILING)
# Host-side sanitizers only (each -fsanitize= behind -Xarch_host): GPU code
# is never built with them.
HOSTSAN = Target("libfa_hip_hostsan.so", ("fa_fwd.hip",), ("include/fa_hip.h",), (
    "-g",
    "-Xarch_host", "-fsanitize=address",
    "-Xarch_host", "-fsanitize=undefined",
    "-Xarch_host", "-fno-omit-frame-pointer",
))

# The attention library (what the product path loads).
LIBRARY = ATTENTION.library
MANIFEST = ATTENTION.manifest


def sources(target=ATTENTION):
    return target.sources()


def _hipcc_version():
    try:
        out = subprocess.run([HIPCC, "--version"], capture_output=True, text=True, timeout=120)
        return out.stdout.strip()
    except (OSError, subprocess.SubprocessError):
        return "unavailable"


def identity(target=ATTENTION):
    h = hashlib.sha256()
    for path in target.sources():
        h.update(str(path.relative_to(REPO)).encode())
        h.update(path.read_bytes())
    h.update(" ".join(FLAGS + target.flags).encode())
    return h.hexdigest()


def up_to_date(target=ATTENTION):
    if not target.library.is_file() or not target.manifest.is_file():
        return False
    try:
        manifest = json.loads(target.manifest.read_text())
    except (OSError, ValueError):
        return False
    return (manifest.get("identity") == identity(target)
            and manifest.get("sha256") == hashlib.sha256(target.library.read_bytes()).hexdigest())


def build(force=False, verbose=False, target=ATTENTION):
    """Compile ``target`` unless an identical build is already in place.

    Concurrent callers (parallel test workers, several harness processes)
    serialise on an exclusive lock file beside the libraries; whoever waits
    re-checks the manifest afterwards and finds the fresh build.
    """
    if not force and up_to_date(target):
        if verbose:
            print(f"up to date: {target.library}")
        return target.library
    LIBDIR.mkdir(exist_ok=True)
    with open(LIBDIR / ".build.lock", "a") as lock:
        fcntl.flock(lock, fcntl.LOCK_EX)
        if not force and up_to_date(target):
            return target.library
        return _compile(target, verbose)


def build_all(force=False, verbose=False):
    return [build(force=force, verbose=verbose, target=t) for t in TARGETS]


def _compile(target, verbose):
    ident = identity(target)
    with tempfile.TemporaryDirectory(dir=LIBDIR) as tmp:
        out = Path(tmp) / target.name
        cmd = [HIPCC, *FLAGS, *target.flags, f"-I{INCLUDE}", *(str(CSRC / s) for s in target.hip),
               "-o", str(out)]
        if verbose:
            print(" ".join(cmd))
        res = subprocess.run(cmd, capture_output=True, text=True, cwd=tmp)
        if res.returncode != 0:
            sys.stderr.write(res.stdout + res.stderr)
            raise RuntimeError(f"hipcc failed with status {res.returncode}")
        target.manifest.unlink(missing_ok=True)
        shutil.move(str(out), target.library)
    target.manifest.write_text(json.dumps({
        "identity": ident,
        "sha256": hashlib.sha256(target.library.read_bytes()).hexdigest(),
        "arch": ARCH,
        "flags": list(FLAGS + target.flags),
        "hipcc": _hipcc_version(),
        "sources": [str(p.relative_to(REPO)) for p in target.sources()],
    }, indent=1))
    if verbose:
        print(f"built: {target.library}")
    return target.library


def main(argv=None):
    ap = argparse.ArgumentParser(description=__doc__.splitlines()[0])
    ap.add_argument("--force", action="store_true", help="rebuild even when up to date")
    ap.add_argument("--sanitize", action="store_true",
                    help="also build libfa_hip_hostsan.so (host code under ASan and UBSan)")
    args = ap.parse_args(argv)
    build_all(force=args.force, verbose=True)
    if args.sanitize:
        build(force=args.force, verbose=True, target=HOSTSAN)


if __name__ == "__main__":
    main()
