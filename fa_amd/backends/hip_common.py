"""Shared declaration of the two HIP backends (FP32- and FP16-accumulated O).

Both backends drive the same ``libfa_hip.so`` through the ``hip`` project
driver; they differ only in the accumulation variant passed to ``fa_fwd``.
This mirrors how the reference's two CCE projects share one operator
interface (``backends/cce_fa_nk_nz_vector_fp32_v5_sumpack/backend.py:58-81``):
``project`` declares the recipe, ``load`` opens the built library before any
input exists, ``adapt`` maps the canonical tensors to positional arguments.
"""

import sys
from pathlib import Path

PACKAGE_ROOT = Path(__file__).resolve().parent.parent
LIBRARY = "_lib/libfa_hip.so"
MANIFEST = "_lib/build.json"


def project(case, prebuilt=False):
    """The HIP project recipe: sources under ``fa_amd/csrc``, built by ``fa_amd/build.py``.

    The build is content-hashed. When the library on disk matches the sources
    (a check that only reads files) the recipe carries no build command, so
    loading an up-to-date library never starts a process; ``prebuilt=True``
    skips the build command unconditionally and only checks the artifacts.
    """
    from fa_amd import build
    from fa_amd.core.drivers.hip import Project

    current = prebuilt or build.up_to_date()
    command = () if current else (sys.executable, str(PACKAGE_ROOT / "build.py"))
    return Project(PACKAGE_ROOT, (LIBRARY, MANIFEST), command)


def load(acc, case, project, kernel=0):
    from fa_amd.binding import AttentionConfig, Operator

    return Operator(project.artifact_paths()[0], AttentionConfig(acc=acc, kernel=kernel))


def adapt(case, canonical):
    return tuple(canonical[name] for name in ("q", "k", "v"))
