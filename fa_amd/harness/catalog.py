"""The backend catalog: which attention implementations exist and how to run them.

A backend is a directory ``<root>/<name>/`` holding ``backend.py`` with a
module-level ``META`` (``fa_amd.harness.contract.Meta``) and the hooks of its
type (``fa_amd.harness.drivers``). The catalog imports every such module once,
keys it by the directory name (``META.name`` is only a label, as in the
reference's plugin API), and checks the one global rule: exactly one backend
is the correctness reference. Backend modules import torch and load
libraries inside functions, so building the catalog is cheap and works on a
host without a GPU.

Typical use::

    cat = Catalog.default()
    bind = cat.prepare("hip_fa_fp32acc", case)    # loads the library
    forward = bind(canonical)                     # adapts the inputs
    out = forward()                               # one forward
"""

from __future__ import annotations

import importlib
from dataclasses import dataclass
from pathlib import Path
from types import ModuleType

from fa_amd.harness import drivers

BACKENDS_PACKAGE = "fa_amd.backends"


@dataclass(frozen=True)
class Backend:
    """One catalog entry: the directory name and the imported module."""
    name: str
    module: ModuleType

    @property
    def meta(self):
        return self.module.META

    @property
    def driver(self):
        return drivers.driver(self.meta.type)

    @property
    def is_attention(self) -> bool:
        return not self.meta.diagnostic


class Catalog:
    """Backends found under one package directory, keyed by directory name."""

    def __init__(self, entries):
        self._entries = dict(entries)
        refs = [name for name, e in self._entries.items() if e.meta.is_reference]
        if len(refs) != 1:
            raise ValueError(f"exactly one reference backend is required, found {refs or 'none'}")
        self._reference = refs[0]

    @classmethod
    def scan(cls, package: str = BACKENDS_PACKAGE) -> "Catalog":
        root = Path(importlib.import_module(package).__file__).resolve().parent
        entries = {}
        for path in sorted(root.glob("*/backend.py")):
            name = path.parent.name
            module = importlib.import_module(f"{package}.{name}.backend")
            if not hasattr(module, "META"):
                raise TypeError(f"{module.__name__} declares no META")
            entries[name] = Backend(name, module)
        return cls(entries)

    _default = None

    @classmethod
    def default(cls, rescan: bool = False) -> "Catalog":
        """The catalog of this package's backends (scanned once per process)."""
        if cls._default is None or rescan:
            cls._default = cls.scan()
        return cls._default

    def __contains__(self, name) -> bool:
        return name in self._entries

    def __getitem__(self, name) -> Backend:
        try:
            return self._entries[name]
        except KeyError:
            raise KeyError(f"no backend {name!r} (known: {', '.join(self._entries)})") from None

    def names(self, include_diagnostic: bool = False) -> list:
        return [n for n, e in self._entries.items() if include_diagnostic or e.is_attention]

    @property
    def reference(self) -> Backend:
        return self._entries[self._reference]

    def attention(self, name) -> Backend:
        """The entry for ``name``, refusing diagnostic-only modules."""
        entry = self[name]
        if not entry.is_attention:
            raise ValueError(f"{name} is a diagnostic backend, not an attention implementation")
        return entry

    def name_of(self, module) -> str:
        """Directory name under which ``module`` is registered."""
        hits = [n for n, e in self._entries.items() if e.module is module]
        if len(hits) != 1:
            raise ValueError(f"{getattr(module, '__name__', module)!r} is registered "
                             f"{len(hits)} times")
        return hits[0]

    def prepare(self, name, case):
        """``bind(canonical) -> zero-argument forward`` for backend ``name``."""
        entry = self[name]
        return entry.driver.prepare(entry.module, case)

    def build(self, name, case) -> bool:
        """Run the backend's build step if it has one; True when it did."""
        entry = self[name]
        if not entry.driver.needs_build(entry.module):
            return False
        entry.driver.build(entry.module, case)
        return True
