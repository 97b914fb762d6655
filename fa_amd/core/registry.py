"""Backend discovery and driver lookup.

A backend is a module ``fa_amd/backends/<dir>/backend.py`` exposing a
module-level ``META`` (``fa_amd.core.contract.Meta``) and its type's hooks.
The registry keys backends by directory name and maps ``META.type`` to the
driver module. Importing a backend module must stay cheap (torch and the
shared library are imported inside functions), so discovery is safe on a host
without a GPU. Follows ``core/registry.py:1-88`` of the reference.
"""

import importlib
import os

_BACKENDS = None  # dirname -> module
_DRIVERS = {
    "external": "fa_amd.core.drivers.external",
    "hip": "fa_amd.core.drivers.hip",
}


def _backends_dir():
    return os.path.join(os.path.dirname(os.path.dirname(os.path.abspath(__file__))), "backends")


def prepare_call(spec, case):
    """Load early-loading drivers' libraries before any input tensor exists.

    Returns ``bind(canonical) -> zero-argument call``
    (reference ``core/registry.py:26-32``).
    """
    driver = driver_for(spec.META)
    prepare = getattr(driver, "prepare", None)
    if prepare is not None:
        return prepare(spec, case)
    return lambda canonical: driver.make_call(spec, case, canonical)


def discover(force=False):
    global _BACKENDS
    if _BACKENDS is not None and not force:
        return _BACKENDS
    backends = {}
    root = _backends_dir()
    for dirname in sorted(os.listdir(root)):
        if not os.path.isfile(os.path.join(root, dirname, "backend.py")):
            continue
        backends[dirname] = importlib.import_module(f"fa_amd.backends.{dirname}.backend")
    _BACKENDS = backends
    return backends


def get(name):
    """Return the backend module registered under ``name``."""
    return discover()[name]


def all_names(include_diagnostics=False):
    return [name for name, spec in discover().items()
            if include_diagnostics or not spec.META.diagnostic]


def require_attention(spec):
    if spec.META.diagnostic:
        raise ValueError(f"{name_of(spec)} is diagnostic-only, not an attention backend")


def name_of(spec):
    """Registry key of a backend module, independent of the legacy ``META.name``."""
    names = [name for name, module in discover().items() if module is spec]
    if len(names) != 1:
        raise ValueError(f"expected one registered name for {spec!r}, found {names!r}")
    return names[0]


def get_reference():
    """Return ``(name, module)`` of the single ``is_reference`` backend."""
    refs = [(n, m) for n, m in discover().items() if m.META.is_reference]
    if len(refs) != 1:
        raise ValueError(f"expected exactly one reference backend, found {len(refs)}")
    return refs[0]


def driver_for(meta):
    return importlib.import_module(_DRIVERS[meta.type])


def needs_compile(spec):
    driver = driver_for(spec.META)
    predicate = getattr(driver, "needs_compile", None)
    return bool(predicate(spec) if predicate else getattr(driver, "requires_compile", False))
