"""Drivers: how the harness turns a backend module into one callable forward.

A backend's ``META.type`` names its driver. Every driver answers three
questions about a backend module:

* ``needs_build(module)`` -- does running it require a compile step first?
* ``build(module, case)`` -- run that step. CPU only (no device is touched),
  idempotent, safe to call again.
* ``prepare(module, case)`` -- do everything that does not need the inputs
  (build, load libraries) and return ``bind``; ``bind(canonical)`` maps the
  canonical input tensors to the backend's arguments and returns a
  zero-argument callable that runs one forward and returns the output tensor.

Loading happens in ``prepare``, before the harness draws any input, so a
library's device-side setup never competes with (or gets timed alongside)
the inputs; ``bind`` only adapts arguments.

Backend types:

``"external"`` -- the reference's generic contract, unchanged, so a backend
    written for the reference runs here as is: an optional ``build(case)``
    (CPU-safe, idempotent), ``adapt(case, canonical)`` returning an opaque
    argument object, and ``call(op_args)`` returning the output.

``"hip"`` -- a backend over this package's ``libfa_hip.so``: ``operator(case)``
    returns a callable ``(q, k, v) -> o`` with the library already loaded,
    ``adapt(case, canonical)`` returns the positional tuple it is called with.
    The shared library is the only build product; its content-hashed build
    (``fa_amd.build``) is brought up to date before the operator is created.
"""

from __future__ import annotations


class UnknownBackendType(KeyError):
    """``META.type`` names no driver."""


class ExternalDriver:
    kind = "external"

    def needs_build(self, module) -> bool:
        return callable(getattr(module, "build", None))

    def build(self, module, case) -> None:
        hook = getattr(module, "build", None)
        if hook is None:
            return
        if not callable(hook):
            raise TypeError(f"{module.__name__}.build must be callable")
        hook(case)

    def prepare(self, module, case):
        self.build(module, case)

        def bind(canonical):
            op_args = module.adapt(case, canonical)
            return lambda: module.call(op_args)

        return bind


class HipDriver:
    kind = "hip"

    REQUIRED = ("operator", "adapt")

    def needs_build(self, module) -> bool:
        return True

    def _check(self, module):
        missing = [hook for hook in self.REQUIRED if not callable(getattr(module, hook, None))]
        if missing:
            raise TypeError(f"{module.__name__}: a hip backend defines operator() and adapt(); "
                            f"missing {', '.join(missing)}")

    def build(self, module, case) -> None:
        self._check(module)
        from fa_amd import build

        build.build()

    def prepare(self, module, case):
        self.build(module, case)
        forward = module.operator(case)
        if not callable(forward):
            raise TypeError(f"{module.__name__}.operator(case) must return a callable")

        def bind(canonical):
            args = module.adapt(case, canonical)
            if not isinstance(args, tuple):
                raise TypeError(f"{module.__name__}.adapt must return a tuple of arguments")
            return lambda: forward(*args)

        return bind


DRIVERS = {driver.kind: driver for driver in (ExternalDriver(), HipDriver())}


def driver(kind: str):
    """The driver object for a ``META.type``."""
    try:
        return DRIVERS[kind]
    except KeyError:
        raise UnknownBackendType(f"no driver for backend type {kind!r} "
                                 f"(known: {', '.join(sorted(DRIVERS))})") from None
