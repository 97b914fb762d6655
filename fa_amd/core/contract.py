"""Backend metadata and the contracts the harness talks to.

Same two roles as the reference's plugin API (``core/contract.py:1-41``):

  * A *backend* is a module ``fa_amd/backends/<name>/backend.py`` exposing
    ``META`` plus the hooks its type requires. The registry keys backends by
    directory name.
  * A *driver* (``fa_amd/core/drivers/<type>.py``) turns a backend declaration
    into something runnable and builds it. The harness picks the driver by
    ``META.type``.

The harness (runner, bench) only ever uses ``META`` and the driver, so it is
backend-agnostic.

Backend module contract by type:
  type == "external": optional idempotent, CPU-safe ``build(case)``;
                      ``adapt(case, canonical) -> opaque op_args``;
                      ``call(op_args) -> canonical output``
                      (the reference's external type, ``core/drivers/external.py``)
  type == "hip"     : ``project(case) -> fa_amd.core.drivers.hip.Project``
                      ``load(case, project) -> built operator callable``, called
                      before any input exists;
                      ``adapt(case, canonical) -> positional args tuple``.
                      The MI355X counterpart of the reference's "ascendc"
                      project type (``core/drivers/ascendc.py:17-120``): a
                      hipcc-built shared library with a C ABI instead of a
                      CANN operator package.

Driver module contract:
  requires_compile: bool
  needs_compile(spec) -> bool              # optional per-backend override
  compile(spec, case) -> None
  prepare(spec, case) -> bind(canonical)   # optional early library loading
  make_call(spec, case, canonical) -> Callable[[], Tensor]   # one forward
"""

from dataclasses import dataclass


class KernelNameError(ValueError):
    """A backend violated the harness's device-kernel naming contract."""


@dataclass(frozen=True)
class Meta:
    name: str                    # legacy label; the registry keys backends by directory name
    type: str                    # "external" | "hip"
    op_type: str                 # fallback kernel-name filter for profiling, used when the
                                 # device kernel name does not contain the directory name
    is_reference: bool = False   # exactly one backend is the correctness reference
    author: str = ""
    date: str = ""
    notes: str = ""
    diagnostic: bool = False     # not an attention implementation; excluded from FA checks
