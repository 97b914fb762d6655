"""The plugin interface a backend implements to be run by the harness.

Interface kept identical to the reference's so a backend written for one
registers in the other (``core/contract.py:47-62`` there):

* ``Meta`` -- the module-level ``META`` record every backend declares. Its
  fields and defaults are the reference's: ``name`` (a legacy label; the
  catalog keys backends by their directory), ``type`` (which driver runs the
  backend), ``op_type`` (the substring that identifies the backend's device
  kernel in a profile when its directory name does not), ``is_reference``
  (exactly one backend is the correctness reference), ``author``, ``date``,
  ``notes`` and ``diagnostic`` (a module that is not an attention
  implementation and is never checked as one).
* ``KernelNameError`` -- raised when a backend breaks the rule that its
  device kernel can be recognised by name; the harness never swallows it.

What each ``type`` asks of a backend module is documented by the driver that
implements it (``fa_amd.harness.drivers``).
"""

from dataclasses import dataclass


class KernelNameError(ValueError):
    """A backend's device kernel cannot be attributed to it by name."""


@dataclass(frozen=True)
class Meta:
    name: str
    type: str
    op_type: str
    is_reference: bool = False
    author: str = ""
    date: str = ""
    notes: str = ""
    diagnostic: bool = False
