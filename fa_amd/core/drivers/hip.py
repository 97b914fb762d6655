"""HIP shared-library project driver.

The MI355X counterpart of the reference's standard-project driver
(``core/drivers/ascendc.py:1-120``): a backend declares a ``Project`` recipe
(HIP sources under ``csrc/``, an argv build command, the artifacts it must
produce), the driver validates the recipe, runs the build under an exclusive
``flock`` so concurrent workers never race on one build directory, checks that
every declared artifact exists, and only then loads the library. ``prepare``
loads the library before any input tensor exists; ``bind(canonical)`` adapts
the inputs and returns the zero-argument call.
"""

from contextlib import contextmanager
from dataclasses import dataclass
import fcntl
from pathlib import Path
import subprocess

requires_compile = True


@dataclass(frozen=True)
class Project:
    """Explicit HIP project recipe; commands are argv tuples, never shell strings.

    An empty ``build_command`` means "use the already-built artifacts".
    Build commands must be CPU-safe (hipcc cross-compiles gfx950 without a
    GPU) and idempotent.
    """

    root: Path
    artifacts: tuple
    build_command: tuple = ()
    timeout_seconds: float = 600

    def validate(self):
        root = Path(self.root).resolve()
        csrc = root / "csrc"
        if not csrc.is_dir() or not any(p.is_file() and p.suffix == ".hip" for p in csrc.rglob("*")):
            raise ValueError(f"HIP project needs csrc/*.hip sources: {root}")
        if not isinstance(self.build_command, tuple) or any(
            not isinstance(arg, str) or not arg for arg in self.build_command
        ):
            raise TypeError("build_command must be a tuple of nonempty argv strings")
        if not isinstance(self.artifacts, tuple) or not self.artifacts:
            raise ValueError("HIP project must declare its build artifacts")
        for item in self.artifacts:
            if not isinstance(item, str) or not item or Path(item).is_absolute():
                raise ValueError("artifacts must be nonempty project-relative paths")
            if not (root / item).resolve().is_relative_to(root):
                raise ValueError(f"artifact escapes project root: {item}")
        if self.timeout_seconds <= 0:
            raise ValueError("timeout_seconds must be positive")
        return root

    def artifact_paths(self):
        root = self.validate()
        return tuple(root / item for item in self.artifacts)


def _project(spec, case):
    for method in ("project", "load", "adapt"):
        if not callable(getattr(spec, method, None)):
            raise TypeError(
                f"hip backend requires {method}(); generic adapt/call backends "
                'must use type="external"'
            )
    project = spec.project(case)
    if not isinstance(project, Project):
        raise TypeError("project(case) must return fa_amd.core.drivers.hip.Project")
    project.validate()
    return project


@contextmanager
def _prepared(spec, case):
    project = _project(spec, case)
    root = Path(project.root).resolve()
    with (root / ".fa_hip.lock").open("a") as lock:
        fcntl.flock(lock, fcntl.LOCK_EX)
        if project.build_command:
            with (root / ".fa_hip_build.log").open("w") as log:
                subprocess.run(
                    list(project.build_command),
                    cwd=root,
                    stdout=log,
                    stderr=log,
                    check=True,
                    timeout=project.timeout_seconds,
                )
        missing = [str(p) for p in project.artifact_paths() if not p.is_file()]
        if missing:
            raise FileNotFoundError(f"HIP build artifacts missing: {missing}")
        yield project


def compile(spec, case):
    with _prepared(spec, case):
        pass


def prepare(spec, case):
    """Load the shared library before canonical inputs touch the device."""
    with _prepared(spec, case) as project:
        operator = spec.load(case, project)
    if not callable(operator):
        raise TypeError("load(case, project) must return the built operator's callable binding")

    def bind(canonical):
        op_args = spec.adapt(case, canonical)
        if not isinstance(op_args, tuple):
            raise TypeError("hip adapt(case, canonical) must return a positional-argument tuple")
        return lambda: operator(*op_args)

    return bind


def make_call(spec, case, canonical):
    return prepare(spec, case)(canonical)
