"""Model build requests (reference interface: etx/api/models.py:1-50): plan a kind='model' workload and produce the
executable that runs it.  The native decode provider ('native') links nothing: its executable is a launcher over the
prebuilt gfx950 library."""
from __future__ import annotations

from dataclasses import dataclass, field
from pathlib import Path

from .types import SCHEMA_VERSION, Configuration, PlanRequest


class BuildRefused(ValueError):
    """The requested build variant is refused before anything is created."""


def _absolute(value, what: str) -> None:
    if type(value) is not str or "\0" in value or not Path(value).is_absolute():
        raise ValueError(f"{what} {value!r}: an absolute path is required")


def _strings(values, what: str) -> tuple:
    if isinstance(values, str) or any(type(v) is not str or "\0" in v for v in values):
        raise ValueError(f"{what}: a sequence of strings is required")
    return tuple(values)


@dataclass(frozen=True)
class ModelBuildRequest:
    plan: PlanRequest              # a kind='model' workload, its target and planner options
    root: str                      # repository the build runs in
    output: str                    # directory receiving the emitted files and the executable `run`
    host: str                      # host translation unit (the reference links one; the native provider only checks it exists)
    flags: tuple[str, ...] = ()
    includes: tuple[str, ...] = ()
    resource_usage: bool = False
    compiler: str = "hipcc"
    deadline_s: float = 1800.0
    extra_sources: tuple[str, ...] = ()
    provider: str = "host-link"
    variant: Configuration = field(default_factory=lambda: Configuration({}))
    schema_version: int = SCHEMA_VERSION

    def __post_init__(self):
        if not isinstance(self.plan, PlanRequest) or self.plan.workload.kind != "model":
            raise ValueError("a model build needs a PlanRequest of a kind='model' workload")
        for what in ("root", "output", "host"):
            _absolute(getattr(self, what), what)
        object.__setattr__(self, "variant", Configuration(self.variant))
        if type(self.provider) is not str or not self.provider:
            raise ValueError("provider must be a nonempty name")
        for what in ("flags", "includes", "extra_sources"):
            object.__setattr__(self, what, _strings(getattr(self, what), what))
        for path in self.includes:
            _absolute(path, "include directory")
        if type(self.compiler) is not str or not self.compiler or self.compiler.startswith("-"):
            raise ValueError("compiler must name an executable or docker:<image>")
        if type(self.deadline_s) not in (int, float) or not self.deadline_s > 0:
            raise ValueError("deadline must be a positive number of seconds")
        if type(self.schema_version) is not int or self.schema_version != SCHEMA_VERSION:
            raise ValueError("model build schema version not supported")
