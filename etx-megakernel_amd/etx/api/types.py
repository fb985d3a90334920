"""Declarations of the etx API surface the decode path is reached through: configurations, kernel and workload
declarations, plan requests and planned workloads.

The interface is the reference's (etx/api/types.py:28-186): the same class names, fields and defaults, the same
kinds of refusal (ValueError for bad values, TypeError for wrong types) and the same identity, the sha256 of the
record's canonical JSON (sorted keys, no whitespace, finite numbers only), so a declaration written against the
reference is accepted here unchanged and names the same workload.  The implementation is this package's own: a
Configuration is built by one validating canonicaliser and keeps only its canonical text.
"""
from __future__ import annotations

import hashlib
import json
import math
from collections.abc import Iterator, Mapping
from dataclasses import dataclass, field
from typing import Literal

SCHEMA_VERSION = 1

_ENCODER = json.JSONEncoder(sort_keys=True, separators=(",", ":"), allow_nan=False)


def _plain(value, where: str = "configuration"):
    """A JSON-ready copy of `value`: strings, booleans, integers, finite floats and None as they are, mappings with
    string keys as dicts, lists and tuples as lists.  Anything else is refused (ValueError)."""
    kind = type(value)
    if value is None or kind in (str, bool, int):
        return value
    if kind is float:
        if not math.isfinite(value):
            raise ValueError(f"{where}: {value!r} is not a finite number")
        return value
    if isinstance(value, Mapping):
        out = {}
        for key, item in value.items():
            if type(key) is not str:
                raise ValueError(f"{where}: key {key!r} is not a string")
            out[key] = _plain(item, f"{where}.{key}")
        return out
    if isinstance(value, (list, tuple)):
        return [_plain(item, f"{where}[{i}]") for i, item in enumerate(value)]
    raise ValueError(f"{where}: {kind.__name__} is not a JSON value")


def canonical(value) -> str:
    """The canonical JSON text of a JSON-ready value (the text every identity here hashes)."""
    return _ENCODER.encode(_plain(value))


def digest(value) -> str:
    return hashlib.sha256(canonical(value).encode()).hexdigest()


@dataclass(frozen=True, init=False)
class Configuration(Mapping):
    """An immutable JSON object.  Only the canonical text is stored; every read decodes a fresh copy, so callers
    can never reach the stored value."""
    _json: str

    def __init__(self, values: Mapping):
        if isinstance(values, Configuration):
            text = values._json
        elif isinstance(values, Mapping):
            text = canonical(values)
        else:
            raise ValueError("a configuration is built from a mapping")
        object.__setattr__(self, "_json", text)

    def to_dict(self) -> dict:
        return json.loads(self._json)

    def __getitem__(self, key):
        return self.to_dict()[key]

    def __iter__(self) -> Iterator[str]:
        return iter(self.to_dict())

    def __len__(self) -> int:
        return len(self.to_dict())


def _check_name(value) -> None:
    if not (type(value) is str and value and value == value.strip()):
        raise ValueError(f"name {value!r}: a nonempty string without surrounding blanks is required")


def _check_schema(value, what: str) -> None:
    if type(value) is not int or value != SCHEMA_VERSION:
        raise ValueError(f"{what}: schema version {value!r} is not supported (expected {SCHEMA_VERSION})")


_IMPLEMENTATIONS = ("graph", "imported", "native")
_KINDS = ("model",) + _IMPLEMENTATIONS


@dataclass(frozen=True)
class KernelSpec:
    name: str
    implementation: Literal["graph", "imported", "native"]
    config: Configuration

    def __post_init__(self):
        _check_name(self.name)
        if self.implementation not in _IMPLEMENTATIONS:
            raise ValueError(f"implementation {self.implementation!r} is not one of {_IMPLEMENTATIONS}")
        object.__setattr__(self, "config", Configuration(self.config))


@dataclass(frozen=True)
class WorkloadSpec:
    name: str
    kind: Literal["model", "graph", "imported", "native"]
    config: Configuration
    schema_version: int = SCHEMA_VERSION

    def __post_init__(self):
        _check_name(self.name)
        if self.kind not in _KINDS:
            raise ValueError(f"workload kind {self.kind!r} is not one of {_KINDS}")
        _check_schema(self.schema_version, "workload")
        object.__setattr__(self, "config", Configuration(self.config))

    def to_dict(self) -> dict:
        return {"schema_version": self.schema_version, "name": self.name, "kind": self.kind,
                "config": self.config.to_dict()}

    @classmethod
    def from_dict(cls, value: Mapping) -> "WorkloadSpec":
        keys = {"schema_version", "name", "kind", "config"}
        if not isinstance(value, Mapping) or set(value) != keys:
            raise ValueError(f"a workload record holds exactly {sorted(keys)}")
        return cls(name=value["name"], kind=value["kind"], config=value["config"],
                   schema_version=value["schema_version"])

    @property
    def identity(self) -> str:
        return digest(self.to_dict())


def _empty() -> Configuration:
    return Configuration({})


@dataclass(frozen=True)
class PlanRequest:
    """A workload to plan for a target, with integer shape bindings and runtime / planner options."""
    workload: WorkloadSpec
    target: str = "gfx942"
    bindings: Configuration = field(default_factory=_empty)
    runtime: Configuration = field(default_factory=_empty)
    options: Configuration = field(default_factory=_empty)

    def __post_init__(self):
        if not isinstance(self.workload, WorkloadSpec):
            raise TypeError("a plan request needs a WorkloadSpec")
        _check_name(self.target)
        for name in ("bindings", "runtime", "options"):
            object.__setattr__(self, name, Configuration(getattr(self, name)))
        for key, value in self.bindings.items():
            if type(value) is not int or value < 0:
                raise ValueError(f"binding {key!r} = {value!r}: bindings are nonnegative integers")

    def to_dict(self) -> dict:
        return {"workload": self.workload.to_dict(), "target": self.target, "bindings": self.bindings.to_dict(),
                "runtime": self.runtime.to_dict(), "options": self.options.to_dict()}


@dataclass(frozen=True)
class PlannedWorkload:
    """What the planner decided for a request: the machine it planned for, the options in force, a report and the
    decisions as lines.  A record, not an executable and not a correctness certificate."""
    request: PlanRequest
    machine: Configuration
    options: Configuration
    report: Configuration
    decisions: tuple[str, ...]
    schema_version: int = SCHEMA_VERSION

    def __post_init__(self):
        if not isinstance(self.request, PlanRequest):
            raise TypeError("a planned workload needs its PlanRequest")
        _check_schema(self.schema_version, "planned workload")
        for name in ("machine", "options", "report"):
            object.__setattr__(self, name, Configuration(getattr(self, name)))
        lines = tuple(self.decisions)
        if any(type(line) is not str for line in lines):
            raise ValueError("decisions are lines of text")
        object.__setattr__(self, "decisions", lines)

    def to_dict(self) -> dict:
        return {"schema_version": self.schema_version, "request": self.request.to_dict(),
                "machine": self.machine.to_dict(), "options": self.options.to_dict(),
                "report": self.report.to_dict(), "decisions": list(self.decisions)}

    @classmethod
    def from_dict(cls, value: Mapping) -> "PlannedWorkload":
        keys = {"schema_version", "request", "machine", "options", "report", "decisions"}
        if not isinstance(value, Mapping) or set(value) != keys:
            raise ValueError(f"a planned-workload record holds exactly {sorted(keys)}")
        req = dict(value["request"])
        req["workload"] = WorkloadSpec.from_dict(req["workload"])
        return cls(request=PlanRequest(**req), machine=value["machine"], options=value["options"],
                   report=value["report"], decisions=tuple(value["decisions"]),
                   schema_version=value["schema_version"])

    @property
    def identity(self) -> str:
        return digest(self.to_dict())


@dataclass(frozen=True)
class Inspection:
    schema_version: int
    identity: str
    declaration: WorkloadSpec
    status: Literal["DECLARED"] = "DECLARED"
