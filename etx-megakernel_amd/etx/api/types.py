"""Versioned declarations of the etx API surface the decode path is reached through.

Mirrors etx/api/types.py of the reference (Configuration :28-48, KernelSpec :56-66, WorkloadSpec :69-98):
same field names, same validation and the same errors (ValueError / TypeError), so a declaration written
against the reference is accepted here unchanged.
"""
from __future__ import annotations

import hashlib
import json
import math
from collections.abc import Iterator, Mapping
from dataclasses import dataclass
from typing import Literal

SCHEMA_VERSION = 1


def _json_value(value):
    if value is None or type(value) in (str, bool, int):
        return value
    if type(value) is float and math.isfinite(value):
        return value
    if isinstance(value, Mapping):
        if any(type(k) is not str for k in value):
            raise ValueError("configuration keys must be strings")
        return {k: _json_value(v) for k, v in value.items()}
    if isinstance(value, (list, tuple)):
        return [_json_value(v) for v in value]
    raise ValueError(f"configuration requires finite JSON values, got {type(value).__name__}")


@dataclass(frozen=True, init=False)
class Configuration(Mapping):
    """Immutable JSON value store; containers handed out are detached copies."""
    _json: str

    def __init__(self, values: Mapping):
        if not isinstance(values, Mapping):
            raise ValueError("configuration must be a mapping")
        object.__setattr__(self, "_json", json.dumps(_json_value(values), sort_keys=True, separators=(",", ":"),
                                                     allow_nan=False))

    def to_dict(self) -> dict:
        return json.loads(self._json)

    def __getitem__(self, key):
        return self.to_dict()[key]

    def __iter__(self) -> Iterator[str]:
        return iter(self.to_dict())

    def __len__(self) -> int:
        return len(self.to_dict())


def _name(value: str):
    if type(value) is not str or not value or value != value.strip():
        raise ValueError("name must be a nonempty string without surrounding whitespace")


@dataclass(frozen=True)
class KernelSpec:
    name: str
    implementation: Literal["graph", "imported", "native"]
    config: Configuration

    def __post_init__(self):
        _name(self.name)
        if self.implementation not in ("graph", "imported", "native"):
            raise ValueError("unknown kernel implementation")
        object.__setattr__(self, "config", Configuration(self.config))


@dataclass(frozen=True)
class WorkloadSpec:
    name: str
    kind: Literal["model", "graph", "imported", "native"]
    config: Configuration
    schema_version: int = SCHEMA_VERSION

    def __post_init__(self):
        _name(self.name)
        if self.kind not in ("model", "graph", "imported", "native"):
            raise ValueError("unknown workload kind")
        if type(self.schema_version) is not int or self.schema_version != SCHEMA_VERSION:
            raise ValueError("unsupported workload schema")
        object.__setattr__(self, "config", Configuration(self.config))

    def to_dict(self) -> dict:
        return dict(schema_version=self.schema_version, name=self.name, kind=self.kind, config=self.config.to_dict())

    @classmethod
    def from_dict(cls, value: Mapping) -> "WorkloadSpec":
        if not isinstance(value, Mapping) or set(value) != {"schema_version", "name", "kind", "config"}:
            raise ValueError("workload record requires exactly schema_version/name/kind/config")
        return cls(**value)

    @property
    def identity(self) -> str:
        encoded = json.dumps(self.to_dict(), sort_keys=True, separators=(",", ":"), allow_nan=False)
        return hashlib.sha256(encoded.encode()).hexdigest()
