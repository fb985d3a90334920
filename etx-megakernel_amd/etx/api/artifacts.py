"""Source artifacts: the emitted files of a planned workload (reference interface: etx/api/artifacts.py:1-62).

A SourceArtifact is text payloads by relative path plus, per rank (device), the payload that describes that rank's
launch and the header a C/C++ host includes.  For the native decode path a rank's source is its launch record
(rank<r>.json: the library symbol, the etxmk_config, the grid) and its header declares the same configuration as a
C initializer (rank<r>.h).  Sources are not builds: status is always 'SOURCES'."""
from __future__ import annotations

import hashlib
from dataclasses import dataclass
from pathlib import PurePosixPath

from .types import SCHEMA_VERSION, Configuration, PlannedWorkload, digest


def payload_path(value) -> str:
    """A payload name: a normalized relative POSIX path, not the reserved manifest name."""
    if type(value) is not str or not value or "\\" in value or "\0" in value:
        raise ValueError(f"payload path {value!r} is not a plain relative path")
    parts = value.split("/")
    if PurePosixPath(value).is_absolute() or any(p in ("", ".", "..") for p in parts):
        raise ValueError(f"payload path {value!r} must be normalized and relative")
    if value == "manifest.json":
        raise ValueError("manifest.json is reserved for the artifact's manifest")
    return value


def _names(values, what: str) -> tuple:
    if isinstance(values, str) or any(type(v) is not str for v in values):
        raise ValueError(f"{what}: a sequence of payload names is required")
    return tuple(values)


@dataclass(frozen=True)
class SourceArtifact:
    planned: PlannedWorkload
    files: Configuration
    rank_sources: tuple[str, ...]
    rank_headers: tuple[str, ...]
    external_sources: tuple[str, ...] = ()
    status: str = "SOURCES"
    schema_version: int = SCHEMA_VERSION

    def __post_init__(self):
        if not isinstance(self.planned, PlannedWorkload):
            raise TypeError("a source artifact belongs to a PlannedWorkload")
        if self.status != "SOURCES":
            raise ValueError("a source artifact is sources only (status 'SOURCES')")
        if type(self.schema_version) is not int or self.schema_version != SCHEMA_VERSION:
            raise ValueError("source artifact schema version not supported")
        object.__setattr__(self, "files", Configuration(self.files))
        for name, text in self.files.items():
            payload_path(name)
            if type(text) is not str:
                raise ValueError(f"payload {name!r} is not text")
        for what in ("rank_sources", "rank_headers", "external_sources"):
            object.__setattr__(self, what, _names(getattr(self, what), what))
        ranks = self.planned.report["devices"]
        for what, names in (("rank_sources", self.rank_sources), ("rank_headers", self.rank_headers)):
            if len(names) != ranks or len(set(names)) != ranks or not all(n in self.files for n in names):
                raise ValueError(f"{what}: one distinct payload per rank ({ranks}) is required")
        if set(self.rank_sources) & set(self.rank_headers):
            raise ValueError("a payload cannot be both a rank source and a rank header")

    def manifest(self) -> dict:
        return {"schema_version": self.schema_version, "status": self.status, "planned": self.planned.to_dict(),
                "rank_sources": list(self.rank_sources), "rank_headers": list(self.rank_headers),
                "external_sources": list(self.external_sources),
                "payloads": {n: hashlib.sha256(t.encode()).hexdigest() for n, t in self.files.items()}}

    @property
    def identity(self) -> str:
        return digest(self.manifest())
