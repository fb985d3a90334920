"""Bounded host processes and the evidence of their runs (reference interface: etx/api/execution.py:1-82).  A
complete process is not device qualification."""
from __future__ import annotations

import math
from dataclasses import dataclass, field
from pathlib import Path

from .types import SCHEMA_VERSION, Configuration, digest

_HEX = set("0123456789abcdef")


def _is_digest(value) -> bool:
    return type(value) is str and len(value) == 64 and set(value) <= _HEX


@dataclass(frozen=True)
class ProcessRequest:
    argv: tuple[str, ...]
    cwd: str
    deadline_s: float
    environment: Configuration = field(default_factory=lambda: Configuration({}))
    silence_s: float = 30.0
    schema_version: int = SCHEMA_VERSION

    def __post_init__(self):
        if isinstance(self.argv, str) or not self.argv:
            raise ValueError("argv must be a nonempty sequence")
        argv = tuple(self.argv)
        if any(type(a) is not str or "\0" in a for a in argv):
            raise ValueError("argv holds strings without NUL")
        if not Path(argv[0]).is_absolute():
            raise ValueError("the executable path must be absolute")
        object.__setattr__(self, "argv", argv)
        if type(self.cwd) is not str or "\0" in self.cwd or not Path(self.cwd).is_absolute():
            raise ValueError("cwd must be an absolute path")
        for v in (self.deadline_s, self.silence_s):
            if type(v) not in (int, float) or not math.isfinite(v) or v <= 0:
                raise ValueError("deadline and silence are positive finite seconds")
        object.__setattr__(self, "environment", Configuration(self.environment))
        for k, v in self.environment.items():
            if not k or "=" in k or "\0" in k or type(v) is not str or "\0" in v:
                raise ValueError(f"environment entry {k!r} is not a valid string pair")
        if type(self.schema_version) is not int or self.schema_version != SCHEMA_VERSION:
            raise ValueError("process request schema version not supported")

    def to_dict(self) -> dict:
        return {"schema_version": self.schema_version, "argv": list(self.argv), "cwd": self.cwd,
                "deadline_s": self.deadline_s, "silence_s": self.silence_s,
                "environment": self.environment.to_dict()}

    @property
    def identity(self) -> str:
        return digest(self.to_dict())


_STATUSES = ("complete", "failed", "deadline", "interrupted", "error")


@dataclass(frozen=True)
class ProcessResult:
    request_identity: str
    backend: str
    status: str
    returncode: int | None
    output_sha256: str
    events: tuple[str, ...] = ()
    schema_version: int = SCHEMA_VERSION

    def __post_init__(self):
        if self.backend not in ("host-process", "scripted", "recorded"):
            raise ValueError("a process result comes from a host process, a script or a record, not a device")
        if self.status not in _STATUSES:
            raise ValueError(f"process status {self.status!r} is not one of {_STATUSES}")
        if self.returncode is not None and type(self.returncode) is not int:
            raise ValueError("return code must be an integer or None")
        if (self.status == "complete") != (self.returncode == 0):
            raise ValueError("a process is complete exactly when it exited with 0")
        if self.status == "deadline" and self.returncode != 124:
            raise ValueError("a process stopped at its deadline reports 124")
        if not (_is_digest(self.request_identity) and _is_digest(self.output_sha256)):
            raise ValueError("request identity and output digest are sha256 hex strings")
        if type(self.schema_version) is not int or self.schema_version != SCHEMA_VERSION:
            raise ValueError("process result schema version not supported")
        if isinstance(self.events, str) or any(type(e) is not str for e in self.events):
            raise ValueError("events are strings")
        object.__setattr__(self, "events", tuple(self.events))

    def to_dict(self) -> dict:
        return {"schema_version": self.schema_version, "request_identity": self.request_identity,
                "backend": self.backend, "status": self.status, "returncode": self.returncode,
                "output_sha256": self.output_sha256, "events": list(self.events)}
