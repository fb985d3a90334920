"""Runs of a built model artifact (reference interface: etx/api/runs.py:1-68): the request names the build by
directory and identity; the run record pairs it with the process evidence."""
from __future__ import annotations

from dataclasses import dataclass, field
from pathlib import Path

from .execution import ProcessRequest, ProcessResult
from .types import SCHEMA_VERSION, Configuration, digest


@dataclass(frozen=True)
class ArtifactRunRequest:
    directory: str
    build_identity: str
    cwd: str
    deadline_s: float
    arguments: tuple[str, ...] = ()
    environment: Configuration = field(default_factory=lambda: Configuration({}))
    silence_s: float = 30.0
    schema_version: int = SCHEMA_VERSION

    def __post_init__(self):
        if type(self.directory) is not str or "\0" in self.directory or not Path(self.directory).is_absolute():
            raise ValueError("the artifact directory must be an absolute path")
        ident = self.build_identity
        if type(ident) is not str or len(ident) != 64 or not set(ident) <= set("0123456789abcdef"):
            raise ValueError("build identity must be a sha256 hex string")
        if isinstance(self.arguments, str):
            raise ValueError("arguments must be a sequence of strings")
        object.__setattr__(self, "arguments", tuple(self.arguments))
        object.__setattr__(self, "environment", Configuration(self.environment))
        self.process_request()                             # the process request's own checks apply

    def process_request(self) -> ProcessRequest:
        return ProcessRequest((str(Path(self.directory) / "run"), *self.arguments), self.cwd, self.deadline_s,
                              self.environment, self.silence_s, self.schema_version)

    def to_dict(self) -> dict:
        return {"schema_version": self.schema_version, "directory": self.directory,
                "build_identity": self.build_identity, "cwd": self.cwd, "deadline_s": self.deadline_s,
                "arguments": list(self.arguments), "environment": self.environment.to_dict(),
                "silence_s": self.silence_s}

    @property
    def identity(self) -> str:
        return digest(self.to_dict())


@dataclass(frozen=True)
class ArtifactRun:
    request: ArtifactRunRequest
    process: ProcessResult
    schema_version: int = SCHEMA_VERSION

    def __post_init__(self):
        if not isinstance(self.request, ArtifactRunRequest) or not isinstance(self.process, ProcessResult):
            raise TypeError("an artifact run pairs an ArtifactRunRequest with a ProcessResult")
        if self.process.request_identity != self.request.process_request().identity:
            raise ValueError("the process evidence belongs to another request")
        if type(self.schema_version) is not int or self.schema_version != SCHEMA_VERSION:
            raise ValueError("artifact run schema version not supported")

    def to_dict(self) -> dict:
        return {"schema_version": self.schema_version, "request": self.request.to_dict(),
                "process": self.process.to_dict()}

    @property
    def identity(self) -> str:
        return digest(self.to_dict())
