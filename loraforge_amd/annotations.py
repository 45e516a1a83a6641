"""Metadata-only stability marker, mirroring ``loraforge.annotations.ExperimentalAPI``.

Reference: ``src/loraforge/annotations.py:29-86``. The marker attaches an
``ExperimentalInfo`` record as ``__experimental_api__`` and appends a note to the
docstring; it never wraps the decorated callable, so numerical operators gain
no per-call overhead.
"""

from __future__ import annotations

from dataclasses import dataclass
from typing import Callable, TypeVar

F = TypeVar("F", bound=Callable)


@dataclass(frozen=True)
class ExperimentalInfo:
    reason: str
    since: str
    stability: str = "alpha"


def ExperimentalAPI(*, reason: str, since: str = "0.1.0.dev0") -> Callable[[F], F]:
    if not isinstance(reason, str) or not reason.strip():
        raise ValueError("reason must be a nonempty description")
    if not isinstance(since, str) or not since.strip():
        raise ValueError("since must be a nonempty version string")
    info = ExperimentalInfo(reason=reason, since=since)

    def mark(obj: F) -> F:
        if not callable(obj):
            raise TypeError("ExperimentalAPI requires a callable")
        obj.__experimental_api__ = info
        obj.__doc__ = (obj.__doc__ or "") + (
            f"\n\nExperimental API (alpha, since {since}). {reason} API compatibility is not guaranteed."
        )
        return obj

    return mark
