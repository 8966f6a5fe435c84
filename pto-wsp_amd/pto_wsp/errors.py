"""Exceptions (``python/pto_wsp/errors.py`` in the reference)."""

from __future__ import annotations


class PtoError(Exception):
    """Base class for PTO-WSP errors."""


class CompileError(PtoError):
    """Raised when a workload cannot be lowered or built for the requested target
    (the reference wraps codegen failures the same way, ``program.py:434-435``)."""

    def __init__(self, message: str, kernel: str | None = None) -> None:
        super().__init__(message)
        self.kernel = kernel


class ExecutionError(PtoError):
    """Raised by ``Program.synchronize()`` when a device run failed.

    The reference has no run-time error channel (an exception in its execute
    thread is dropped); this backend reports device errors instead.
    """


class IRBridgeError(PtoError):
    """Raised when a Python workload cannot be converted to the codegen module."""
