"""Exceptions, as in the reference's errors module (src/economize/errors.py:24-96): configuration problems raise
:class:`ConfigError`, a ``ValueError``, before any kernel launches."""

from __future__ import annotations

__all__ = ["ConfigError", "EconomizeError", "IncompatibleTechniquesError"]


class EconomizeError(Exception):
    """Base class of the package's errors."""


class ConfigError(EconomizeError, ValueError):
    """An argument, shape, dtype or layout the kernels do not take (errors.py:28)."""


class IncompatibleTechniquesError(EconomizeError):
    """Techniques or attention implementations that cannot run together."""
