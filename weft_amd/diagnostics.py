"""Public error hierarchy, named as the reference's (python/weft/diagnostics.py)."""
from __future__ import annotations


class WeftError(Exception):
    """Base class for public errors."""


class DefinitionError(WeftError):
    """A kernel definition is malformed."""


class LanguageUseError(WeftError):
    """A kernel definition was called as a Python function."""
