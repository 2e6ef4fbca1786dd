"""Errors raised deliberately by the host side (titan/core/errors.py:28-40).

The C-ABI errors live in :mod:`titan_amd._lib` (``QmoeError`` and its
subclasses); these two are the registry's.
"""


class TitanError(Exception):
    """Base class for everything this package raises deliberately."""


class ConfigError(TitanError):
    """A configuration names something that does not exist or cannot be used."""


class KernelError(TitanError):
    """A fast path failed and the registry was told not to fall back."""
