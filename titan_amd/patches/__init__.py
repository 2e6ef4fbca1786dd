"""Overlay patches that reroute :mod:`titan_amd.core` to the HIP kernels.

``install()`` installs all three in the order that makes the precedence rules
hold: the decode GEMV overlay at the bottom, the int8 prefill overlay above it,
the bf16 prefill overlay on top (it hands calls down to int8 when int8 is
enabled).  Each module also installs on its own, like the reference's overlays
(engine/bootstrap/bootstrap.py:14-20).
"""

from __future__ import annotations

from . import gather_qmv, gather_ws, moe_int8

__all__ = ["gather_qmv", "gather_ws", "moe_int8", "install", "uninstall", "stats"]

_ORDER = (gather_qmv, moe_int8, gather_ws)


def install(namespace=None) -> bool:
    """Install every overlay; True when any of them was installed now."""
    done = [m.install(namespace) for m in _ORDER]
    return any(done)


def uninstall() -> None:
    for m in reversed(_ORDER):
        m.uninstall()


def stats() -> dict:
    return {m.__name__.rsplit(".", 1)[-1]: m.stats() for m in _ORDER}
