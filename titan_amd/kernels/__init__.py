"""The call sites' one door to the ops (titan/adapters/mlx/kernels.py:33-160).

A call site asks by its own dotted name and uses what comes back only if
something comes back: ``None`` means "no kernel for this site" and the site
keeps its stock path.  ``ADAPTER_OPS`` maps the site names to the registry's
op names.
"""

from __future__ import annotations

import logging
import threading
from typing import Any, Callable, Optional

logger = logging.getLogger(__name__)

ADAPTER_OPS: dict[str, str | None] = {
    "moe.weighted_sum": "moe_weighted_sum",
    "moe.gather_qmm_ws": "moe_gather_ws",
    "moe.gather_qmm_int8": "moe_gather_int8",
}

_lock = threading.Lock()
_registry: Any = None
_resolved: dict[str, Optional[Callable[..., Any]]] = {}


def _get_registry():
    global _registry
    if _registry is not None:
        return _registry
    with _lock:
        if _registry is None:
            from . import registry as registry_module

            _registry = registry_module.current() or registry_module.build_registry()
        return _registry


def reset() -> None:
    """Forget the registry and every resolution (tests and A/B arms)."""
    global _registry
    with _lock:
        _registry = None
        _resolved.clear()


def get(name: str) -> Optional[Callable[..., Any]]:
    """The dispatcher for a call-site name, or None when the configuration
    turned the op off (kernels.py:140-160)."""
    if name in _resolved:
        return _resolved[name]
    registry = _get_registry()
    op_name = ADAPTER_OPS.get(name)
    if name not in ADAPTER_OPS:
        logger.warning("unknown call-site op %s", name)
    op = None
    if op_name is not None and not registry.fast_disabled(op_name):
        op = registry.resolve(op_name)
    _resolved[name] = op
    return op
