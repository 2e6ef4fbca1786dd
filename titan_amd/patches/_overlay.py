"""Shared machinery of the overlay patches (the ``install()`` contract of
engine/patches/moe-int8/patch.py:105-198 and
engine/patches/round3/gather-ws/patch.py:158-233).

An :class:`Overlay` replaces a namespace attribute (``gather_qmm`` or
``quantized_matmul`` of :mod:`titan_amd.core` by default) with a wrapper that
routes the calls its predicate accepts to a HIP path and hands everything
else, and every routed call that raises, to the implementation it found there.
The wrapper carries a marker attribute so a second ``install()`` is a no-op and
so a patch installed on top can see what is below it.  ``SwitchGLU.__call__``
is wrapped only to record the token count of the call in progress, for the
token floor.

One failure is never handed down: :class:`~titan_amd._lib.QmoeLibraryMissing`
(libqmoe not built or not loadable) propagates, so a deployment without the
native library fails loudly instead of running the stock path unnoticed.
"""

from __future__ import annotations

import logging
import os
from typing import Any, Callable

from .. import core
from .._lib import QmoeLibraryMissing, QmoeUnsupported

logger = logging.getLogger(__name__)


def switch_linears(model):
    """Every QuantizedSwitchLinear reachable from ``model``: the object itself,
    the values of containers, ``named_modules()`` when the object has it (the
    walk of engine/patches/moe-int8/patch.py:182-198), and object attributes,
    each object visited once.  Tensors, Python modules and classes are not
    entered."""
    import types

    import torch

    from ..switch_layers import QuantizedSwitchLinear

    leaves = (str, bytes, int, float, torch.Tensor, types.ModuleType, type)
    seen, out, stack = set(), [], [model]
    while stack:
        obj = stack.pop()
        if obj is None or id(obj) in seen or isinstance(obj, leaves):
            continue
        seen.add(id(obj))
        if isinstance(obj, QuantizedSwitchLinear):
            out.append(obj)
            continue
        if hasattr(obj, "named_modules") and callable(obj.named_modules):
            stack.extend(m for _, m in obj.named_modules() if m is not obj)
        if isinstance(obj, dict):
            stack.extend(obj.values())
        elif isinstance(obj, (list, tuple, set)):
            stack.extend(obj)
        elif hasattr(obj, "__dict__"):
            stack.extend(v for v in vars(obj).values() if not callable(v) or hasattr(v, "__dict__"))
    return out


def arg(args, kwargs, pos, name, default=None):
    """Argument ``name`` at position ``pos`` after (x, w) of the call."""
    if len(args) > pos:
        return args[pos]
    return kwargs.get(name, default)


class Overlay:
    """One overlay patch.

    ``targets`` maps a namespace attribute to ``(should_route, route)``:
    ``should_route(overlay, x, w, args, kwargs) -> bool`` and
    ``route(x, w, args, kwargs) -> tensor``.  ``self_check(fallbacks)`` runs at
    install time with the captured implementations and returns False to refuse
    the install (engine/patches/round2/wsum10/kernel.py:378-449).
    """

    def __init__(self, name: str, marker: str, env_enable: str, default_enabled: bool,
                 targets: dict[str, tuple[Callable, Callable]], env_min_tokens: str | None = None,
                 min_tokens_default: int = 0, env_min_rows: str | None = None, min_rows_default: int = 0,
                 self_check: Callable[[dict], bool] | None = None, extra_stats: tuple[str, ...] = ()):
        self.name, self.marker = name, marker
        self.env_enable, self.default_enabled = env_enable, default_enabled
        self.targets = targets
        self.env_min_tokens, self.min_tokens_default = env_min_tokens, min_tokens_default
        self.env_min_rows, self.min_rows_default = env_min_rows, min_rows_default
        self.self_check = self_check
        self.namespace: Any = None
        self.original: dict[str, Callable] = {}
        self._switchglu_original = None
        self.ctx: dict[str, Any] = {"tokens": None}
        self._stats = {"routed": 0, "fallback": 0, **{k: 0 for k in extra_stats}}

    # -- policy ---------------------------------------------------------
    def enabled(self) -> bool:
        return os.environ.get(self.env_enable, "1" if self.default_enabled else "0") == "1"

    def min_tokens(self) -> int:
        return int(os.environ.get(self.env_min_tokens, str(self.min_tokens_default))) if self.env_min_tokens \
            else self.min_tokens_default

    def min_rows(self) -> int:
        return int(os.environ.get(self.env_min_rows, str(self.min_rows_default))) if self.env_min_rows \
            else self.min_rows_default

    def below_floor(self, rows: int) -> bool:
        """The token floor when a SwitchGLU call is in progress, else the row floor."""
        tokens = self.ctx.get("tokens")
        if tokens is not None:
            return tokens < self.min_tokens()
        return rows < self.min_rows()

    def count(self, key: str) -> None:
        self._stats[key] = self._stats.get(key, 0) + 1

    # -- wrappers -------------------------------------------------------
    def _wrap(self, attr: str) -> Callable:
        should_route, route = self.targets[attr]

        def wrapper(x, w, *args, **kwargs):
            if should_route(self, x, w, args, kwargs):
                try:
                    out = route(x, w, args, kwargs)
                    self._stats["routed"] += 1
                    return out
                except QmoeLibraryMissing:
                    raise
                except QmoeUnsupported as exc:
                    logger.debug("%s: %s; handing down", self.name, exc)
                except Exception as exc:  # noqa: BLE001 - fall through, as the reference does
                    logger.warning("%s kernel failed, falling back: %s", self.name, exc)
            self._stats["fallback"] += 1
            return self.original[attr](x, w, *args, **kwargs)

        setattr(wrapper, self.marker, True)
        wrapper.__name__ = f"{self.name}_{attr}"
        wrapper.__doc__ = getattr(self.original.get(attr), "__doc__", None)
        return wrapper

    def _switchglu_call(self):
        original = self._switchglu_original
        ctx = self.ctx

        def call(glu, x, indices, *a, **kw):
            prev = ctx.get("tokens")
            try:
                ctx["tokens"] = int(indices.numel() // indices.shape[-1]) if indices.dim() else None
            except Exception:  # noqa: BLE001
                ctx["tokens"] = None
            try:
                return original(glu, x, indices, *a, **kw)
            finally:
                ctx["tokens"] = prev

        return call

    # -- the contract ---------------------------------------------------
    def install(self, namespace: Any = None) -> bool:
        """Idempotent; True when this call installed the hooks.  Runs the
        self-check against the captured implementations first and leaves
        everything untouched when it fails."""
        ns = core if namespace is None else namespace
        if self.namespace is not None:
            return False
        if all(getattr(getattr(ns, attr), self.marker, False) for attr in self.targets):
            return False
        found = {attr: getattr(ns, attr) for attr in self.targets}
        if self.self_check is not None and not self.self_check(found):
            logger.warning("%s: self-check failed; not installed", self.name)
            return False
        self.namespace = ns
        self.original = found
        for attr in self.targets:
            setattr(ns, attr, self._wrap(attr))
        from ..switch_layers import SwitchGLU

        if not getattr(SwitchGLU, self.marker, False):
            self._switchglu_original = SwitchGLU.__call__
            SwitchGLU.__call__ = self._switchglu_call()
            setattr(SwitchGLU, self.marker, True)
        logger.info("%s installed (enabled=%s)", self.name, self.enabled())
        return True

    def uninstall(self) -> None:
        if self.namespace is not None:
            for attr, fn in self.original.items():
                setattr(self.namespace, attr, fn)
            self.namespace = None
            self.original = {}
        if self._switchglu_original is not None:
            from ..switch_layers import SwitchGLU

            SwitchGLU.__call__ = self._switchglu_original
            setattr(SwitchGLU, self.marker, False)
            self._switchglu_original = None

    def fallback_of(self, attr: str) -> Callable | None:
        return self.original.get(attr)

    def stats(self) -> dict:
        return dict(self._stats)

    def reset_stats(self) -> None:
        for k in self._stats:
            self._stats[k] = 0
