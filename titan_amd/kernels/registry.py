"""Op registry for the quantized MoE path (titan/kernels/registry.py).

Every op is a :class:`KernelOp`: a name, a reference implementation (plain
torch ops, the stock semantics), a fast implementation (the HIP kernels behind
libqmoe), a ``key`` deriving the call's :class:`ShapeClass`, a ``supports``
predicate over that class and the exactness class the pair is held to
(registry.py:132-185).

Selection happens once per (op, shape class, phase) and is memoised, so the
hot path is a dict lookup (registry.py:250-264).  The dispatcher returned by
:meth:`KernelRegistry.resolve` counts calls, and when ``fail_open`` a fast path
that raises is counted and answered by the reference (registry.py:297-320).
One exception is never swallowed: :class:`~titan_amd._lib.QmoeLibraryMissing`.
A missing or unloadable libqmoe is a deployment error, and answering it with
the reference would hide that the native path never ran.

The phase flag (registry.py:56-85) is a module global: the model loop is
single-threaded by construction.
"""

from __future__ import annotations

from contextlib import contextmanager
from dataclasses import dataclass, field
from typing import Any, Callable, Iterator, Mapping, Sequence

import torch

from .._lib import QmoeLibraryMissing
from ..errors import ConfigError, KernelError

__all__ = [
    "KernelConfig", "KernelOp", "KernelRegistry", "ShapeClass", "build_registry", "current",
    "phase", "reference_only", "set_current", "set_phase", "shape_class",
]


@dataclass(frozen=True)
class KernelConfig:
    """The ``kernels`` policy (titan/config/schema.py:370-390)."""

    enabled: tuple[str, ...] = ()      # empty: every op's default
    disabled: tuple[str, ...] = ()     # forced to the reference
    reference_only: bool = False
    fail_open: bool = True
    prefill_only: tuple[str, ...] = ()


# ------------------------------------------------------------------ phase

_PHASE = "decode"


def set_phase(name: str) -> str:
    """Set the current phase; returns the previous one (registry.py:69-73)."""
    global _PHASE
    previous, _PHASE = _PHASE, str(name)
    return previous


def get_phase() -> str:
    return _PHASE


@contextmanager
def phase(name: str) -> Iterator[None]:
    """Run a block in ``name`` phase and restore the previous one."""
    previous = set_phase(name)
    try:
        yield
    finally:
        set_phase(previous)


# ------------------------------------------------------------ shape class


@dataclass(frozen=True)
class ShapeClass:
    """What selection may depend on (registry.py:93-105): operand shapes and
    dtypes, the device kind (``"gpu"`` for ROCm tensors, else ``"cpu"``) and
    any non-tensor discriminator."""

    shapes: tuple[tuple[int, ...], ...] = ()
    dtypes: tuple[Any, ...] = ()
    device: str = "gpu"
    extra: tuple[Any, ...] = ()


def _device_kind(tensors) -> str:
    return "gpu" if tensors and all(t.is_cuda for t in tensors) else "cpu"


def shape_class(*tensors, extra: Sequence[Any] = (), device: str | None = None) -> ShapeClass:
    """A :class:`ShapeClass` from tensor operands (``None`` entries skipped)."""
    live = [t for t in tensors if t is not None]
    return ShapeClass(
        shapes=tuple(tuple(t.shape) for t in live),
        dtypes=tuple(t.dtype for t in live),
        device=device if device is not None else _device_kind(live),
        extra=tuple(extra),
    )


# --------------------------------------------------------------------- op


@dataclass
class KernelOp:
    """One op (registry.py:132-185).  ``tolerance`` 0.0 means bit-identical to
    the reference; otherwise it is the bound the op's exactness test states."""

    name: str
    reference_fn: Callable[..., Any]
    key: Callable[..., ShapeClass]
    fast_fn: Callable[..., Any] | None = None
    supports_key: Callable[[ShapeClass], bool] = lambda _k: False
    tolerance: float = 0.0
    shapes: tuple[Mapping[str, int], ...] = ()
    exactness: str = "unspecified"
    source: str = ""
    aliases: tuple[str, ...] = ()
    default_off: bool = False
    default_off_reason: str = ""

    def reference(self, *args: Any, **kwargs: Any) -> Any:
        return self.reference_fn(*args, **kwargs)

    def fast(self, *args: Any, **kwargs: Any) -> Any:
        if self.fast_fn is None:
            raise KernelError(f"op {self.name!r} has no fast implementation")
        return self.fast_fn(*args, **kwargs)

    def supports(self, *args: Any, **kwargs: Any) -> bool:
        if self.fast_fn is None:
            return False
        return self.supports_key(self.key(*args, **kwargs))

    @property
    def has_fast(self) -> bool:
        return self.fast_fn is not None


# --------------------------------------------------------------- registry

_FAST = "fast"
_REFERENCE = "reference"


class KernelRegistry:
    """Name -> :class:`KernelOp`, plus the selection memo and counters."""

    def __init__(self, config: KernelConfig | None = None) -> None:
        self.config = config or KernelConfig()
        self._ops: dict[str, KernelOp] = {}
        self._memo: dict[tuple, str] = {}
        self._calls: dict[str, int] = {}
        self._fast_calls: dict[str, int] = {}
        self._fallbacks: dict[str, int] = {}

    def register(self, op: KernelOp) -> None:
        for name in (op.name, *op.aliases):
            existing = self._ops.get(name)
            if existing is not None and existing is not op:
                raise ConfigError(f"op name {name!r} is registered twice")
            self._ops[name] = op

    def get(self, name: str) -> KernelOp:
        try:
            return self._ops[name]
        except KeyError:
            raise ConfigError(f"unknown kernel op {name!r} (known ops: {', '.join(self.names())})") from None

    def names(self) -> tuple[str, ...]:
        return tuple(sorted({op.name for op in self._ops.values()}))

    def validate(self) -> None:
        """Reject a configuration naming an op that does not exist (registry.py:209-216)."""
        for name in (*self.config.disabled, *self.config.enabled, *self.config.prefill_only):
            if name not in self._ops:
                raise ConfigError(f"the kernel configuration lists {name!r}, but no op of that name exists")

    def _fast_allowed(self, op: KernelOp) -> bool:
        """registry.py:219-243: disabled wins, ``enabled`` is an allowlist,
        default-off ops run only when named, prefill-only ops only in prefill."""
        if not op.has_fast or self.config.reference_only:
            return False
        names = {op.name, *op.aliases}
        if names & set(self.config.disabled):
            return False
        asked_for = bool(names & set(self.config.enabled))
        if self.config.enabled and not asked_for:
            return False
        if op.default_off and not asked_for:
            return False
        if names & set(self.config.prefill_only) and _PHASE != "prefill":
            return False
        return True

    def defaults(self) -> Mapping[str, bool]:
        return {name: not self._ops[name].default_off for name in self.names()}

    def fast_disabled(self, name: str) -> bool:
        return not self._fast_allowed(self.get(name))

    def selection(self, name: str, key: ShapeClass) -> str:
        op = self.get(name)
        memo_key = (op.name, key, _PHASE if self.config.prefill_only else "")
        hit = self._memo.get(memo_key)
        if hit is None:
            hit = _FAST if self._fast_allowed(op) and op.supports_key(key) else _REFERENCE
            self._memo[memo_key] = hit
        return hit

    def selections(self) -> Mapping[tuple, str]:
        return dict(self._memo)

    def reset(self) -> None:
        """Drop the memo and the counters; registrations survive."""
        self._memo.clear()
        self._calls.clear()
        self._fast_calls.clear()
        self._fallbacks.clear()

    def resolve(self, name: str) -> Callable[..., Any]:
        op = self.get(name)

        def dispatch(*args: Any, **kwargs: Any) -> Any:
            self._calls[op.name] = self._calls.get(op.name, 0) + 1
            if self.selection(op.name, op.key(*args, **kwargs)) == _REFERENCE:
                return op.reference_fn(*args, **kwargs)
            try:
                out = op.fast_fn(*args, **kwargs)  # type: ignore[misc]
            except QmoeLibraryMissing:
                raise
            except Exception as exc:  # noqa: BLE001 - the fail-open contract
                if not self.config.fail_open or self.config.reference_only:
                    raise KernelError(f"{op.name} fast path failed") from exc
                self._fallbacks[op.name] = self._fallbacks.get(op.name, 0) + 1
                return op.reference_fn(*args, **kwargs)
            self._fast_calls[op.name] = self._fast_calls.get(op.name, 0) + 1
            return out

        dispatch.__name__ = f"qmoe_dispatch_{op.name}"
        dispatch.__doc__ = op.reference_fn.__doc__
        return dispatch

    def call(self, name: str, *args: Any, **kwargs: Any) -> Any:
        return self.resolve(name)(*args, **kwargs)

    def counters(self) -> Mapping[str, int]:
        out: dict[str, int] = {}
        for name, n in self._calls.items():
            out[f"{name}.calls"] = n
        for name, n in self._fast_calls.items():
            out[f"{name}.fast"] = n
        for name, n in self._fallbacks.items():
            out[f"{name}.fallbacks"] = n
        return out


def _op_modules():
    from . import moe_gather_int8, moe_gather_ws, moe_weighted_sum  # noqa: PLC0415

    return (moe_weighted_sum, moe_gather_ws, moe_gather_int8)


def build_registry(config: KernelConfig | None = None) -> KernelRegistry:
    """Register every op, validate the policy and publish the registry
    (registry.py:371-383)."""
    registry = KernelRegistry(config)
    for module in _op_modules():
        registry.register(module.OP)
    registry.validate()
    set_current(registry)
    return registry


def reference_only() -> KernelRegistry:
    """Every fast path off and fail-open off: the control arm of an A/B."""
    registry = build_registry(KernelConfig())
    registry.config = KernelConfig(disabled=registry.names(), reference_only=True, fail_open=False)
    registry.reset()
    set_current(registry)
    return registry


_current: KernelRegistry | None = None


def set_current(registry: KernelRegistry | None) -> None:
    global _current
    _current = registry


def current() -> KernelRegistry | None:
    return _current
