"""The op registry's policy and dispatch (mirrors the reference's
tests/kernels/test_registry.py): selection per shape class, memo, policy
lists, fail-open, phase.  Toy ops on CPU tensors; no GPU."""

import pytest
import torch

from titan_amd import _lib
from titan_amd.errors import ConfigError, KernelError
from titan_amd.kernels import registry as R


def _toy(name="toy", fast=lambda x: x + 1, supports=lambda k: k.shapes[0][0] <= 4, **kw):
    return R.KernelOp(name=name, reference_fn=lambda x: x - 1, fast_fn=fast,
                      key=lambda x: R.shape_class(x, device="gpu"), supports_key=supports, **kw)


def _reg(*ops, **cfg):
    reg = R.KernelRegistry(R.KernelConfig(**cfg))
    for op in ops:
        reg.register(op)
    reg.validate()
    return reg


def test_every_op_is_registered():
    reg = R.build_registry()
    assert reg.names() == ("moe_gather_int8", "moe_gather_ws", "moe_weighted_sum")
    assert R.current() is reg


def test_engine_facing_aliases_resolve():
    reg = R.build_registry()
    assert reg.get("moe_gather_gate_up") is reg.get("moe_gather_int8")


def test_every_op_declares_its_shapes_and_provenance():
    reg = R.build_registry()
    for name in reg.names():
        op = reg.get(name)
        assert op.shapes and op.source and op.exactness != "unspecified", name
        if op.default_off:
            assert op.default_off_reason, name


def test_duplicate_registration_is_an_error():
    reg = _reg(_toy())
    with pytest.raises(ConfigError):
        reg.register(_toy())


def test_unknown_op_names_the_registered_ones():
    reg = _reg(_toy())
    with pytest.raises(ConfigError, match="toy"):
        reg.get("nope")


def test_fast_is_selected_when_supported():
    reg = _reg(_toy())
    assert reg.call("toy", torch.zeros(3)).tolist() == [1.0] * 3


def test_unsupported_shape_class_falls_to_reference():
    reg = _reg(_toy())
    assert reg.call("toy", torch.zeros(8)).tolist() == [-1.0] * 8


def test_selection_is_memoised_per_shape_class():
    seen = []
    reg = _reg(_toy(supports=lambda k: seen.append(k) or True))
    for _ in range(3):
        reg.call("toy", torch.zeros(2))
    assert len(seen) == 1 and len(reg.selections()) == 1


def test_a_different_shape_class_selects_again():
    seen = []
    reg = _reg(_toy(supports=lambda k: seen.append(k) or True))
    reg.call("toy", torch.zeros(2))
    reg.call("toy", torch.zeros(3))
    reg.call("toy", torch.zeros(2, dtype=torch.float64))
    assert len(seen) == 3


def test_shape_class_ignores_values_and_captures_dtype():
    a = R.shape_class(torch.zeros(2, 3), None, torch.ones(4, dtype=torch.int32), extra=(64, 4))
    b = R.shape_class(torch.ones(2, 3), None, torch.zeros(4, dtype=torch.int32), extra=(64, 4))
    assert a == b and a.device == "cpu"
    assert a.dtypes == (torch.float32, torch.int32) and a.shapes == ((2, 3), (4,))


def test_reset_drops_the_memo_not_the_registrations():
    reg = _reg(_toy())
    reg.call("toy", torch.zeros(2))
    reg.reset()
    assert not reg.selections() and not reg.counters() and reg.names() == ("toy",)


def test_disabled_op_uses_the_reference():
    reg = _reg(_toy(), disabled=("toy",))
    assert reg.call("toy", torch.zeros(2)).tolist() == [-1.0, -1.0]
    assert reg.fast_disabled("toy")


def test_enabled_list_is_an_allowlist():
    reg = _reg(_toy(), _toy(name="other"), enabled=("other",))
    assert reg.call("toy", torch.zeros(2)).tolist() == [-1.0, -1.0]
    assert reg.call("other", torch.zeros(2)).tolist() == [1.0, 1.0]


def test_default_off_op_runs_only_when_named():
    op = _toy(default_off=True, default_off_reason="changes the numbers")
    assert _reg(op).call("toy", torch.zeros(1)).item() == -1.0
    assert _reg(_toy(default_off=True), enabled=("toy",)).call("toy", torch.zeros(1)).item() == 1.0


def test_reference_only_turns_everything_off():
    reg = R.reference_only()
    for name in reg.names():
        assert reg.fast_disabled(name)
    assert not reg.config.fail_open
    R.build_registry()  # leave a default registry published


def test_a_stale_disable_flag_is_an_error_not_a_no_op():
    with pytest.raises(ConfigError):
        _reg(_toy(), disabled=("tyo",))


def test_an_alias_may_be_disabled_by_either_name():
    reg = _reg(_toy(aliases=("toy_alias",)), disabled=("toy_alias",))
    assert reg.fast_disabled("toy")


def _boom(x):
    raise RuntimeError("kernel failed")


def test_a_raising_fast_path_falls_back_and_counts():
    reg = _reg(_toy(fast=_boom))
    assert reg.call("toy", torch.zeros(1)).item() == -1.0
    assert reg.counters()["toy.fallbacks"] == 1


def test_fail_open_off_raises_a_kernel_error():
    reg = _reg(_toy(fast=_boom), fail_open=False)
    with pytest.raises(KernelError):
        reg.call("toy", torch.zeros(1))


def test_a_missing_native_library_is_never_answered_by_the_reference():
    def missing(x):
        raise _lib.QmoeLibraryMissing(-1, "libqmoe.so not built")

    reg = _reg(_toy(fast=missing))
    with pytest.raises(_lib.QmoeLibraryMissing):
        reg.call("toy", torch.zeros(1))


def test_an_op_without_a_fast_path_never_selects_one():
    op = R.KernelOp(name="slow", reference_fn=lambda x: x, key=lambda x: R.shape_class(x))
    reg = _reg(op)
    assert reg.fast_disabled("slow") and not op.supports(torch.zeros(1))
    with pytest.raises(KernelError):
        op.fast(torch.zeros(1))


def test_a_prefill_only_op_takes_its_fast_path_only_during_prefill():
    reg = _reg(_toy(), prefill_only=("toy",))
    assert reg.call("toy", torch.zeros(1)).item() == -1.0
    with R.phase("prefill"):
        assert reg.call("toy", torch.zeros(1)).item() == 1.0


def test_the_selection_memo_does_not_leak_across_the_phase():
    reg = _reg(_toy(), prefill_only=("toy",))
    with R.phase("prefill"):
        reg.call("toy", torch.zeros(1))
    assert reg.call("toy", torch.zeros(1)).item() == -1.0


def test_an_op_not_named_prefill_only_is_unaffected_by_the_phase():
    reg = _reg(_toy(), _toy(name="other"), prefill_only=("other",))
    assert reg.call("toy", torch.zeros(1)).item() == 1.0


def test_the_phase_is_restored_even_when_the_block_raises():
    before = R.get_phase()
    with pytest.raises(ValueError):
        with R.phase("prefill"):
            raise ValueError
    assert R.get_phase() == before


def test_a_stale_prefill_only_name_is_rejected_like_a_stale_bisect_flag():
    with pytest.raises(ConfigError):
        _reg(_toy(), prefill_only=("gone",))


def test_real_ops_decline_cpu_tensors():
    """The HIP ops only take ROCm tensors; on CPU every call goes to the stock
    reference, which is what lets the host logic run without a GPU."""
    from titan_amd.kernels import moe_gather_ws, moe_weighted_sum

    x = torch.zeros(64, 1, 256, dtype=torch.bfloat16)
    w = torch.zeros(4, 256, 32, dtype=torch.int32)
    s = torch.zeros(4, 256, 4, dtype=torch.bfloat16)
    idx = torch.zeros(64, dtype=torch.int32)
    assert not moe_gather_ws.OP.supports(x, w, s, s, idx)
    k = moe_gather_ws.key(x, w, s, s, idx)
    assert moe_gather_ws.supports(R.ShapeClass(k.shapes, k.dtypes, "gpu", k.extra))
    xs = torch.zeros(20, 256, dtype=torch.bfloat16)
    assert not moe_weighted_sum.OP.supports(xs, None, torch.zeros(2, 10), (2, 256))
