"""numpy <-> torch plumbing for the tests (bf16 as uint16 bit patterns)."""

import numpy as np
import torch


def bf16_t(a, dev=None) -> torch.Tensor:
    t = torch.from_numpy(np.ascontiguousarray(a, dtype=np.uint16).view(np.int16)).view(torch.bfloat16)
    return t.to(dev) if dev is not None else t


def words_t(a, dev=None) -> torch.Tensor:
    t = torch.from_numpy(np.ascontiguousarray(a, dtype=np.uint32).view(np.int32))
    return t.to(dev) if dev is not None else t


def i32_t(a, dev=None) -> torch.Tensor:
    t = torch.from_numpy(np.ascontiguousarray(a, dtype=np.int32))
    return t.to(dev) if dev is not None else t


def f32_t(a, dev=None) -> torch.Tensor:
    t = torch.from_numpy(np.ascontiguousarray(a, dtype=np.float32))
    return t.to(dev) if dev is not None else t


def bits(t: torch.Tensor) -> np.ndarray:
    """bf16 tensor -> numpy uint16 bit patterns."""
    return t.detach().cpu().contiguous().view(torch.int16).numpy().view(np.uint16)


def assert_close_bf16(orc, got_bits, ref_f64, max_ulp=1, rel_to_max=2.0 ** -8, what=""):
    """The parity bar: within ``max_ulp`` bf16 ULP of the RNE-rounded golden on
    live elements (|ref| >= max|ref|/256) and max-abs error within
    ``rel_to_max`` of max|ref| everywhere.  Prints the report."""
    rep = orc.err_report(got_bits, ref_f64)
    print(f"[parity] {what}: {rep}", flush=True)
    assert rep["max_ulp_live"] <= max_ulp, (what, rep)
    assert rep["rel_to_max"] <= rel_to_max, (what, rep)
    return rep
