"""qmoe_route_noalloc (the routing step with its workspace in the library's
static device scratch) against qmoe_route with a caller workspace, through
the C ABI: every output bit-identical, over consecutive calls that reuse the
scratch with shrinking inputs, on both routing paths (three launches above
8192 pairs, one block below)."""

import numpy as np
import pytest
import torch

from helpers import i32_t
from titan_amd import _lib, ops, synth

pytestmark = pytest.mark.gpu

SCRATCH_BYTES = 1 << 20  # QMOE_ROUTE_NOALLOC_SCRATCH_BYTES in include/qmoe.h


def _noalloc(ids: torch.Tensor, E: int):
    dev = ids.device
    flat = ids.reshape(-1).to(torch.int32).contiguous()
    n = flat.numel()
    tr = ops.tile_rows()
    mt = ops.max_tiles(n, E, tr)
    out = {k: torch.full((n,), -7, dtype=torch.int32, device=dev) for k in ("order", "inv", "srt")}
    out["offsets"] = torch.full((E + 1,), -7, dtype=torch.int32, device=dev)
    out["trow"] = torch.full((mt,), -7, dtype=torch.int32, device=dev)
    out["texp"] = torch.full((mt,), -7, dtype=torch.int32, device=dev)
    out["nt"] = torch.full((1,), -7, dtype=torch.int32, device=dev)
    out["bad"] = torch.full((1,), -7, dtype=torch.int32, device=dev)
    _lib.call("qmoe_route_noalloc", flat.data_ptr(), n, E, tr, out["order"].data_ptr(), out["inv"].data_ptr(),
              out["srt"].data_ptr(), out["offsets"].data_ptr(), out["trow"].data_ptr(), out["texp"].data_ptr(),
              out["nt"].data_ptr(), mt, out["bad"].data_ptr(), torch.cuda.current_stream(dev).cuda_stream)
    return out


def _check_same(got, r):
    torch.cuda.synchronize()
    pairs = [("order", r.order), ("inv", r.inv_order), ("srt", r.sorted_ids), ("offsets", r.tiles.offsets),
             ("trow", r.tiles.tile_row), ("texp", r.tiles.tile_exp), ("nt", r.tiles.ntiles), ("bad", r.bad_ids)]
    for name, want in pairs:
        assert torch.equal(got[name].cpu(), want.cpu()), name


def test_noalloc_route_matches_workspace_route(dev):
    rng = np.random.default_rng(77)
    cases = [
        ("workload-3 zipf, 40960 pairs", synth.make(3)["idx"], 256),
        ("9000 pairs with out-of-range ids", np.concatenate(
            [rng.integers(-3, 70, size=9000)]).astype(np.int32), 64),
        ("700 pairs zipf (single-block path)", synth.make(3, tokens=70)["idx"], 256),
        ("10 pairs (decode)", rng.choice(256, 10, replace=False).astype(np.int32)[None], 256),
    ]
    for name, ids, E in cases:
        print(f"[case] noalloc route: {name}", flush=True)
        t = i32_t(ids, dev)
        got = _noalloc(t, E)
        _check_same(got, ops.route(t, E))


def test_noalloc_route_rejects_oversized_calls(dev):
    print("[case] noalloc route: oversized call rejected", flush=True)
    E = 8192
    n = (SCRATCH_BYTES // 4 // (E + 1) + 1) * 1024  # one chunk more than the scratch holds
    assert int(_lib.load().qmoe_route_workspace_size(n, E)) > SCRATCH_BYTES
    ids = torch.zeros(n, dtype=torch.int32, device=dev)
    with pytest.raises(_lib.QmoeUnsupported, match="scratch"):
        _noalloc(ids, E)
