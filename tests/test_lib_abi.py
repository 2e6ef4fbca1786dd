"""The C-ABI library: builds, loads without a GPU, exports exactly what
include/qmoe.h declares, and rejects bad arguments before touching the device."""

import ctypes
import re
import subprocess
from pathlib import Path

import pytest

from titan_amd import _lib

ROOT = Path(__file__).resolve().parent.parent
HEADER = ROOT / "include" / "qmoe.h"


def declared():
    text = HEADER.read_text()
    return sorted(set(re.findall(r"\b(qmoe_[a-z0-9_]+)\s*\(", text)))


@pytest.fixture(scope="module")
def L():
    if not _lib.LIB_PATH.exists():
        from titan_amd import build

        build.build()
    return _lib.load()


def test_header_declares_the_bound_signatures():
    assert declared() == sorted(_lib.SIGNATURES), (declared(), sorted(_lib.SIGNATURES))


def test_every_declared_symbol_is_exported(L):
    out = subprocess.run(["nm", "-D", "--defined-only", str(_lib.LIB_PATH)], capture_output=True, text=True,
                         check=True).stdout
    exported = set(re.findall(r"\bT (qmoe_[a-z0-9_]+)$", out, flags=re.M))
    missing = set(declared()) - exported
    assert not missing, missing
    for name in declared():
        assert getattr(L, name) is not None


def test_abi_version_matches_header(L):
    m = re.search(r"#define QMOE_ABI_VERSION (\d+)", HEADER.read_text())
    assert L.qmoe_abi_version() == int(m.group(1))


def test_tile_rows_and_workspace_queries(L):
    assert L.qmoe_gemm_tile_rows() == 128
    ws = L.qmoe_route_workspace_size(40960, 256)
    assert ws % 256 == 0 and ws >= 4 * (64 + 257 * 40)  # 40960 rows = 40 chunks of 1024
    assert L.qmoe_route_workspace_size(-1, 256) == 0


def test_bad_arguments_are_rejected_without_a_device(L):
    rc = L.qmoe_gather_qmv(None, None, None, 4, 2048, None, None, None, 8, 128, 64, 4, None, None)
    assert rc == _lib.ERR_INVALID
    assert "null" in _lib.last_error()
    rc = L.qmoe_weighted_sum(None, None, None, 2, 0, 256, 2, None, None)
    assert rc == _lib.ERR_INVALID


def test_unsupported_configurations_say_so(L):
    dummy = ctypes.c_void_p(16)  # never dereferenced: rejected on the host
    rc = L.qmoe_gather_qmv(dummy, None, dummy, 4, 2048, dummy, dummy, dummy, 8, 128, 64, 3, dummy, None)
    assert rc == _lib.ERR_UNSUPPORTED and "bits=3" in _lib.last_error()
    # 8-bit codes: K = 2048 * n (n <= 4) or a lane split (K <= 4096), and no fused decode kernel
    rc = L.qmoe_quantized_matmul(dummy, 1, 10240, dummy, dummy, dummy, 64, 64, 8, dummy, None)
    assert rc == _lib.ERR_UNSUPPORTED and "K=10240" in _lib.last_error()
    rc = L.qmoe_moe_gate_up_swiglu(dummy, dummy, 1, 2, 2048, dummy, dummy, dummy, 4, 64, 64, 8, dummy, None)
    assert rc == _lib.ERR_UNSUPPORTED and "bits=8" in _lib.last_error()
    rc = L.qmoe_gather_qmv(dummy, None, dummy, 4, 2048, dummy, dummy, dummy, 8, 128, 48, 4, dummy, None)
    assert rc == _lib.ERR_UNSUPPORTED
    rc = L.qmoe_gather_qmm_sorted(dummy, None, 10, 2048, dummy, dummy, dummy, 8, 200, 64, 4, dummy, dummy,
                                  dummy, dummy, 10, dummy, None)
    assert rc == _lib.ERR_UNSUPPORTED and "N=200" in _lib.last_error()
    # the grouped GEMMs' epilogue addresses rows with 32-bit offsets: N <= 2^24
    rc = L.qmoe_gather_qmm_sorted_tiles(dummy, None, 10, 2048, dummy, dummy, 8, (1 << 24) + 256, dummy, dummy,
                                        dummy, dummy, 10, dummy, None)
    assert rc == _lib.ERR_UNSUPPORTED and "too large" in _lib.last_error()
    rc = L.qmoe_route(dummy, 10, 8, 128, dummy, dummy, dummy, dummy, dummy, dummy, dummy, 100, None, 0, None)
    assert rc == _lib.ERR_WORKSPACE


def test_check_maps_codes_to_exceptions(L):
    with pytest.raises(_lib.QmoeUnsupported):
        _lib.call("qmoe_weighted_sum", 16, None, 16, 2, 10, 256, 9, 16, None)
    with pytest.raises(_lib.QmoeError):
        _lib.call("qmoe_weighted_sum", None, None, None, 2, 10, 256, 2, None, None)


def test_peaks_library_exports_its_header():
    """libqmoe_peaks.so (the bench's measured-ceiling probes) exports what
    include/qmoe_peaks.h declares."""
    from titan_amd import build

    if not build.PEAKS_LIB.exists():
        build.build()
    names = sorted(set(re.findall(r"\b(qmoe_peak_[a-z0-9_]+)\s*\(", (ROOT / "include" / "qmoe_peaks.h").read_text())))
    out = subprocess.run(["nm", "-D", "--defined-only", str(build.PEAKS_LIB)], capture_output=True, text=True,
                         check=True).stdout
    exported = set(re.findall(r"\bT (qmoe_peak_[a-z0-9_]+)$", out, flags=re.M))
    assert names and set(names) <= exported, (names, exported)
    L = ctypes.CDLL(str(build.PEAKS_LIB))
    assert L.qmoe_peak_stream_blocks() > 0 and L.qmoe_peak_mfma_waves() > 0


def test_header_is_plain_c_and_a_c_program_links(tmp_path):
    """The boundary a C, cgo or FFI caller binds: the headers compile as
    C11 with warnings as errors, and a C program links libqmoe.so, reads the
    ABI version and gets QMOE_ERR_INVALID plus a message for a null pointer
    (host-side checks only: no device is touched)."""
    import shutil

    if shutil.which("gcc") is None:
        pytest.skip("no gcc")
    src = tmp_path / "probe.c"
    src.write_text(
        '#include <stdio.h>\n#include "qmoe.h"\n#include "qmoe_peaks.h"\n'
        "int main(void) {\n"
        "  if (qmoe_abi_version() != QMOE_ABI_VERSION) return 2;\n"
        "  int rc = qmoe_gather_qmv(NULL, NULL, NULL, 4, 2048, NULL, NULL, NULL, 8, 128, 64, 4, NULL, NULL);\n"
        '  printf("%d %s\\n", rc, qmoe_last_error());\n'
        "  return rc == QMOE_ERR_INVALID ? 0 : 3;\n"
        "}\n")
    exe = tmp_path / "probe"
    libdir = str(_lib.LIB_PATH.parent)
    subprocess.run(["gcc", "-std=c11", "-Wall", "-Wextra", "-Werror", "-pedantic", "-I", str(HEADER.parent),
                    str(src), "-L", libdir, "-lqmoe", f"-Wl,-rpath,{libdir}", "-o", str(exe)], check=True)
    out = subprocess.run([str(exe)], capture_output=True, text=True)
    assert out.returncode == 0, out
    assert "null" in out.stdout
