"""C-ABI library checks that need no GPU: it loads, exports every symbol
include/mhc_amd.h declares, and rejects bad arguments before any device work."""
from __future__ import annotations

import ctypes
import re
from pathlib import Path

import pytest

ROOT = Path(__file__).resolve().parent.parent
HEADER = ROOT / "include" / "mhc_amd.h"


@pytest.fixture(scope="module")
def lib():
    from model import _hip
    if not _hip.LIB_PATH.exists():
        import __graft_entry__
        __graft_entry__.build()
    return _hip.load()


def declared_functions():
    text = HEADER.read_text()
    return sorted(set(re.findall(r"^\s*(?:const char\*|int64_t|int)\s+(mhc_\w+)\s*\(", text, re.M)))


def test_header_declares_the_boundary():
    names = declared_functions()
    for fn in ("mhc_pre_fwd", "mhc_pre_nohres_fwd", "mhc_post_fwd", "mhc_post_nohres_fwd",
               "mhc_head_fwd", "mhc_sinkhorn_fwd", "mhc_stream_expand_fwd", "mhc_phi_pack",
               "mhc_phi_packed_bytes", "mhc_last_error", "mhc_abi_version"):
        assert fn in names


def test_library_exports_every_declared_symbol(lib):
    raw = ctypes.CDLL(str(ROOT / "minimind-mhc_amd" / "libmhc_amd.so"))
    for name in declared_functions():
        assert hasattr(raw, name), name


def test_binding_signatures_cover_header(lib):
    from model import _hip
    assert set(_hip._SIGNATURES) == set(declared_functions())


def test_packed_sizes(lib):
    # n=4, C=768, full: 4 streams x 24 column blocks x 2 tiles x 64 lanes x 16 B
    assert lib.mhc_phi_packed_bytes(4, 768, 0) == 4 * 24 * 2 * 64 * 16
    assert lib.mhc_phi_packed_bytes(8, 768, 0) == 8 * 24 * 5 * 64 * 16   # FD 80 -> 5 tiles
    assert lib.mhc_phi_packed_bytes(4, 768, 1) == 4 * 24 * 1 * 64 * 16
    # n = 16 and C > 1024 take the K-streamed kernel: FD 288 -> 18 tiles
    assert lib.mhc_phi_packed_bytes(16, 768, 0) == 16 * 24 * 18 * 64 * 16
    assert lib.mhc_phi_packed_bytes(4, 2048, 0) == 4 * 64 * 2 * 64 * 16
    assert lib.mhc_phi_packed_bytes(4, 100, 0) == 0                      # C % 8 != 0
    assert lib.mhc_phi_packed_bytes(3, 768, 0) == 0                      # n not a power of two
    assert lib.mhc_phi_packed_bytes(1, 2048, 2) == 0                     # head n=1 is RMSNorm
    assert lib.mhc_phi_packed_bytes(1, 768, 2) == 0


def test_sinkhorn_bwd_max_iters(lib):
    # checkpointed recompute: one cap for every n
    for n in (1, 2, 3, 4, 8, 16):
        assert lib.mhc_sinkhorn_bwd_max_iters(n) == 256
    assert lib.mhc_sinkhorn_bwd_max_iters(0) == 0
    assert lib.mhc_sinkhorn_bwd_max_iters(17) == 0


def test_split_packed_sizes(lib):
    # fp32 split image: 16-column tiles of 8 features (hi | lo), n in {1, 2, 4}
    assert lib.mhc_phi_split_bytes(4, 768, 0) == 4 * 24 * 3 * 64 * 16   # FD 24 -> 3 tiles
    assert lib.mhc_phi_split_bytes(4, 768, 1) == 4 * 24 * 1 * 64 * 16   # FD 8
    assert lib.mhc_phi_split_bytes(4, 768, 2) == 4 * 24 * 1 * 64 * 16   # FD 4
    assert lib.mhc_phi_split_bytes(2, 512, 0) == 2 * 16 * 1 * 64 * 16   # FD 8
    assert lib.mhc_phi_split_bytes(1, 200, 0) == 1 * 7 * 1 * 64 * 16    # FD 3, ragged C
    # K-streamed fp32: the bf16 K-streamed image twice (hi, then lo)
    assert lib.mhc_phi_split_bytes(8, 768, 0) == 2 * lib.mhc_phi_packed_bytes(8, 768, 0)
    assert lib.mhc_phi_split_bytes(8, 768, 0) == 2 * 8 * 24 * 5 * 64 * 16   # FD 80 -> 5 tiles
    assert lib.mhc_phi_split_bytes(8, 200, 2) == 2 * 8 * 7 * 1 * 64 * 16    # head FD 8
    assert lib.mhc_phi_split_bytes(4, 2048, 0) == 2 * 4 * 64 * 2 * 64 * 16  # C > 1024
    assert lib.mhc_phi_split_bytes(2, 1536, 1) == 2 * 2 * 48 * 1 * 64 * 16
    assert lib.mhc_phi_split_bytes(16, 768, 0) == 0                     # no fp32 instance
    assert lib.mhc_phi_split_bytes(1, 2048, 0) == 0
    assert lib.mhc_phi_split_bytes(4, 100, 0) == 0                      # C % 8 != 0
    assert lib.mhc_phi_split_bytes(8, 100, 0) == 0
    assert lib.mhc_phi_split_bytes(1, 768, 2) == 0                      # head n=1 is RMSNorm
    rc = lib.mhc_phi_pack_split(None, 0, None, 16, 768, 0, None)
    assert rc == 1 and b"no split layout" in lib.mhc_last_error()


def test_validation_errors_need_no_device(lib):
    # n = 0 is rejected by argument checks, before any HIP call
    rc = lib.mhc_pre_fwd(None, 1, None, 1, None, None, None, None, None, None, None, 1,
                         None, None, None, None, None, None, None, 16, 0, 768,
                         2.0, 1e-6, 1e-6, 20, 1e-6, None, None)
    assert rc == 1
    assert b"n must be in" in lib.mhc_last_error()
    rc = lib.mhc_post_fwd(None, 1, None, None, 1, None, 1, None, 16, 4, 768, None, None)
    assert rc == 1
    rc = lib.mhc_sinkhorn_fwd(ctypes.c_void_p(16), ctypes.c_void_p(32), 0, 4, 64, 20, 1e-6, None)
    assert rc == 1 and b"n must be" in lib.mhc_last_error()
    rc = lib.mhc_stream_expand_fwd(ctypes.c_void_p(16), ctypes.c_void_p(32), 3, 4, 4, 8, None)
    assert rc == 1
    # empty problems succeed without launching
    assert lib.mhc_sinkhorn_fwd(ctypes.c_void_p(16), ctypes.c_void_p(32), 0, 0, 4, 20, 1e-6, None) == 0
    assert lib.mhc_phi_pack(None, 0, None, 4, 768, 0, None) == 1  # fp32 phi has no MFMA image


def test_norm_entry_points_validate_without_device(lib):
    p = ctypes.c_void_p(256)
    # the *_norm_fwd variants require the gain
    rc = lib.mhc_pre_norm_fwd(p, 1, p, 1, None, p, p, p, p, p, p, 1, p, None, p, None, p, None,
                              None, 16, 4, 64, 2.0, 1e-6, 1e-6, 20, 1e-6, None, 1, 1e-6, None, None)
    assert rc == 1 and b"norm_weight is required" in lib.mhc_last_error()
    rc = lib.mhc_pre_nohres_norm_fwd(p, 1, p, 1, None, p, p, p, p, 1, p, None, p, None, None,
                                     16, 4, 64, 2.0, 1e-6, 1e-6, None, 1, 1e-6, None, None)
    assert rc == 1 and b"norm_weight is required" in lib.mhc_last_error()
    rc = lib.mhc_head_norm_fwd(p, 1, p, 1, None, p, p, 1, p, None, None, 16, 4, 64, 1e-6, 1e-6,
                               p, 7, 1e-6, None, None)
    assert rc == 1 and b"bad norm dtype" in lib.mhc_last_error()
    rc = lib.mhc_expand_norm_fwd(p, 1, p, 1, p, 16, 4, 64, -1.0, None, None)
    assert rc == 1 and b"eps" in lib.mhc_last_error()
    rc = lib.mhc_expand_norm_fwd(p, 1, p, 1, p, 16, 0, 64, 1e-6, None, None)
    assert rc == 1 and b"bad shape" in lib.mhc_last_error()
    assert lib.mhc_expand_norm_fwd(None, 1, None, 1, None, 0, 4, 64, 1e-6, None, None) == 0


def test_sums_of_squares_argument_checks(lib):
    """x_ssq / out_ssq are defined for bf16 streams with C % 128 == 0 only;
    other shapes are refused before any device work."""
    p = ctypes.c_void_p(256)
    f = ctypes.c_void_p(512)
    # pre with x_ssq at C = 100 (not a multiple of 128), and with an fp32 stream
    for dt, C in ((1, 100), (0, 768)):
        rc = lib.mhc_pre_fwd(p, dt, p, dt, None, p, p, p, p, p, p, dt, p, None, p, None, p, None,
                             None, 16, 8, C, 2.0, 1e-6, 1e-6, 20, 1e-6, f, None)
        assert rc == 1 and b"x_ssq" in lib.mhc_last_error(), (dt, C)
    rc = lib.mhc_post_fwd(p, 1, p, p, 1, p, 1, ctypes.c_void_p(4096), 16, 8, 96, f, None)
    assert rc == 1 and b"out_ssq" in lib.mhc_last_error()
    rc = lib.mhc_expand_norm_fwd(p, 0, p, 0, ctypes.c_void_p(4096), 16, 8, 256, 1e-6, f, None)
    assert rc == 1 and b"out_ssq" in lib.mhc_last_error()


def test_row_staging_round_trip(lib):
    old = lib.mhc_pre_row_staging(-1)
    assert old in (0, 1)
    assert lib.mhc_pre_row_staging(1 - old) == old
    assert lib.mhc_pre_row_staging(-1) == 1 - old
    assert lib.mhc_pre_row_staging(old) == 1 - old
    assert lib.mhc_pre_row_staging(-1) == old


def test_token_threshold_round_trip(lib):
    old = lib.mhc_pre_token_threshold(-1)
    assert old >= 0
    assert lib.mhc_pre_token_threshold(17) == old
    assert lib.mhc_pre_token_threshold(-1) == 17
    assert lib.mhc_pre_token_threshold(old) == 17
    assert lib.mhc_pre_token_threshold(-1) == old


def test_integration_stub_matches_the_header(lib, monkeypatch):
    """The ctypes binding INTEGRATION.md shows declares every entry point it
    binds with the argument list this package's binding (and so the header)
    has: a stale stub would pass the stream in another argument's place."""
    from model import _hip as H
    text = (ROOT / "INTEGRATION.md").read_text()
    sec = text[text.index("## 2."):]
    code = re.search(r"```python\n(.*?)```", sec, re.S).group(1)
    monkeypatch.setenv("MHC_AMD_LIB", str(H.LIB_PATH))
    ns = {}
    exec(compile(code, "INTEGRATION.md", "exec"), ns)
    stub = ns["_lib"]
    bound = [name for name in H._SIGNATURES if getattr(getattr(stub, name), "argtypes", None)]
    assert "mhc_pre_fwd" in bound and "mhc_post_fwd" in bound
    for name in bound:
        assert list(getattr(stub, name).argtypes) == list(H._SIGNATURES[name][1]), name
