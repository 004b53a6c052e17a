"""The C-ABI library (libfrq.so) loads and exports every entry point that
include/frq.h declares; without a GPU it reports that instead of computing."""
import ctypes as C
import os
import re

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))


def declared_symbols():
    src = open(os.path.join(ROOT, "include", "frq.h")).read()
    src = re.sub(r"/\*.*?\*/", "", src, flags=re.S)
    return sorted(set(re.findall(r"\b(frq_[a-z0-9_]+)\s*\(", src)))


def test_header_declares_the_boundary():
    syms = declared_symbols()
    for s in ["frq_init", "frq_free", "frq_upload_i8", "frq_upload_i4", "frq_mm", "frq_mm_dev",
              "frq_moe", "frq_expert_mm", "frq_last_error"]:
        assert s in syms


def test_library_exports_every_declared_symbol():
    import fieldrun_amd as fa
    lib = C.CDLL(fa.LIB_PATH)
    missing = [s for s in declared_symbols() if not hasattr(lib, s)]
    assert not missing, missing
    # and the Python binding types every one of them
    assert set(declared_symbols()) == set(fa.SIGNATURES)


def test_version_and_errors_without_device():
    import fieldrun_amd as fa
    assert b"gfx950" in fa.lib.frq_version()
    if fa.device_count() > 0:
        pytest.skip("a GPU is visible; the no-device path is not reachable here")
    assert not fa.lib.frq_init(0)
    assert fa.lib.frq_last_error()  # a message, not a crash
    with pytest.raises(fa.FrqError) as ei:
        fa.Context(0)
    assert ei.value.code == fa.FRQ_ERR_NODEV


def test_null_arguments_are_errors_not_crashes():
    import fieldrun_amd as fa
    assert fa.lib.frq_mm(None, None, None, 1, None) == fa.FRQ_ERR_ARG
    assert fa.lib.frq_sync(None) == fa.FRQ_ERR_ARG
    assert fa.lib.frq_moe(None, None, None, 1, None, 1, 1, None, None) == fa.FRQ_ERR_ARG
    assert not fa.lib.frq_upload_i8(None, None, None, 4, 4)
    assert fa.lib.frq_w_info(None, None, None, None, None) == fa.FRQ_ERR_ARG
    fa.lib.frq_free(None)
    fa.lib.frq_w_free(None)
