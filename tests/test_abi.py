"""The C ABI library loads (no GPU needed) and exports every entry point include/otpu.h
declares, with the argument counts the ctypes binding uses."""
import os
import re

import pytest

from opentpu_amd import _lib

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))


def declared():
    src = open(os.path.join(ROOT, "include", "otpu.h")).read()
    src = re.sub(r"/\*.*?\*/", "", src, flags=re.S)
    out = {}
    for m in re.finditer(r"(?:int64_t|int|const char\*)\s+(otpu_\w+)\s*\(([^)]*)\)\s*;", src):
        args = [a for a in m.group(2).split(",") if a.strip() and a.strip() != "void"]
        out[m.group(1)] = len(args)
    return out


def test_header_declares_the_entry_points():
    d = declared()
    for name in ("otpu_qact", "otpu_mm", "otpu_mm_acc", "otpu_mm_batched", "otpu_lm_head_argmax",
                 "otpu_argmax", "otpu_pack_int8", "otpu_pack_x4", "otpu_last_error", "otpu_version",
                 "otpu_sample_work_bytes", "otpu_lda", "otpu_mm_spl"):
        assert name in d
    assert set(d) == set(_lib.SIGNATURES), set(d) ^ set(_lib.SIGNATURES)


@pytest.mark.skipif(not os.path.exists(_lib.LIB_PATH), reason="libotpu_amd.so not built")
def test_library_exports_every_declared_symbol():
    lib = _lib.load()
    for name, nargs in declared().items():
        fn = getattr(lib, name)                       # raises if not exported
        assert name in _lib.SIGNATURES, name
        assert len(_lib.SIGNATURES[name][0]) == nargs, name
        assert fn is not None
    assert lib.otpu_version() == _lib.ABI_VERSION


def test_header_constants_match_the_binding():
    """The sizes the header states (OTPU_QALIGN, OTPU_LM_STATE_BYTES) are the ones the Python
    binding allocates with, and the LM head's state holds its 64 maxima 256 bytes apart after the
    result's 256 bytes."""
    src = open(os.path.join(ROOT, "include", "otpu.h")).read()
    consts = {m.group(1): int(m.group(2)) for m in re.finditer(r"#define (OTPU_\w+)\s+(\d+)", src)}
    assert consts["OTPU_QALIGN"] == _lib.QALIGN
    assert consts["OTPU_ABI_VERSION"] == _lib.ABI_VERSION
    assert consts["OTPU_LM_STATE_BYTES"] == _lib.LM_STATE_BYTES == 256 * (1 + 64)
