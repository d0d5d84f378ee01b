"""The C-ABI library loads and exports every function include/uocr_moe.h
declares; host-only helpers behave (no GPU needed)."""
import ctypes
import os
import re

import uocr_moe as um

REPO = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))


def declared():
    text = open(os.path.join(REPO, "include", "uocr_moe.h")).read()
    return set(re.findall(r"^\s*(?:const\s+)?[\w\s\*]+?\b(uocr_\w+)\s*\(", text, re.M))


def test_header_and_binding_agree():
    names = declared()
    assert names, "no declarations parsed"
    assert names == set(um.EXPORTS)


def test_library_exports_every_symbol():
    lib = ctypes.CDLL(um.LIB_PATH)
    for name in declared():
        assert hasattr(lib, name), name


def test_scratch_budget_grows_with_tokens():
    cfg = um.config()
    small, big = um.scratch_bytes(cfg, 1), um.scratch_bytes(cfg, 4096)
    assert 0 < small < big
    # Dominated by the routed hidden and output rows: T*k*(I + H) floats.
    assert big >= 4096 * 6 * (896 + 1280) * 4
