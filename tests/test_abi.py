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


def test_token_cap_is_derived_from_byte_ranges():
    """uocr_moe_max_tokens keeps every 32-bit buffer range of the MFMA engine
    below 2^31 bytes: x planes T*H*2, routed hidden planes T*k*I*2, shared
    hidden planes T*S*2, and T*k*H elements of expert outputs."""
    limit = (1 << 31) - 1

    def expect(H, I, E, SH, K):
        per = max(2 * H, 2 * K * I, 2 * I * SH, K * H)
        return limit // per

    # The model shape: routed hidden planes dominate (k*I*2 = 10752 B/token).
    cfg = um.config()
    n = um.max_tokens(cfg)
    assert n == expect(1280, 896, 64, 2, 6) == 199728
    assert n * 6 * 896 * 2 < 1 << 31 and (n + 1) * 6 * 896 * 2 >= limit - 6 * 896 * 2
    # Shapes validate_config accepts where a fixed 262,144-token cap wraps:
    # k=8, I=1024 (T*k*I*2 = 2^32 at 262,144), a wide shared expert, a wide
    # hidden row.
    for H, I, E, SH, K in [(1280, 1024, 64, 2, 8), (2048, 4096, 8, 2, 2), (8192, 64, 8, 1, 1)]:
        c = um.config(H, I, E, SH, K, normalize=True)
        m = um.max_tokens(c)
        assert m == expect(H, I, E, SH, K)
        assert m < 262144
        assert m * max(2 * H, 2 * K * I, 2 * I * SH, K * H) <= limit


def test_decode_timeline_layout():
    """uocr_moe_trace ends with the decode_stamps pointer (eight pointers in
    all) and the binding's row count per role follows the header's
    UOCR_DECODE_STAMP_ROWS: router-logit, shared gate/up, routed gate/up and
    down workgroups of the one-token launch."""
    assert [f[0] for f in um.Trace._fields_][-1] == "decode_stamps"
    assert ctypes.sizeof(um.Trace) == 8 * ctypes.sizeof(ctypes.c_void_p)
    text = open(os.path.join(REPO, "include", "uocr_moe.h")).read()
    assert re.search(r"#define UOCR_DECODE_STAMPS 8\b", text)
    m = re.search(r"#define UOCR_DECODE_STAMP_ROWS\(E, S, k, I, H\) \\\n\s*(.+)\n", text)
    assert m, "row formula not found"
    formula = m.group(1).replace("/", "//")
    for (H, I, E, SH, K) in ((1280, 896, 64, 2, 6), (2048, 512, 37, 2, 8), (256, 64, 8, 1, 2)):
        rows = um.decode_stamp_rows(H, I, E, SH, K)
        want = eval(formula, {}, {"E": E, "S": I * SH, "k": K, "I": I, "H": H})
        assert sum(rows.values()) == want
        assert list(rows) == list(um.DECODE_ROLES)
    assert um.DECODE_STAMPS == 8
