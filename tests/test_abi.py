"""The C-ABI library loads on a CPU-only host and exports every symbol
include/qk.h declares; host-side argument checks work without a GPU."""
import ctypes as C

from conftest import qk


def test_library_exports_header_symbols():
    L = C.CDLL(qk.LIB)
    names = qk.header_functions()
    assert len(names) >= 25
    missing = [n for n in names if not hasattr(L, n)]
    assert not missing, missing


def test_calls_before_init_fail_cleanly():
    lib = qk.QK()
    L = lib.L
    rc = L.hip_quantize_q8k(None, 1, 256, None, None)
    assert rc == 3 and "hip_qk_init" in lib.last_error()
    rc = L.hip_matvec_q4k(None, 1, 256, None, None, None)
    assert rc == 3
    assert lib.label() == "uninitialized"


def test_tier_selection_host_only():
    lib = qk.QK()
    assert [lib.tier_label(t) for t in range(4)] == ["scalar", "AVX1", "AVX2-FMA", "AVX-VNNI"]
    assert lib.L.hip_qk_set_tier(7) == 1
    lib.set_tier(qk.TIER_AUTO)
    assert lib.tier() in (0, 1, 2, 3)
    lib.set_tier(qk.TIER_SCALAR)
    assert lib.tier() == 0
    lib.set_tier(qk.TIER_AUTO)


def test_header_block_sizes():
    import re
    text = open(qk.HEADER).read()
    for name, size in (("qk_q8k_block", 292), ("qk_q4k_block", 144), ("qk_q5k_block", 176),
                       ("qk_q6k_block", 210), ("qk_q8_0_block", 34)):
        assert re.search(rf"}} {name};\s+/\* {size} B", text), name
