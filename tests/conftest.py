"""Shared fixtures. GPU tests are marked `gpu`; everything else runs on CPU."""
import importlib.util
import os
import sys

import numpy as np
import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))


def load(relpath, name):
    """Import a module by file path (the package directory name holds a dot)."""
    if name in sys.modules:
        return sys.modules[name]
    spec = importlib.util.spec_from_file_location(name, os.path.join(ROOT, relpath))
    mod = importlib.util.module_from_spec(spec)
    sys.modules[name] = mod
    spec.loader.exec_module(mod)
    return mod


qk = load("qwen.haiku_amd/qk.py", "qk_binding")
synth = load("qwen.haiku_amd/synth.py", "qk_synth")
oracle = load("oracle/oracle.py", "qk_oracle_py")


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (gfx950) GPU")


@pytest.fixture(scope="session")
def orc():
    return oracle.Oracle()


@pytest.fixture(scope="session")
def ref():
    if not oracle.Ref.available():
        pytest.skip("oracle/_ref/libqkref.so not built (reference sources absent)")
    return oracle.Ref()


@pytest.fixture(scope="session")
def lib():
    import torch
    if not torch.cuda.is_available():
        pytest.fail("GPU test on a machine without a GPU")
    L = qk.QK()            # raises if libqk.so is missing: no fallback
    L.init(0)
    return L


@pytest.fixture
def tier(lib):
    """Restore the auto-detected tier after a test that changes it."""
    yield lib
    lib.set_tier(qk.TIER_AUTO)


def bits(a):
    return np.ascontiguousarray(a, np.float32).view(np.uint32)


def assert_bits_equal(got, want, what=""):
    """Bit-for-bit equality, except that two NaNs match whatever their bits:
    a NaN an operation creates (inf * 0, inf - inf) is 0xffc00000 on x86 and
    0x7fc00000 on the GPU; NaNs that propagate from an input keep their
    bits on both and are compared as such only through this rule."""
    g, w = bits(got).ravel(), bits(want).ravel()
    both_nan = np.isnan(np.asarray(got, np.float32).ravel()) & np.isnan(np.asarray(want, np.float32).ravel())
    bad = np.nonzero((g != w) & ~both_nan)[0]
    if bad.size:
        i = bad[0]
        raise AssertionError(f"{what}: {bad.size} of {g.size} differ; first at {i}: "
                             f"got {np.asarray(got).ravel()[i]!r} want {np.asarray(want).ravel()[i]!r}")
