"""CPU checks of the decode chain's elementwise links (residual add +
RMSNorm, SiLU, SwiGLU): the oracle against the reference compiled from its
own sources, against closed forms, and the device expf restatement
against the host libm over every float input."""
import os
import subprocess
from decimal import Decimal, getcontext
from fractions import Fraction

import numpy as np
import pytest

from cases import edge_rows, special_rows
from conftest import ROOT, assert_bits_equal, synth

CSRC = os.path.join(ROOT, "qwen.haiku_amd", "csrc")


def norm_rows(k, seed=0):
    """Rows for add + RMSNorm: the quantizer edge rows, NaN / inf rows,
    activations, and rows whose squares span many binades (the sequential
    double sum rounds)."""
    rng = np.random.default_rng(seed)
    mixed = (rng.standard_normal(k) * np.exp2(rng.integers(-30, 20, k))).astype(np.float32)
    huge = np.full(k, 1e20, np.float32)                # squares overflow: rscale = 0
    return np.concatenate([edge_rows(k), special_rows(k), synth.activations(5, k, seed=seed),
                           mixed[None], huge[None]]).astype(np.float32)


@pytest.mark.parametrize("k", [4, 256, 1000, 1024, 3584])
def test_add_rmsnorm_oracle_matches_reference(orc, ref, k):
    h = norm_rows(k, seed=k)
    rng = np.random.default_rng(k + 1)
    delta = rng.standard_normal(h.shape).astype(np.float32)
    w = (1 + 0.02 * rng.standard_normal(k)).astype(np.float32)
    for d in (None, delta):
        got = orc.add_rmsnorm(h, d, w, 1e-6)
        want = ref.add_rmsnorm(h, d, w, 1e-6)
        assert_bits_equal(got[0], want[0], f"h + delta k={k}")
        assert_bits_equal(got[1], want[1], f"rms_norm k={k}")


def test_add_rmsnorm_closed_forms(orc):
    """Constant rows: the double sum of k equal squares is exact, so
    x = (c * (1 / sqrtf(c*c + eps))) * w with float32 steps; a zero row
    gives rscale = 1/sqrtf(eps) and x = 0; an added delta is one rounding."""
    k = 1024
    w = np.linspace(0.5, 1.5, k, dtype=np.float32)
    eps = np.float32(1e-6)
    for c in (np.float32(0.75), np.float32(-3.0), np.float32(1e-3), np.float32(0.0)):
        h = np.full((1, k), c, np.float32)
        _, x = orc.add_rmsnorm(h, None, w, eps)
        rs = np.float32(1.0) / np.sqrt(np.float32(c * c) + eps)
        assert_bits_equal(x[0], (c * rs) * w, f"constant row {c}")
    a = np.full((1, k), np.float32(1.0), np.float32)
    b = np.full((1, k), np.float32(2.0 ** -24), np.float32)
    r, _ = orc.add_rmsnorm(a, b, w, eps)
    assert_bits_equal(r[0], np.full(k, 1.0, np.float32), "1 + 2^-24 rounds to 1 (ties to even)")


def test_add_rmsnorm_sum_is_sequential_double(orc):
    """The sum of squares is sequential in double (slm/tensor.c:357-360).
    In this row each 2^-26 square after the first two falls below half an
    ulp of the running sum and is lost, and the mean lands on the other
    side of a float rounding boundary than the exact (or pairwise) sum's
    does, so the norm tells the orders apart."""
    k = 256
    eps = np.float32(1e-6)
    x = np.full(k, np.float32(2.0 ** -13), np.float32)
    x[0] = np.array([0x46800DDC], np.uint32).view(np.float32)[0]   # about 2^14
    x[1] = np.float32(4.0)
    seq = 0.0
    for v in x:
        seq += float(np.float32(v * v))                # Python floats are IEEE doubles
    exact = float(sum(Fraction(float(np.float32(v * v))) for v in x))
    def rscale(ssq):
        return np.float32(1.0) / np.sqrt(np.float32(ssq / k) + eps)
    assert rscale(seq) != rscale(exact)                # the row discriminates
    assert rscale(float(np.sum((x * x).astype(np.float64)))) == rscale(exact)
    w = np.ones(k, np.float32)
    _, got = orc.add_rmsnorm(x[None], None, w, eps)
    assert_bits_equal(got[0], (x * rscale(seq)) * w, "sequential double sum")


def silu_inputs():
    """Every 4099th float bit pattern plus the cut-offs of expf and dense
    samples where silu changes regime."""
    u = np.arange(0, 1 << 32, 4099, dtype=np.uint64).astype(np.uint32).view(np.float32)
    dense = np.concatenate([np.linspace(-110, 110, 200001, dtype=np.float32),
                            np.linspace(-1e-3, 1e-3, 20001, dtype=np.float32),
                            np.array([0.0, -0.0, np.inf, -np.inf, np.nan, 88.72283, -88.72283, 103.97208,
                                      -103.97208, 1e-45, -1e-45, 3.4e38, -3.4e38], np.float32)])
    return np.concatenate([u, dense]).astype(np.float32)


def test_silu_swiglu_oracle_matches_reference(orc, ref):
    x = silu_inputs()
    assert_bits_equal(orc.silu(x), ref.silu(x), "silu")
    up = np.random.default_rng(3).standard_normal(x.size).astype(np.float32)
    assert_bits_equal(orc.swiglu(x, up), ref.swiglu(x, up), "swiglu")


def test_silu_closed_forms(orc):
    """silu(0) = 0, silu(-0) = -0, silu(+inf) = +inf, silu(-inf) is NaN
    (-inf / inf), large negative inputs give -0 or tiny negatives, large
    positive ones are the identity."""
    x = np.array([0.0, -0.0, np.inf, -np.inf, 1e30, -1e30, 200.0], np.float32)
    y = orc.silu(x)
    assert y[0] == 0 and not np.signbit(y[0])
    assert y[1] == 0 and np.signbit(y[1])
    assert y[2] == np.inf and np.isnan(y[3])
    assert y[4] == np.float32(1e30) and y[5] == 0 and np.signbit(y[5])
    assert y[6] == np.float32(200.0)


# ---- the device expf restatement ----------------------------------------------

def host_has_fma():
    try:
        with open("/proc/cpuinfo") as f:
            return any(line.startswith("flags") and " fma " in line + " " for line in f)
    except OSError:
        return False


def test_expf_table_is_exp2():
    """qk_exp2_32[i] + (i << 47) are the bits of 2^(i/32) rounded to double
    (computed here from 70-digit decimals, well away from a rounding tie)."""
    text = open(os.path.join(CSRC, "qk_expf.h")).read()
    body = text[text.index("qk_exp2_32[32] = {") :].split("};")[0]
    tab = [int(t, 16) for t in body.replace("ULL", "").split("{")[1].replace(",", " ").split()]
    assert len(tab) == 32
    getcontext().prec = 70
    for i, entry in enumerate(tab):
        v = Decimal(2) ** (Decimal(i) / Decimal(32))
        d = float(v)                                   # correctly rounded from the decimal string
        ulp = np.spacing(d)
        frac = (Fraction(v) - Fraction(d)) / Fraction(ulp)
        assert abs(frac) < Fraction(1, 2) - Fraction(1, 10 ** 6), f"entry {i} is near a tie"
        want = (int(np.float64(d).view(np.uint64)) - (i << 47)) & 0xFFFFFFFFFFFFFFFF
        assert entry == want, f"entry {i}: {entry:#x} != {want:#x}"


def test_expf_matches_libm_everywhere(tmp_path):
    """The device expf (qk_expf.h, compiled here as C) equals the host libm
    expf on all 2^32 inputs. glibc on an FMA host runs its fused build,
    which the header restates; a host without FMA runs the unfused one."""
    if not host_has_fma():
        pytest.skip("host CPU has no FMA: its glibc expf is the unfused build")
    exe = tmp_path / "expf_check"
    subprocess.run(["gcc", "-O2", "-std=gnu99", "-ffp-contract=off", "-fno-fast-math", f"-I{CSRC}", "-o", str(exe),
                    os.path.join(ROOT, "tests", "expf_check.c"), "-lm", "-lpthread"], check=True)
    out = subprocess.run([str(exe), os.environ.get("QK_EXPF_STRIDE", "1")], check=True, capture_output=True,
                         text=True).stdout.split()
    assert out[0] == "0", f"{out[0]} mismatches, first input bits {out[1]}"
