"""GPU parity of the decode chain's elementwise links and of a whole FFN
block kept on the device (residual add + RMSNorm -> Q8_K -> gate/up GEMV
-> SiLU * up -> Q8_K -> down GEMV), through the C ABI, against the CPU
oracle. Bar: bit-exact (both float-epilogue families for the GEMVs)."""
import numpy as np
import pytest

from conftest import assert_bits_equal, oracle, qk, synth
from test_chain_oracle import norm_rows, silu_inputs

pytestmark = pytest.mark.gpu

EPI_TIERS = [(oracle.EPI_SEPARATE, qk.TIER_SCALAR), (oracle.EPI_FUSED, qk.TIER_AVX2)]


def dev(a):
    import torch
    return torch.from_numpy(np.ascontiguousarray(a)).cuda()


def host(t):
    import torch
    torch.cuda.synchronize()
    return t.cpu().numpy()


def empty(shape, dtype=None):
    import torch
    return torch.empty(shape, dtype=dtype or torch.float32, device="cuda")


def step(msg):
    print(f"[gpu] {msg}", flush=True)


def q8k_rows(m, k):
    import torch
    return empty((m, (k // 256) * qk.Q8K_BYTES), torch.uint8)


@pytest.mark.parametrize("k", [256, 1024, 3584, 16384])
@pytest.mark.parametrize("with_delta", [False, True])
def test_add_rmsnorm_bit_exact(lib, orc, k, with_delta):
    step(f"add_rmsnorm k={k} delta={with_delta}")
    h = norm_rows(k, seed=k)
    m = h.shape[0]
    rng = np.random.default_rng(k)
    delta = rng.standard_normal(h.shape).astype(np.float32) if with_delta else None
    w = (1 + 0.02 * rng.standard_normal(k)).astype(np.float32)
    want_r, want_x = orc.add_rmsnorm(h, delta, w, 1e-6)
    hd, ho, xo, xq = dev(h), empty((m, k)), empty((m, k)), q8k_rows(m, k)
    lib.add_rmsnorm_q8k(hd, None if delta is None else dev(delta), dev(w), 1e-6, h_out=ho, x_out=xo, xq=xq)
    assert_bits_equal(host(ho), want_r, "h + delta")
    assert_bits_equal(host(xo), want_x, "rms_norm")
    np.testing.assert_array_equal(host(xq), orc.quantize_q8k(want_x))


def test_add_rmsnorm_in_place_and_partial_outputs(lib, orc):
    """h_out == h (the residual stream updated in place), xq without x_out,
    x_out without xq at a width that is not a multiple of 256, and a
    prefill batch of 512 rows."""
    step("add_rmsnorm in place / partial outputs / m=512")
    rng = np.random.default_rng(7)
    for m, k in ((1, 1024), (512, 1024), (3, 1000)):
        h = synth.activations(m, k, seed=m)
        delta = rng.standard_normal((m, k)).astype(np.float32)
        w = (1 + 0.02 * rng.standard_normal(k)).astype(np.float32)
        want_r, want_x = orc.add_rmsnorm(h, delta, w, 1e-6)
        hd = dev(h)
        if k % 256 == 0:
            xq = q8k_rows(m, k)
            lib.add_rmsnorm_q8k(hd, dev(delta), dev(w), 1e-6, h_out=hd, xq=xq)
            np.testing.assert_array_equal(host(xq), orc.quantize_q8k(want_x))
        else:
            xo = empty((m, k))
            lib.add_rmsnorm_q8k(hd, dev(delta), dev(w), 1e-6, h_out=hd, x_out=xo)
            assert_bits_equal(host(xo), want_x, f"rms_norm m={m} k={k}")
        assert_bits_equal(host(hd), want_r, f"in-place h m={m} k={k}")


def norm_block_rows(k, rng):
    """Rows for the norm's block walk (64 squares per block, added in one
    step when every add of the block is exact, else one by one): blocks
    at scales that change by up to 2^40 from block to block (exact and
    rounding blocks in one row), powers of two (squares with one set bit),
    a lone huge value followed by tiny ones (the tiny squares round away),
    and the row whose sequential sum differs from its exact and pairwise
    sums."""
    rows = []
    for _ in range(6):
        scale = np.repeat(np.exp2(rng.integers(-20, 21, (k + 63) // 64)), 64)[:k]
        rows.append(rng.standard_normal(k) * scale)
    rows.append(np.exp2(rng.integers(-40, 20, k)).astype(np.float64) * rng.choice([-1, 1], k))
    tiny = rng.standard_normal(k) * 2.0 ** -20
    tiny[k // 3] = 3.0e4
    rows.append(tiny)
    rows.append(rng.uniform(-1, 1, k))
    disc = np.full(k, np.float32(2.0 ** -13))
    disc[0] = np.array([0x46800DDC], np.uint32).view(np.float32)[0]
    disc[min(1, k - 1)] = 4.0
    rows.append(disc)
    return np.asarray(rows, np.float32)


@pytest.mark.parametrize("k", [4, 100, 256, 1000, 1024, 3584, 16384])
def test_add_rmsnorm_block_paths(lib, orc, k):
    step(f"add_rmsnorm block paths k={k}")
    rng = np.random.default_rng(k + 5)
    h = norm_block_rows(k, rng)
    w = (1 + 0.02 * rng.standard_normal(k)).astype(np.float32)
    xo = empty(h.shape)
    lib.add_rmsnorm_q8k(dev(h), None, dev(w), 1e-6, x_out=xo)
    assert_bits_equal(host(xo), orc.add_rmsnorm(h, None, w, 1e-6)[1], f"block paths k={k}")


def test_add_rmsnorm_many_scales(lib, orc):
    """4096 constant rows spanning 60 binades: as many distinct
    rscale = 1/sqrtf(mean + eps) values, each correctly rounded."""
    step("add_rmsnorm 4096 constant rows")
    k = 256
    rng = np.random.default_rng(11)
    c = (rng.uniform(1, 2, 4096) * np.exp2(rng.integers(-30, 30, 4096))).astype(np.float32)
    h = np.repeat(c[:, None], k, axis=1)
    w = np.ones(k, np.float32)
    xo = empty((4096, k))
    lib.add_rmsnorm_q8k(dev(h), None, dev(w), 1e-6, x_out=xo)
    assert_bits_equal(host(xo), orc.add_rmsnorm(h, None, w, 1e-6)[1], "constant rows")


def test_silu_bit_exact(lib, orc):
    """Every 4099th float bit pattern, the expf cut-offs and dense regime
    changes, plus every 61st pattern (70 M inputs, all exponents)."""
    x = silu_inputs()
    step(f"silu {x.size} inputs")
    assert_bits_equal(host(lib.silu(dev(x))), orc.silu(x), "silu")
    u = np.arange(0, 1 << 32, 61, dtype=np.uint64).astype(np.uint32).view(np.float32)
    step(f"silu {u.size} inputs")
    got = host(lib.silu(dev(u)))
    want = orc.silu(u)
    bad = np.flatnonzero((got.view(np.uint32) != want.view(np.uint32)) & ~(np.isnan(got) & np.isnan(want)))
    assert bad.size == 0, f"{bad.size} mismatches, first x bits {u.view(np.uint32)[bad[0]]:#010x}"


@pytest.mark.parametrize("m,k", [(1, 3584), (512, 3584), (4, 1024), (3, 1000)])
def test_swiglu_bit_exact(lib, orc, m, k):
    step(f"swiglu m={m} k={k}")
    rng = np.random.default_rng(m * k)
    gate = (rng.standard_normal((m, k)) * 4).astype(np.float32)
    gate.ravel()[: min(16, gate.size)] = [0.0, -0.0, np.inf, -np.inf, np.nan, 89.0, -89.0, 104.0, -104.0,
                                           1e-40, -1e-40, 3e38, -3e38, 20.0, -20.0, 0.5][: min(16, gate.size)]
    up = rng.standard_normal((m, k)).astype(np.float32)
    want = orc.swiglu(gate, up).reshape(m, k)
    act = empty((m, k))
    xq = q8k_rows(m, k) if k % 256 == 0 else None
    lib.swiglu_q8k(dev(gate), dev(up), act=act, xq=xq)
    assert_bits_equal(host(act), want, "swiglu")
    if xq is not None:
        np.testing.assert_array_equal(host(xq), orc.quantize_q8k(want))


def test_chain_rejects_bad_shapes(lib):
    step("chain argument checks")
    x = empty((1, 1024))
    w = empty(1024)
    with pytest.raises(qk.QKError):                    # no output at all
        lib.add_rmsnorm_q8k(x, None, w, 1e-6)
    with pytest.raises(qk.QKError):                    # a Q8_K row needs k % 256 == 0
        lib.add_rmsnorm_q8k(empty((1, 1000)), None, empty(1000), 1e-6, xq=q8k_rows(1, 1024))
    with pytest.raises(qk.QKError):                    # beyond the LDS row limit
        lib.add_rmsnorm_q8k(empty((1, 16640)), None, empty(16640), 1e-6, x_out=empty((1, 16640)))
    with pytest.raises(qk.QKError):                    # delta aliasing h_out
        lib.add_rmsnorm_q8k(x, x, w, 1e-6, h_out=x, x_out=empty((1, 1024)))
    with pytest.raises(qk.QKError):
        lib.swiglu_q8k(empty((1, 1000)), empty((1, 1000)), xq=q8k_rows(1, 1024))


# ---- a whole FFN block on the device ------------------------------------------------

def ffn_weights(hdim, ffn, seed):
    return (synth.blocks(12, ffn, hdim, seed=seed, tag=12),          # gate, Q4_K
            synth.blocks(12, ffn, hdim, seed=seed + 1, tag=12),      # up, Q4_K
            synth.blocks(14, hdim, ffn, seed=seed + 2, tag=14))      # down, Q6_K


def ffn_oracle(orc, h, mix, norm_w, wg, wu, wd, hdim, ffn, epi):
    """slm/qwen.c:936-962 for one token batch: h += mix; x = ffn_norm(h);
    down(silu(gate(x)) * up(x)); then the residual add."""
    r, x = orc.add_rmsnorm(h, mix, norm_w, 1e-6)
    g = orc.matmul(12, wg, ffn, hdim, x, epi)
    u = orc.matmul(12, wu, ffn, hdim, x, epi)
    a = orc.swiglu(g, u).reshape(g.shape)
    d = orc.matmul(14, wd, hdim, ffn, a, epi)
    return r, d, (r + d).astype(np.float32)


@pytest.mark.parametrize("epi,tier_id", EPI_TIERS)
@pytest.mark.parametrize("m", [1, 64])
def test_ffn_block_on_device(tier, orc, epi, tier_id, m):
    """Decode (m = 1: grouped GEMV launches) and prefill (m = 64: GEMMs):
    every intermediate stays in device memory; the block's output and the
    residual stream equal the oracle's bit for bit."""
    import torch
    tier.set_tier(tier_id)
    hdim, ffn = 1024, 3584
    step(f"ffn block m={m} tier={tier_id}")
    wg, wu, wd = ffn_weights(hdim, ffn, seed=40)
    rng = np.random.default_rng(m)
    h = synth.activations(m, hdim, seed=m + 10)
    mix = rng.standard_normal((m, hdim)).astype(np.float32)
    norm_w = (1 + 0.02 * rng.standard_normal(hdim)).astype(np.float32)
    want_r, want_d, want_out = ffn_oracle(orc, h, mix, norm_w, wg, wu, wd, hdim, ffn, epi)

    hd, Wg, Wu, Wd = dev(h), dev(wg.ravel()), dev(wu.ravel()), dev(wd.ravel())
    xq, aq = q8k_rows(m, hdim), q8k_rows(m, ffn)
    g, u, d = empty((m, ffn)), empty((m, ffn)), empty((m, hdim))
    tier.add_rmsnorm_q8k(hd, dev(mix), dev(norm_w), 1e-6, h_out=hd, xq=xq)
    if m == 1:
        tier.matvec_group([(12, Wg, ffn, hdim, xq, g), (12, Wu, ffn, hdim, xq, u)])
    else:
        tier.matmul(12, Wg, ffn, hdim, xq, m, g)
        tier.matmul(12, Wu, ffn, hdim, xq, m, u)
    tier.swiglu_q8k(g, u, xq=aq)
    if m == 1:
        tier.matvec(14, Wd, hdim, ffn, aq, d)
    else:
        tier.matmul(14, Wd, hdim, ffn, aq, m, d)
    assert_bits_equal(host(hd), want_r, "residual stream")
    assert_bits_equal(host(d), want_d, "ffn output")
    out = torch.empty_like(hd)
    tier.add_rmsnorm_q8k(hd, d, dev(norm_w), 1e-6, h_out=out, x_out=empty((m, hdim)))
    assert_bits_equal(host(out), want_out, "h + ffn output")
