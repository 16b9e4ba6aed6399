"""Pins the CPU oracle (oracle/qk_oracle.c) before it is trusted as the
checker of the GPU path.

Three independent anchors:
  * golden vectors written by the reference's own C (tests/golden/*.npz,
    both float-epilogue families: scalar and AVX2-FMA tiers);
  * the reference compiled from its sources (oracle/_ref), when present;
  * closed forms: exhaustive fp16 conversions against numpy, magic-number
    rounding against np.rint, the 6-bit scale unpack against its packing,
    integer dot products against an int64 numpy restatement, and
    quantizer invariants.
"""
import os

import numpy as np
import pytest

from cases import edge_rows, special_rows
from conftest import assert_bits_equal, bits, oracle, synth

GOLD = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden")
TYPES = {"q4k": 12, "q5k": 13, "q6k": 14, "q8_0": 8}


def gold(name):
    return np.load(os.path.join(GOLD, name), allow_pickle=False)


# ---- fp16 / rounding closed forms --------------------------------------------

def test_f16_widening_exhaustive(orc):
    h = np.arange(65536, dtype=np.uint32)
    want = h.astype(np.uint16).view(np.float16).astype(np.float32)
    got = np.array([orc.f16_to_f32(int(v)) for v in h], np.float32)
    nan = np.isnan(want)
    assert np.isnan(got[nan]).all()
    assert_bits_equal(got[~nan], want[~nan], "fp16->fp32")


def test_f16_narrowing_rne(orc):
    rng = np.random.default_rng(0)
    v = np.concatenate([
        rng.normal(0, 1, 20000), rng.normal(0, 1e-5, 20000), rng.normal(0, 3e4, 20000),
        rng.uniform(-7e-8, 7e-8, 20000),
    ]).astype(np.float32)
    # exact halfway points between fp16 neighbours, subnormal and normal
    hs = np.arange(0, 0x7bff, 37, dtype=np.uint16).view(np.float16).astype(np.float32)
    mids = (hs[:-1].astype(np.float64) + np.nextafter(hs[:-1].astype(np.float16), np.float16(np.inf)).astype(np.float64)) / 2
    edge = np.array([65504, 65519.99, 65520, 65536, 1e9, 2.0 ** -24, 2.0 ** -25, 2.0 ** -25 * 1.0001,
                     2.0 ** -26, 6.1e-5, 0.0, -0.0, np.inf, -np.inf], np.float32)
    v = np.concatenate([v, mids.astype(np.float32), -mids.astype(np.float32), edge])
    want = v.astype(np.float16).view(np.uint16)
    got = np.array([orc.f32_to_f16(x) for x in v], np.uint16)
    np.testing.assert_array_equal(got, want)


def test_nearest_int_is_round_half_even(orc):
    rng = np.random.default_rng(1)
    v = np.concatenate([rng.uniform(-300, 300, 5000), np.arange(-130, 130) + 0.5]).astype(np.float32)
    got = np.array([orc.nearest_int(x) for x in v])
    np.testing.assert_array_equal(got, np.rint(v.astype(np.float64)).astype(np.int64))


# ---- 6-bit scale/min unpack ------------------------------------------------------

def test_scale_min_inverts_packing(orc):
    rng = np.random.default_rng(2)
    sc = rng.integers(0, 64, (500, 8))
    mn = rng.integers(0, 64, (500, 8))
    packed = synth.pack_scales_mins(sc, mn)
    for r in range(0, 500, 7):
        for j in range(8):
            assert orc.scale_min(packed[r], j) == (sc[r, j], mn[r, j])


def test_scale_min_exhaustive_vs_reference(orc, ref):
    # each (sc, m) of sub-block j depends on at most two bytes: sweep them all
    s = np.zeros(12, np.uint8)
    for j in range(8):
        for a in range(0, 256, 3):
            for b in range(0, 256, 5):
                s[:] = 0x5a
                if j < 4:
                    s[j], s[j + 4] = a, b
                else:
                    s[j + 4], s[j - 4], s[j] = a, b, (a * 7 + b) & 0xff
                assert orc.scale_min(s, j) == ref.scale_min(s, j)


# ---- quantizers --------------------------------------------------------------------

def test_q8k_golden(orc):
    g = gold("quant.npz")
    np.testing.assert_array_equal(orc.quantize_q8k(g["x"]), g["q8k"])


def test_q8_0_golden(orc):
    g = gold("quant.npz")
    np.testing.assert_array_equal(orc.quantize_q8_0(g["x"]), g["q8_0"])


def _q8k_fields(xq_row):
    blk = xq_row.reshape(-1, 292)
    d = blk[:, 0:4].copy().view(np.float32).ravel()
    qs = blk[:, 4:260].copy().view(np.int8)
    bs = blk[:, 260:292].copy().view(np.int16)
    return d, qs, bs


def test_q8k_invariants(orc):
    x = np.concatenate([edge_rows(1024), synth.activations(8, 1024, seed=5)])
    xq = orc.quantize_q8k(x)
    for r in range(x.shape[0]):
        d, qs, bs = _q8k_fields(xq[r])
        np.testing.assert_array_equal(bs, qs.reshape(-1, 16, 16).sum(-1).astype(np.int16).reshape(bs.shape))
        xb = x[r].reshape(-1, 256)
        for b in range(xb.shape[0]):
            a = np.abs(xb[b])
            if a.max() == 0:
                assert d[b] == 0 and not qs[b].any()
                continue
            if not np.isfinite(np.float32(-127.0) / xb[b][int(np.argmax(a))]):
                # |xmax| < 127 * 2^-128: iscale = -inf, the reference stores
                # d = -0 / +0 and every quant saturates at -128.
                assert d[b] == 0 and (qs[b] == -128).all()
                continue
            assert (np.abs(qs[b].astype(np.int32)) <= 127).all()
            i = int(np.argmax(a))                 # first index of the maximum
            assert qs[b][i] == -127               # the max element always maps to -127
            assert np.sign(d[b]) == -np.sign(xb[b][i])


def test_q8k_tie_and_halves(orc):
    x = edge_rows(256)
    xq = orc.quantize_q8k(x)
    d, qs, _ = _q8k_fields(xq[1])                 # x[5] = -3, x[77] = +3: first wins
    assert d[0] > 0 and qs[0][5] == -127 and qs[0][77] == 127
    d, qs, _ = _q8k_fields(xq[3])                 # xmax = -127: iscale = 1, halves -> even
    assert d[0] == 1.0
    h = x[3]
    np.testing.assert_array_equal(qs[0].astype(np.int64), np.clip(np.rint(h.astype(np.float64)), -128, 127))


def test_q8_0_halves_away_from_zero(orc):
    x = edge_rows(32)
    xq = orc.quantize_q8_0(x[9:10])               # amax = 127 -> d = 1, id = 1
    q = xq[0, 2:34].view(np.int8).astype(np.int64)
    v = x[9].astype(np.float64)
    np.testing.assert_array_equal(q, np.sign(v) * np.floor(np.abs(v) + 0.5))


def test_quantizers_vs_reference(orc, ref):
    x = np.concatenate([edge_rows(2048), special_rows(2048), synth.activations(32, 2048, seed=9)])
    np.testing.assert_array_equal(orc.quantize_q8k(x), ref.quantize_q8k(x))
    np.testing.assert_array_equal(orc.quantize_q8k(x), ref.quantize_q8k(x, quants_h=True))
    np.testing.assert_array_equal(orc.quantize_q8_0(x), ref.quantize_q8_0(x))


# ---- dot products --------------------------------------------------------------------

def unpack_int_weights(wtype, blocks):
    """Independent numpy restatement: (nb, 256) integer weights, per-element
    integer scale and min (ggml block formats, simd/quants.h:95-130)."""
    b = blocks.reshape(-1, {12: 144, 13: 176, 14: 210}[wtype])
    nb = b.shape[0]
    if wtype in (12, 13):
        s = b[:, 4:16].astype(np.int64)
        sc = np.zeros((nb, 8), np.int64)
        mn = np.zeros((nb, 8), np.int64)
        sc[:, :4], mn[:, :4] = s[:, 0:4] & 63, s[:, 4:8] & 63
        sc[:, 4:] = (s[:, 8:12] & 15) | ((s[:, 0:4] >> 6) << 4)
        mn[:, 4:] = (s[:, 8:12] >> 4) | ((s[:, 4:8] >> 6) << 4)
        qs = b[:, 16:144] if wtype == 12 else b[:, 48:176]
        q = np.zeros((nb, 256), np.int64)
        for c in range(4):
            q[:, 64 * c:64 * c + 32] = qs[:, 32 * c:32 * c + 32] & 15
            q[:, 64 * c + 32:64 * c + 64] = qs[:, 32 * c:32 * c + 32] >> 4
            if wtype == 13:
                qh = b[:, 16:48].astype(np.int64)
                q[:, 64 * c:64 * c + 32] += ((qh >> (2 * c)) & 1) << 4
                q[:, 64 * c + 32:64 * c + 64] += ((qh >> (2 * c + 1)) & 1) << 4
        return q, np.repeat(sc, 32, axis=1), np.repeat(mn, 32, axis=1)
    ql, qh = b[:, 0:128].astype(np.int64), b[:, 128:192].astype(np.int64)
    sc = b[:, 192:208].view(np.int8).astype(np.int64)
    q = np.zeros((nb, 256), np.int64)
    for h in range(2):
        for l in range(32):
            for qq in range(4):
                lo = ql[:, 64 * h + l + 32 * (qq & 1)]
                lo = (lo >> 4) if qq >= 2 else (lo & 15)
                q[:, 128 * h + 32 * qq + l] = lo | (((qh[:, 32 * h + l] >> (2 * qq)) & 3) << 4)
    return q, np.repeat(sc, 16, axis=1), None


@pytest.mark.parametrize("wtype", [12, 13, 14])
def test_block_integer_parts_brute_force(orc, wtype):
    w = synth.blocks(wtype, 16, 256, seed=3, tag=wtype)
    x = np.concatenate([synth.activations(4, 256, seed=3), edge_rows(256)[[1, 3, 5, 6]]])
    xq = orc.quantize_q8k(x)
    q, sc, mn = unpack_int_weights(wtype, w)
    for t in range(xq.shape[0]):
        _, qs, _ = _q8k_fields(xq[t])
        a = qs[0].astype(np.int64)
        for r in range(16):
            isum, mins = orc.block_ints(wtype, w[r], xq[t])
            if wtype == 14:
                want_isum = int((sc[r] * q[r] * a).sum())
                want_mins = int((sc[r] * a).sum())
            else:
                want_isum = int((sc[r] * q[r] * a).sum())
                want_mins = int((mn[r] * a).sum())
            assert (isum, mins) == (want_isum, want_mins), (t, r)


@pytest.mark.parametrize("name", list(TYPES))
def test_dots_golden_both_tiers(orc, name):
    g = gold("dots.npz")
    wt = TYPES[name]
    w, xq = g[f"{name}_w"], g[f"{name}_xq"]
    k = g[f"{name}_x"].shape[1]
    np.testing.assert_array_equal(orc.quantize_for(wt, g[f"{name}_x"]), xq)
    for tag, epi in (("sep", oracle.EPI_SEPARATE), ("fused", oracle.EPI_FUSED)):
        got = np.array([[orc.row_dot(wt, w[j], xq[t], k, epi) for j in range(w.shape[0])]
                        for t in range(xq.shape[0])], np.float32)
        assert_bits_equal(got, g[f"{name}_y_{tag}"], f"{name} {tag}")
    if wt != 14:
        # the fixture separates the two epilogues: a dropped/added FMA fails it
        assert (bits(g[f"{name}_y_sep"]) != bits(g[f"{name}_y_fused"])).any()


@pytest.mark.parametrize("name", ["q4k", "q5k", "q6k"])
def test_dequant_golden(orc, name):
    g = gold("dots.npz")
    wt = TYPES[name]
    w = g[f"{name}_w"]
    nb = w.size // {12: 144, 13: 176, 14: 210}[wt]
    assert_bits_equal(orc.dequant(wt, w, nb), g[f"{name}_deq"], name)


@pytest.mark.parametrize("wtype", [12, 13, 14])
def test_dequant_closed_form(orc, wtype):
    # With d = 1, dmin = 0 (Q4_K/Q5_K) the dequant is sc * q exactly; Q6_K
    # gives sc * (q - 32). Compare against the numpy unpacking.
    w = synth.blocks(wtype, 4, 512, seed=11, tag=wtype).reshape(-1, {12: 144, 13: 176, 14: 210}[wtype]).copy()
    one = np.array([1.0], np.float16).view(np.uint8)
    if wtype == 14:
        w[:, 208:210] = one
    else:
        w[:, 0:2] = one
        w[:, 2:4] = 0
    q, sc, _ = unpack_int_weights(wtype, w)
    want = (sc * (q - 32 if wtype == 14 else q)).astype(np.float32).ravel()
    np.testing.assert_array_equal(orc.dequant(wtype, w, w.shape[0]), want)


@pytest.mark.parametrize("wtype", [12, 13, 14, 8])
def test_matmul_vs_reference(orc, ref, wtype):
    k, n, m = 1024, 64, 3
    w = synth.blocks(wtype, n, k, seed=4, tag=wtype)
    x = np.concatenate([synth.activations(m, k, seed=4), edge_rows(k)[[0, 3, 6]]])
    want = ref.matmul(wtype, w, n, k, x)           # tensor_matmul_*_f32 itself
    epi = oracle.TIER_EPI[ref.dispatched_tier()]
    assert_bits_equal(orc.matmul(wtype, w, n, k, x, epi), want, "matmul")
    assert_bits_equal(ref.matmul(wtype, w, n, k, x, threads=4), want, "row-split baseline")


@pytest.mark.parametrize("wtype", [12, 13, 14, 8])
def test_every_tier_vs_reference(orc, ref, wtype):
    k, n = 768 if wtype != 8 else 96, 40
    w = synth.blocks(wtype, n, k, seed=6, tag=wtype)
    xq = orc.quantize_for(wtype, synth.activations(2, k, seed=6))
    for tier in ref.tiers():
        epi = oracle.TIER_EPI[tier]
        for t in range(2):
            got = np.array([orc.row_dot(wtype, w[j], xq[t], k, epi) for j in range(n)], np.float32)
            want = np.array([ref.row_dot(wtype, w[j], xq[t], k, tier) for j in range(n)], np.float32)
            assert_bits_equal(got, want, f"tier {tier}")


def test_dot_close_to_float_math(orc):
    # dequantized fp64 dot of the quantized activation agrees with the
    # integer path to float rounding (a sign or index slip would not)
    k = 1024
    for wtype in (12, 13, 14):
        w = synth.blocks(wtype, 8, k, seed=8, tag=wtype)
        x = synth.activations(1, k, seed=8)
        xq = orc.quantize_q8k(x)[0]
        d, qs, _ = _q8k_fields(xq)
        a = (qs.astype(np.float64) * d[:, None].astype(np.float64)).ravel()
        wd = orc.dequant(wtype, w, w.size // {12: 144, 13: 176, 14: 210}[wtype]).reshape(8, k).astype(np.float64)
        for r in range(8):
            got = orc.row_dot(wtype, w[r], xq, k, oracle.EPI_SEPARATE)
            want = float(wd[r] @ a)
            scale = float(np.abs(wd[r] * a).sum())
            assert abs(got - want) <= 1e-5 * scale + 1e-30, (wtype, r, got, want)


# ---- argmax / top-k -----------------------------------------------------------------

def test_select_golden(orc):
    g = gold("select.npz")
    assert orc.argmax(g["v"]) == int(g["argmax"]) == 10
    ti, tv = orc.topk_collect(g["v"], 40)
    np.testing.assert_array_equal(ti, g["topk_idx"])
    np.testing.assert_array_equal(tv, g["topk_val"])


def test_argmax_first_index_rules(orc):
    v = np.array([1.0, 3.0, 3.0, -1.0], np.float32)
    assert orc.argmax(v) == 1
    v = np.array([np.nan, 5.0, 2.0], np.float32)
    assert orc.argmax(v) == 0                        # v[0] NaN: nothing compares greater
    v = np.array([-0.0, 0.0, -1.0], np.float32)
    assert orc.argmax(v) == 0
