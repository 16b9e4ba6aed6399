"""GPU parity: libqk (through its C ABI) against the CPU oracle on the same
inputs. Bar: bit-exact for quantizers, dequant and every row dot (both
float-epilogue families), identical argmax token; top-k as a set.

Sizes: the benchmark configurations 0-3 at full size (the decode GEMV,
the decode set, the LM head, the prefill GEMM), plus ragged and edge
shapes."""
import numpy as np
import pytest

from cases import edge_rows, special_rows
from conftest import assert_bits_equal, oracle, qk, synth

pytestmark = pytest.mark.gpu

EPI_TIERS = [(oracle.EPI_SEPARATE, qk.TIER_SCALAR), (oracle.EPI_FUSED, qk.TIER_AVX2)]


def dev(a):
    import torch
    return torch.from_numpy(np.ascontiguousarray(a)).cuda()


def host(t):
    import torch
    torch.cuda.synchronize()
    return t.cpu().numpy()


def step(msg):
    print(f"[gpu] {msg}", flush=True)


# ---- quantizers ---------------------------------------------------------------

@pytest.mark.parametrize("k", [256, 1024, 3584, 16384])
def test_quantize_q8k_bit_exact(lib, orc, k):
    step(f"quantize_q8k k={k}")
    x = np.concatenate([edge_rows(k), special_rows(k), synth.activations(37, k, seed=k)])
    got = host(lib.quantize_q8k(dev(x)))
    np.testing.assert_array_equal(got, orc.quantize_q8k(x))


@pytest.mark.parametrize("k", [32, 1024, 2080])
def test_quantize_q8_0_bit_exact(lib, orc, k):
    step(f"quantize_q8_0 k={k}")
    x = np.concatenate([edge_rows(k), special_rows(k), synth.activations(21, k, seed=k)])
    got = host(lib.quantize_q8_0(dev(x)))
    np.testing.assert_array_equal(got, orc.quantize_q8_0(x))


def test_quantize_prefill_rows(lib, orc):
    step("quantize_q8k m=512 k=1024")
    x = synth.activations(512, 1024, seed=0)
    np.testing.assert_array_equal(host(lib.quantize_q8k(dev(x))), orc.quantize_q8k(x))


# ---- dequant ---------------------------------------------------------------------

@pytest.mark.parametrize("wtype", [12, 13, 14])
def test_dequant_bit_exact(lib, orc, wtype):
    step(f"dequant type={wtype}")
    w = synth.blocks(wtype, 33, 1024, seed=2, tag=wtype)
    nb = w.size // qk.BLOCK_BYTES[wtype]
    got = host(lib.dequant(wtype, dev(w.ravel()), nb))
    assert_bits_equal(got, orc.dequant(wtype, w, nb), f"dequant {wtype}")


# ---- decode GEMV -------------------------------------------------------------------

SHAPES = [
    (12, 3584, 1024), (13, 2048, 1024), (13, 512, 1024), (13, 1024, 2048),
    (14, 1024, 3584), (8, 1024, 1024),                     # config 1
    (12, 7, 256), (12, 33, 768), (12, 65, 1280), (13, 19, 512), (14, 17, 768),
    (14, 100, 2560), (12, 40, 16384), (14, 9, 16384), (8, 45, 96), (8, 3, 16384),
    (13, 21, 8192), (8, 70, 512),                          # Q5_K rows of two items; Q8_0 512 rows path
    (12, 40000, 256), (13, 40000, 256),                    # more tiles than workgroups: items in a loop
    (12, 9, 65536), (13, 3, 25600), (14, 5, 65536), (8, 7, 65536),   # k up to the 65536 limit
]


@pytest.mark.parametrize("wtype,n,k", SHAPES)
@pytest.mark.parametrize("epi,t", EPI_TIERS)
def test_matvec(tier, orc, wtype, n, k, epi, t):
    lib = tier
    step(f"matvec type={wtype} n={n} k={k} tier={t}")
    lib.set_tier(t)
    w = synth.blocks(wtype, n, k, seed=n, tag=wtype)
    if wtype == 8:                                     # quants of -128 (a valid GGUF byte): the first block
        w[0, 2:34] = 0x80                              # of row 0 and the last block of the last row
        w[-1, -32:] = 0x80
    x = np.concatenate([synth.activations(2, k, seed=k), edge_rows(k)[[0, 6, 7]]])
    xq = orc.quantize_for(wtype, x)
    wd = dev(w)
    xqd = dev(xq)
    for r in range(x.shape[0]):
        got = host(lib.matvec(wtype, wd, n, k, xqd[r]))
        want = orc.matmul_xq(wtype, w, n, k, xq[r:r + 1], 1, epi)[0]
        assert_bits_equal(got, want, f"row {r}")


def test_matvec_group_matches_single(lib, orc):
    step("matvec_group config 1")
    import torch
    specs = [(12, 3584, 1024), (12, 3584, 1024), (14, 1024, 3584), (13, 2048, 1024),
             (13, 512, 1024), (13, 1024, 2048), (8, 1024, 1024)]
    items, wants = [], []
    for i, (t, n, k) in enumerate(specs):
        w = synth.blocks(t, n, k, seed=1, tag=i)
        x = synth.activations(1, k, seed=1, tag=i)
        xq = orc.quantize_for(t, x)
        y = torch.empty(n, dtype=torch.float32, device="cuda")
        items.append((t, dev(w), n, k, dev(xq[0]), y))
        wants.append(orc.matmul_xq(t, w, n, k, xq, 1, oracle.TIER_EPI[lib.tier()])[0])
    lib.matvec_group(items)
    for (t, _, n, k, _, y), want in zip(items, wants):
        assert_bits_equal(host(y), want, f"group type {t} {n}x{k}")


F32_SHAPES = [(12, 3584, 1024), (14, 1024, 3584), (13, 2048, 1024), (13, 1024, 2048), (8, 1024, 1024),
              (8, 70, 512), (8, 45, 96), (8, 3, 16384), (12, 33, 768), (13, 21, 8192), (14, 100, 2560),
              (12, 40, 16384), (14, 9, 16384), (12, 40000, 256), (14, 30000, 1024),
              (12, 9, 65536), (8, 5, 65536)]             # rows quantized into 78 / 74 KB of LDS


@pytest.mark.parametrize("wtype,n,k", F32_SHAPES)
@pytest.mark.parametrize("epi,t", EPI_TIERS)
def test_matvec_group_f32_quantizes_in_launch(tier, orc, wtype, n, k, epi, t):
    # fp32 rows in, the workgroups quantize them: the result must be the
    # reference's quantize-then-dot (tensor_matmul_*_f32 at one token),
    # including rows whose quantization hits the edge cases
    lib = tier
    import torch
    step(f"matvec_group_f32 type={wtype} n={n} k={k} tier={t}")
    lib.set_tier(t)
    w = synth.blocks(wtype, n, k, seed=n + 7, tag=wtype)
    xs = np.concatenate([synth.activations(2, k, seed=k + 3), edge_rows(k)[[0, 1, 3, 6, 7]], special_rows(k)])
    wd = dev(w)
    for r in range(xs.shape[0]):
        xd = dev(xs[r])
        y = torch.empty(n, dtype=torch.float32, device="cuda")
        lib.matvec_group_f32([(wtype, wd, n, k, xd, y)])
        want = orc.matmul(wtype, w, n, k, xs[r:r + 1], epi)[0]
        assert_bits_equal(host(y), want, f"row {r}")


def test_matvec_group_f32_layer(lib, orc):
    # config 1 as one dispatch from fp32 activations, entries sharing rows
    # the way a decode layer does
    import torch
    step("matvec_group_f32 config 1 layer")
    k_rows = {1024: synth.activations(1, 1024, seed=60)[0], 3584: synth.activations(1, 3584, seed=61)[0],
              2048: synth.activations(1, 2048, seed=62)[0]}
    xd = {k: dev(v) for k, v in k_rows.items()}
    specs = [(12, 3584, 1024), (12, 3584, 1024), (14, 1024, 3584), (13, 2048, 1024),
             (13, 512, 1024), (13, 1024, 2048), (8, 1024, 1024)]
    items, wants = [], []
    for i, (t, n, k) in enumerate(specs):
        w = synth.blocks(t, n, k, seed=63, tag=i)
        y = torch.empty(n, dtype=torch.float32, device="cuda")
        items.append((t, dev(w), n, k, xd[k], y))
        wants.append(orc.matmul(t, w, n, k, k_rows[k][None], oracle.TIER_EPI[lib.tier()])[0])
    lib.matvec_group_f32(items)
    for (t, _, n, k, _, y), want in zip(items, wants):
        assert_bits_equal(host(y), want, f"type {t} {n}x{k}")


def test_quantize_then_matvec_on_device(lib, orc):
    step("quantize + matvec chain")
    k, n = 1024, 3584
    w = synth.blocks(12, n, k, seed=0)
    x = synth.activations(1, k, seed=0)
    xq = lib.quantize_q8k(dev(x))
    got = host(lib.matvec(12, dev(w), n, k, xq))
    want = orc.matmul(12, w, n, k, x, oracle.TIER_EPI[lib.tier()])[0]
    assert_bits_equal(got, want, "config 0")


# ---- chunked-prefill GEMM ------------------------------------------------------------

GEMM_SHAPES = [
    (12, 3584, 1024, 512), (12, 3584, 1024, 128), (14, 1024, 3584, 512),    # config 3
    (13, 2048, 1024, 96), (13, 1024, 2048, 33),
    (12, 100, 768, 37), (13, 65, 256, 1), (14, 63, 512, 65), (14, 129, 1280, 7),
    (12, 64, 256, 64), (12, 1, 512, 3), (12, 1000, 512, 650),   # super-blocks across waves up to 704 tokens
    (12, 2050, 512, 777),                                        # weight rows in registers, 32-token tiles
    # 64-row tiles for every type: 64-token tiles (at least 256 of them,
    # fewer than 192 128-token tiles, or more than 256 for Q5_K), else
    # 128-token tiles (Q4_K / Q5_K); the others run 32-row tiles with a
    # four-way k split
    (13, 4096, 1024, 512), (14, 4096, 1024, 300), (12, 4160, 512, 260),
    (12, 8256, 256, 128), (13, 2112, 256, 1100),
    (12, 40, 65536, 9), (14, 33, 25600, 3),                                  # k up to the limit
    # 128-token tiles (at least 192 of them) with partial row and token
    # tiles, and a single super-block
    (12, 4100, 512, 300), (13, 3000, 256, 520),
    # Q8_0: config 1's matrix and the model's ssm_alpha / ssm_beta at a
    # 512-token prompt; a step of one block (65 = 8 * 8 + 1); partial row
    # and token tiles; one block; k at the limit
    (8, 1024, 1024, 512), (8, 16, 1024, 512), (8, 33, 2080, 65), (8, 45, 96, 37),
    (8, 100, 512, 129), (8, 1, 32, 1), (8, 70, 65536, 5),
]


@pytest.mark.parametrize("wtype,n,k,m", GEMM_SHAPES)
@pytest.mark.parametrize("epi,t", EPI_TIERS)
def test_matmul_gemm(tier, orc, wtype, n, k, m, epi, t):
    lib = tier
    step(f"matmul type={wtype} n={n} k={k} m={m} tier={t}")
    lib.set_tier(t)
    w = synth.blocks(wtype, n, k, seed=m, tag=wtype)
    if wtype == 8:
        w[0, 2:34] = 0x80                              # quants of -128 (a valid GGUF byte)
    x = synth.activations(m, k, seed=m + 1)
    if m >= 4:
        x[1:4] = edge_rows(k)[[0, 6, 7]]               # zero / huge / subnormal rows
    xq = orc.quantize_for(wtype, x)
    got = host(lib.matmul(wtype, dev(w), n, k, dev(xq), m))
    want = orc.matmul_xq(wtype, w, n, k, xq, m, epi)
    assert_bits_equal(got, want, f"gemm {wtype} {m}x{n}x{k}")


def test_matmul_gemm_m2048(lib, orc):
    step("matmul config 3 M=2048")
    n, k, m = 3584, 1024, 2048
    w = synth.blocks(12, n, k, seed=0)
    x = synth.activations(m, k, seed=0)
    xq = lib.quantize_q8k(dev(x))
    got = host(lib.matmul(12, dev(w), n, k, xq, m))
    want = orc.matmul(12, w, n, k, x, oracle.TIER_EPI[lib.tier()], threads=16)
    assert_bits_equal(got, want, "gemm M=2048")


# ---- LM head ---------------------------------------------------------------------------

# Group sizes of the top-k bound (maxima of 1, 4 or 16 GEMV workgroups,
# at most 512 of them): k <= 32 uses 16, (248320, 40) and (9000, 64) use
# 4, (248320, 256) and (5000, 256) use 1, (300, 200) has fewer maxima
# than k (no bound).
# Past 1024 tiles the LM-head waves run several items with two register
# sets in turn: (16400, 1024) has 1025 tiles; (100003, 2048), (50001,
# 4096) and (262147, 256) have rows of 8, 16 and 4 groups (the last with
# three groups past the row end) and a partial last tile.
@pytest.mark.parametrize("n,k,topk", [(248320, 1024, 40), (31040, 1024, 40), (5000, 512, 256), (77, 256, 1),
                                      (300, 256, 200), (9000, 256, 64), (248320, 1024, 256), (31040, 1024, 100),
                                      (16400, 1024, 40), (100003, 2048, 40), (50001, 4096, 10),
                                      (262147, 256, 40)])
def test_lmhead_argmax_topk(lib, orc, n, k, topk):
    step(f"lmhead n={n} k={k} topk={topk}")
    w = synth.blocks(14, n, k, seed=2)
    x = synth.activations(1, k, seed=2)
    xq = orc.quantize_q8k(x)
    epi = oracle.TIER_EPI[lib.tier()]
    want = orc.matmul_xq(14, w, n, k, xq, 1, epi)[0]
    logits, am, ti, tv = lib.lmhead(dev(w), n, k, dev(xq[0]), topk=topk)
    assert_bits_equal(host(logits), want, "logits")
    assert int(host(am)[0]) == orc.argmax(want)
    ti, tv = host(ti), host(tv)
    ri, rv = orc.topk_collect(want, topk)
    kth = np.sort(rv)[0]
    if (want == kth).sum() == 1:                   # no tie at the k-th value
        assert set(ti.tolist()) == set(ri.tolist())
    assert_bits_equal(tv, want[ti], "topk values")
    assert (np.diff(tv) <= 0).all()


@pytest.mark.parametrize("n,k,topk", [(31040, 1024, 40), (5000, 512, 256), (16400, 1024, 40), (262147, 256, 40)])
@pytest.mark.parametrize("epi,t", EPI_TIERS)
def test_lmhead_both_tiers(tier, orc, n, k, topk, epi, t):
    # the LM-head GEMV is instantiated per float-epilogue family
    lib = tier
    step(f"lmhead n={n} k={k} topk={topk} tier={t}")
    lib.set_tier(t)
    w = synth.blocks(14, n, k, seed=21)
    xq = orc.quantize_q8k(synth.activations(1, k, seed=21))
    want = orc.matmul_xq(14, w, n, k, xq, 1, epi)[0]
    logits, am, ti, tv = lib.lmhead(dev(w), n, k, dev(xq[0]), topk=topk)
    assert_bits_equal(host(logits), want, "logits")
    assert int(host(am)[0]) == orc.argmax(want)
    ri, rv = orc.topk_collect(want, topk)
    if (want == np.sort(rv)[0]).sum() == 1:
        assert set(host(ti).tolist()) == set(ri.tolist())
    assert_bits_equal(host(tv), want[host(ti)], "topk values")


F16_NAN = np.uint16(0x7E00)


def _q6k_nan_rows(w, rows):
    """Give Q6_K rows an fp16 NaN d (bytes 208-209 of every block), so
    their logits are NaN whatever the activations."""
    nb = w.shape[1] // 210
    for r in rows:
        for b in range(nb):
            w[r, 210 * b + 208:210 * b + 210] = np.frombuffer(F16_NAN.tobytes(), np.uint8)


@pytest.mark.parametrize("case", ["row0", "middle", "all"])
def test_lmhead_argmax_nan_rules(lib, orc, case):
    # sample_argmax (slm/model.c:401-412): a NaN logit at row 0 keeps
    # index 0 (nothing compares greater than NaN); a NaN anywhere else
    # never wins; an all-NaN row gives 0
    step(f"lmhead NaN rule {case}")
    k, n, topk = 512, 9000, 40
    w = synth.blocks(14, n, k, seed=9)
    xq = orc.quantize_q8k(synth.activations(1, k, seed=9))
    epi = oracle.TIER_EPI[lib.tier()]
    clean = orc.matmul_xq(14, w, n, k, xq, 1, epi)[0]
    top = orc.argmax(clean)
    if case == "row0":
        _q6k_nan_rows(w, [0])
    elif case == "middle":
        _q6k_nan_rows(w, [5, 1000, top, n - 1])    # the true maximum becomes NaN too
    else:
        _q6k_nan_rows(w, range(n))
    want = orc.matmul_xq(14, w, n, k, xq, 1, epi)[0]
    assert np.isnan(want).sum() == {"row0": 1, "middle": 4, "all": n}[case]
    logits, am, ti, tv = lib.lmhead(dev(w), n, k, dev(xq[0]), topk=topk)
    assert_bits_equal(host(logits), want, "logits")
    got = int(host(am)[0])
    assert got == orc.argmax(want), (got, orc.argmax(want))
    # the top-k set is topk_collect's (slm/sampler.c:70-93): a NaN of the
    # first k rows keeps its fill slot (it never compares as the worst
    # slot), a later NaN never enters, and a NaN at row 0 freezes the fill
    # (rows 0..k-1); ranked numbers first (value-descending), then the NaN
    # rows by row
    ci, _ = orc.topk_collect(want, topk)
    gi, gv = host(ti), host(tv)
    assert set(gi.tolist()) == set(ci.tolist())
    assert_bits_equal(gv, want[gi], "top-k values")
    nums = ~np.isnan(gv)
    assert nums.sum() == 0 or np.all(nums[:nums.sum()])          # numbers before NaN rows
    assert np.all(np.diff(gv[nums]) <= 0)
    assert np.all(np.diff(gi[~nums]) > 0)
    if case in ("row0", "all"):
        assert got == 0
        assert set(gi.tolist()) == set(range(topk))
    else:
        assert got != top and not np.isnan(want[got])
        nan_fill = {r for r in range(topk) if np.isnan(want[r])}
        assert nan_fill == {5} and 5 in set(gi.tolist())


def test_lmhead_two_streams_concurrently(lib, orc):
    # two LM-head calls in flight at once on two streams, each with its own
    # matrix and activations: per-stream selection scratch keeps them apart
    import torch
    step("lmhead on two streams")
    k, topk = 1024, 40
    epi = oracle.TIER_EPI[lib.tier()]
    cases = []
    for i, n in enumerate((40000, 31040)):
        w = synth.blocks(14, n, k, seed=30 + i)
        xq = orc.quantize_q8k(synth.activations(1, k, seed=30 + i))
        cases.append((n, w, xq, orc.matmul_xq(14, w, n, k, xq, 1, epi)[0]))
    streams = [torch.cuda.Stream(), torch.cuda.Stream()]
    on_dev = [(dev(w), dev(xq[0])) for (_, w, xq, _) in cases]
    torch.cuda.synchronize()
    for rep in range(3):
        outs = []
        for (n, _, _, _), (wd, xd), s in zip(cases, on_dev, streams):
            with torch.cuda.stream(s):
                outs.append(lib.lmhead(wd, n, k, xd, topk=topk, want_logits=False))
        torch.cuda.synchronize()
        for (n, w, xq, want), (_, am, ti, tv) in zip(cases, outs):
            assert int(host(am)[0]) == orc.argmax(want), f"rep {rep} n={n}"
            ri, rv = orc.topk_collect(want, topk)
            if (want == np.sort(rv)[0]).sum() == 1:
                assert set(host(ti).tolist()) == set(ri.tolist()), f"rep {rep} n={n}"
            assert_bits_equal(host(tv), want[host(ti)], f"rep {rep} n={n} topk values")


def test_lmhead_argmax_ties(lib, orc):
    step("lmhead argmax rules")
    # duplicate rows give tied logits: the first index must win
    k, n = 256, 4096
    w = synth.blocks(14, n, k, seed=5)
    w[3000] = w[17]
    w[2000] = w[17]
    xq = orc.quantize_q8k(synth.activations(1, k, seed=5))
    epi = oracle.TIER_EPI[lib.tier()]
    want = orc.matmul_xq(14, w, n, k, xq, 1, epi)[0]
    top = orc.argmax(want)
    w[[3000, 2000]] = w[top]                       # tie the maximum at later rows
    want = orc.matmul_xq(14, w, n, k, xq, 1, epi)[0]
    logits, am, _, _ = lib.lmhead(dev(w), n, k, dev(xq[0]), topk=0)
    assert int(host(am)[0]) == orc.argmax(want) == top


# ---- host seam ---------------------------------------------------------------------------

# Q5_K / Q6_K prefill GEMMs go through int8 MFMA planes packed at the
# first one (both kernels: up to 1024 output tiles and beyond)
@pytest.mark.parametrize("wtype,n,k,m", [(12, 3584, 1024, 1), (13, 512, 1024, 1), (14, 1024, 3584, 1),
                                          (8, 1024, 1024, 1), (8, 64, 1024, 21), (12, 3584, 1024, 64),
                                          (13, 512, 1024, 21), (14, 1024, 3584, 9), (14, 1024, 3584, 600),
                                          (13, 2048, 1024, 700)])
def test_matmul_host_seam(lib, orc, wtype, n, k, m):
    step(f"host seam type={wtype} n={n} k={k} m={m}")
    w = synth.blocks(wtype, n, k, seed=3, tag=wtype)
    x = synth.activations(m, k, seed=3)
    got = lib.matmul_host(wtype, w, n, k, x)
    want = orc.matmul(wtype, w, n, k, x, oracle.TIER_EPI[lib.tier()])
    assert_bits_equal(got, want, "tensor_matmul seam")
    lib.unregister_weight(w)


@pytest.mark.parametrize("t", [12, 13, 14])
def test_host_seam_reload_at_same_address(lib, orc, t):
    # a model unloaded and another loaded at the same host addresses (the
    # GGUF mapping reused): hip_qk_unregister_range, which the seam calls
    # before munmap, drops the old device copy (and, for Q5_K / Q6_K, the
    # MFMA planes the first prefill made), so the new bytes are used
    import ctypes as C
    step(f"host seam reload at the same address type={t}")
    n, k = 512, 1024
    buf = synth.blocks(t, n, k, seed=40)
    x = synth.activations(2, k, seed=40)
    epi = oracle.TIER_EPI[lib.tier()]
    assert_bits_equal(lib.matmul_host(t, buf, n, k, x), orc.matmul(t, buf, n, k, x, epi), "first model")
    lib.L.hip_qk_unregister_range.argtypes = [C.c_void_p, C.c_size_t]
    assert lib.L.hip_qk_unregister_range(buf.ctypes.data_as(C.c_void_p), buf.nbytes) == 1
    assert lib.L.hip_qk_device_weight(buf.ctypes.data_as(C.c_void_p)) is None
    buf[...] = synth.blocks(t, n, k, seed=41)      # the next model, same address
    assert_bits_equal(lib.matmul_host(t, buf, n, k, x), orc.matmul(t, buf, n, k, x, epi), "second model")
    # a range that covers no weight drops nothing
    assert lib.L.hip_qk_unregister_range(C.c_void_p(buf.ctypes.data + buf.nbytes), 4096) == 0
    lib.unregister_weight(buf)


def test_lmhead_host_seam(lib, orc):
    step("lmhead host seam")
    n, k = 20000, 1024
    w = synth.blocks(14, n, k, seed=4)
    x = synth.activations(1, k, seed=4)
    logits, am, ti, tv = lib.lmhead_host(w, n, k, x[0], topk=40)
    want = orc.matmul(14, w, n, k, x, oracle.TIER_EPI[lib.tier()])[0]
    assert_bits_equal(logits, want, "logits")
    assert am == orc.argmax(want)
    lib.unregister_weight(w)


# ---- argument checks ---------------------------------------------------------------------

def test_rejects_bad_shapes(lib):
    # the C ABI's own checks, called directly: every call is rejected on the
    # host before any launch
    import ctypes as C
    import torch
    w = torch.zeros(144 * 4, dtype=torch.uint8, device="cuda")
    xq = torch.zeros(292 * 4, dtype=torch.uint8, device="cuda")
    y = torch.zeros(4, dtype=torch.float32, device="cuda")
    wp, xp, yp = C.c_void_p(w.data_ptr()), C.c_void_p(xq.data_ptr()), C.c_void_p(y.data_ptr())
    L = lib.L
    assert L.hip_matvec_q4k(wp, 4, 1000, xp, yp, None) == 1          # k % 256
    assert L.hip_matvec_q4k(C.c_void_p(w.data_ptr() + 1), 1, 256, xp, yp, None) == 1   # misaligned
    assert L.hip_matvec_q4k(wp, 1, 65536 + 256, xp, yp, None) == 1   # k above 65536
    assert L.hip_matvec_q8_0(wp, 1, 65536 + 32, xp, yp, None) == 1
    assert L.hip_matmul_q8_0(wp, 1, 65536 + 32, xp, 2, yp, None) == 1
    assert L.hip_matmul_q8_0(wp, 4, 64, xp, 0, yp, None) == 1         # m = 0
    # grids whose 32-bit work-item count would wrap
    fp = C.c_void_p(y.data_ptr())
    assert L.hip_quantize_q8k(fp, (1 << 26) + 1, 256, xp, None) == 1
    assert L.hip_quantize_q8_0(fp, (1 << 27) + 1, 32, xp, None) == 1
    assert L.hip_dequant_q4k(wp, (1 << 26) + 1, yp, None) == 1
    assert L.hip_add_rmsnorm_q8k(fp, None, fp, C.c_float(1e-6), 1 << 24, 256, fp, None, xp, None) == 1
    assert L.hip_matmul_q8_0(wp, 4, 64, xp, 65535 * 32 + 1, yp, None) == 1   # above 65535 token tiles of 32
    assert "m=" in lib.last_error()
    assert L.hip_matvec_q4k(wp, 0, 256, xp, yp, None) == 1           # empty
    assert L.hip_matvec_q4k(None, 1, 256, xp, yp, None) == 1         # null
    am = torch.zeros(1, dtype=torch.int32, device="cuda")
    assert L.hip_lmhead_q6k_argmax_topk(wp, 4, 256, xp, 5, yp, C.c_void_p(am.data_ptr()), None, None, None) == 1
    assert L.hip_matmul_q4k(wp, 4, 256, xp, 0, yp, None) == 1        # m = 0
    assert L.hip_matmul_q4k(wp, 4, 1000, xp, 2, yp, None) == 1       # k % 256
    assert "k=" in lib.last_error() or "m=" in lib.last_error()
    # the host seam: bad shapes and a token count above the GEMM's bound
    # are refused before any host or device buffer is touched
    import numpy as _np
    hw = _np.zeros(144 * 4, _np.uint8)
    hx = _np.zeros(256, _np.float32)
    ho = _np.zeros(4, _np.float32)
    hp = lambda a: a.ctypes.data_as(C.c_void_p)
    assert L.hip_qk_matmul_host(hp(hw), 12, 4, 1000, hp(hx), 1, hp(ho)) == 1
    assert L.hip_qk_matmul_host(hp(hw), 12, 4, 256, hp(hx), 65535 * 64 + 1, hp(ho)) == 1
    assert "n_tok" in lib.last_error()
    assert L.hip_qk_matmul_host(hp(hw), 8, 4, 64, hp(hx), 65535 * 32 + 1, hp(ho)) == 1
    assert "n_tok" in lib.last_error()
    assert L.hip_qk_matmul_host(hp(hw), 7, 4, 256, hp(hx), 1, hp(ho)) == 6
    assert L.hip_qk_init(1) != 0                                       # another device while initialized
    with pytest.raises(ValueError):                                   # binding's size guard
        lib.matvec(12, w, 8, 256, xq, y)


def _valkey(v):
    """Order-preserving uint32 key of a float32 (value order; NaN lowest)."""
    b = np.asarray(v, np.float32).view(np.uint32).astype(np.uint64)
    b = np.where(np.asarray(v) == 0, 0, b)
    key = np.where(b & 0x80000000, ~b & 0xffffffff, b | 0x80000000)
    return np.where(np.isnan(v), 0, key).astype(np.uint64)


def test_lmhead_topk_many_ties_ranked(lib, orc):
    # 20 distinct rows repeated 1100 times: the maximum ties at 1100 rows,
    # so more candidates pass the filter than one block ranks directly
    # (1024) but fewer than the candidate buffer holds (4096); the k-th
    # largest of them is selected first, then ranked. Ties go to low rows.
    step("lmhead top-k selected candidates")
    period, reps, k, topk = 20, 1100, 256, 10
    w = np.tile(synth.blocks(14, period, k, seed=8), (reps, 1))
    n = period * reps
    xq = orc.quantize_q8k(synth.activations(1, k, seed=8))
    want = orc.matmul_xq(14, w, n, k, xq, 1, oracle.TIER_EPI[lib.tier()])[0]
    top = orc.argmax(want)
    # every logit whose key shares the maximum's top 16 bits passes
    passing = int((_valkey(want) >= (int(_valkey(want[top])) & 0xffff0000)).sum())
    assert 1024 < passing <= 4096, passing
    logits, am, ti, tv = lib.lmhead(dev(w), n, k, dev(xq[0]), topk=topk)
    assert_bits_equal(host(logits), want, "logits")
    assert int(host(am)[0]) == top
    np.testing.assert_array_equal(host(ti), top + period * np.arange(topk))
    assert_bits_equal(host(tv), want[host(ti)], "topk values")
    ri, _ = orc.topk_collect(want, topk)
    assert set(ri.tolist()) == set((top + period * np.arange(topk)).tolist())


def test_lmhead_topk_flat_logits_fallback(lib, orc):
    # identical rows: every logit ties, far more than the candidate buffer
    # passes the filter and the exact fallback runs; ties go to low rows
    step("lmhead top-k fallback")
    n, k, topk = 20000, 256, 10
    row = synth.blocks(14, 1, k, seed=6)
    w = np.repeat(row, n, axis=0)
    xq = orc.quantize_q8k(synth.activations(1, k, seed=6))
    logits, am, ti, tv = lib.lmhead(dev(w), n, k, dev(xq[0]), topk=topk)
    want = orc.matmul_xq(14, w, n, k, xq, 1, oracle.TIER_EPI[lib.tier()])[0]
    assert_bits_equal(host(logits), want, "logits")
    assert int(host(am)[0]) == 0
    np.testing.assert_array_equal(host(ti), np.arange(topk))
    ri, _ = orc.topk_collect(want, topk)
    assert set(ri.tolist()) == set(range(topk))


# ---- concurrency and streams -------------------------------------------------------------

def test_host_seam_from_several_threads(lib, orc):
    # The reference's model (and so its weights) may be shared by several
    # contexts on several host threads (slm/slm.h:33-36); the seam's weight
    # registry and staging buffers must hold up under concurrent calls.
    import threading
    step("host seam, 4 threads")
    cases = [(12, 512, 1024, 1), (13, 256, 1024, 3), (14, 128, 1024, 1), (8, 256, 1024, 2)]
    data = []
    for i, (t, n, k, m) in enumerate(cases):
        w = synth.blocks(t, n, k, seed=11, tag=i)
        x = synth.activations(m, k, seed=11 + i)
        data.append((t, w, n, k, x, orc.matmul(t, w, n, k, x, oracle.TIER_EPI[lib.tier()])))
    errors = []

    def worker(i):
        try:
            t, w, n, k, x, want = data[i]
            for _ in range(5):
                got = lib.matmul_host(t, w, n, k, x)
                assert_bits_equal(got, want, f"thread {i}")
        except Exception as e:              # reported below, on the main thread
            errors.append(e)

    threads = [threading.Thread(target=worker, args=(i,)) for i in range(len(data))]
    for th in threads:
        th.start()
    for th in threads:
        th.join(120)
    assert not any(th.is_alive() for th in threads)
    assert not errors, errors[0]
    for t, w, n, k, x, want in data:
        lib.unregister_weight(w)


def test_matvec_on_a_side_stream(lib, orc):
    # Entry points take the caller's stream; work queued there is ordered
    # after the caller's own work on it and finishes before its sync.
    import torch
    step("matvec on a side stream")
    t, n, k = 12, 3584, 1024
    w = synth.blocks(t, n, k, seed=12)
    x = synth.activations(1, k, seed=12)
    want = orc.matmul(t, w, n, k, x, oracle.TIER_EPI[lib.tier()])[0]
    side = torch.cuda.Stream()
    with torch.cuda.stream(side):
        wd = dev(w)
        xd = torch.from_numpy(x).cuda()
        xq = lib.quantize_q8k(xd)[0]
        y = lib.matvec(t, wd, n, k, xq)
    side.synchronize()
    assert_bits_equal(host(y), want, "side stream")


def test_graph_capture_replays(lib, orc):
    # quantize -> GEMV group -> LM head (argmax, top-k) captured once in a
    # HIP graph and replayed on new inputs, with eager work between the
    # replays; every replay must equal the oracle. The library clears its
    # own counters with kernels (no memset nodes in the graph).
    import torch
    step("graph capture and replay")
    k, n4, nv, topk = 1024, 512, 4096, 8
    epi = oracle.TIER_EPI[lib.tier()]
    q4 = synth.blocks(12, n4, k, seed=13)
    q6 = synth.blocks(14, nv, k, seed=14)
    wq4, wq6 = dev(q4), dev(q6)
    x_static = torch.zeros((1, k), dtype=torch.float32, device="cuda")
    xq_static = torch.empty((1, (k // 256) * 292), dtype=torch.uint8, device="cuda")
    y4 = torch.empty(n4, dtype=torch.float32, device="cuda")
    logits = torch.empty(nv, dtype=torch.float32, device="cuda")

    def run():
        lib.quantize_q8k(x_static, out=xq_static)
        lib.matvec_group([(12, wq4, n4, k, xq_static[0], y4)])
        return lib.lmhead(wq6, nv, k, xq_static[0], topk=topk, logits=logits)

    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):                  # warm-up: the stream's LM-head scratch exists before capture
        run()
    torch.cuda.current_stream().wait_stream(side)
    torch.cuda.synchronize()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g, stream=side):
        _, am, ti, tv = run()
    for rep in range(3):
        x = synth.activations(1, k, seed=100 + rep)
        x_static.copy_(torch.from_numpy(x))
        _ = (x_static * 2.0).sum()                 # eager work between replays
        g.replay()
        torch.cuda.synchronize()
        want4 = orc.matmul(12, q4, n4, k, x, epi)[0]
        wantv = orc.matmul(14, q6, nv, k, x, epi)[0]
        assert_bits_equal(host(y4), want4, f"replay {rep} gemv")
        assert_bits_equal(host(logits), wantv, f"replay {rep} logits")
        assert int(host(am)[0]) == orc.argmax(wantv)
        ri, _ = orc.topk_collect(wantv, topk)
        if (wantv == np.sort(wantv)[-topk]).sum() == 1:
            assert set(host(ti).tolist()) == set(ri.tolist())
        assert_bits_equal(host(tv), wantv[host(ti)], f"replay {rep} topk values")
