"""GPU parity of the prefill GEMM over repacked weights: hip_gemm_pack_planes
turns a Q4_K / Q5_K / Q6_K matrix into int8 MFMA planes once, and
hip_matmul_planes must then equal the reference's token loop
(tensor_matmul_q{4k,5k,6k}_f32, slm/tensor.c:827-853, 898-919, 1012-1033)
bit for bit, in both float-epilogue families, exactly as hip_matmul_q* on
the original blocks does. The CPU oracle is the checker.

Cases: config 3 at M = 128 / 512 / 2048 and its Q6_K down projection,
ragged row groups (n not a multiple of 32) and token tiles, one super-block,
k at the limit, and blocks at the ends of their ranges (Q4_K / Q5_K scales
and quants at their maxima, Q6_K int8 scales over the whole byte range), so
the planes' hi digit reaches +-32 and the bsums reach their bounds. Both
kernels are reached for every type: up to 1024 32 x 32 output tiles the
super-blocks run across waves, beyond that 64-token tiles walk them."""
import numpy as np
import pytest

from cases import edge_rows
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


PLANE_SHAPES = [
    (12, 3584, 1024, 512), (12, 3584, 1024, 128), (14, 1024, 3584, 512),    # config 3
    (13, 2048, 1024, 96), (13, 1024, 2048, 33),
    (12, 100, 768, 37), (13, 65, 256, 1), (14, 63, 512, 65), (14, 129, 1280, 7),
    (12, 64, 256, 64), (12, 1, 512, 3), (12, 4100, 512, 600), (13, 3000, 256, 520),
    (14, 4096, 1024, 700), (12, 40, 65536, 9), (14, 33, 25600, 3),
]


@pytest.mark.parametrize("wtype,n,k,m", PLANE_SHAPES)
@pytest.mark.parametrize("epi,t", EPI_TIERS)
def test_matmul_planes(tier, orc, wtype, n, k, m, epi, t):
    lib = tier
    step(f"planes type={wtype} n={n} k={k} m={m} tier={t}")
    lib.set_tier(t)
    w = synth.blocks(wtype, n, k, seed=m, tag=wtype)
    x = synth.activations(m, k, seed=m + 1)
    if m >= 4:
        x[1:4] = edge_rows(k)[[0, 6, 7]]               # zero / huge / subnormal rows
    xq = orc.quantize_for(wtype, x)
    planes = lib.pack_planes(wtype, dev(w), n, k)
    got = host(lib.matmul_planes(wtype, planes, n, k, dev(xq), m))
    want = orc.matmul_xq(wtype, w, n, k, xq, m, epi)
    assert_bits_equal(got, want, f"planes {wtype} {m}x{n}x{k}")


def _extreme_blocks(wtype, n, k, seed):
    """Blocks whose folded weights reach the ends of the planes' range."""
    w = synth.blocks(wtype, n, k, seed=seed, tag=wtype)
    nbk = n * (k // 256)
    blk = w.reshape(nbk, -1)
    rng = np.random.default_rng(seed)
    if wtype in (12, 13):
        sc = np.full((nbk, 8), 63, np.int64)
        mn = np.full((nbk, 8), 63, np.int64)
        half = nbk // 2                                # the other half keeps random scales
        blk[:half, 4:16] = synth.pack_scales_mins(sc[:half], mn[:half])
        blk[:half, (16 if wtype == 12 else 48):] = 0xFF  # quants 15 (Q5_K: 31 with the qh bits)
        if wtype == 13:
            blk[:half, 16:48] = 0xFF
    else:
        blk[:, 192:208] = rng.integers(-128, 128, (nbk, 16)).astype(np.int8).view(np.uint8)
        blk[: nbk // 4, 192:208] = np.int8(-128).view(np.uint8)   # -128 * (0 - 32) = 4096
        blk[: nbk // 8, 0:192] = 0
        blk[nbk // 4: nbk // 2, 192:208] = np.uint8(127)          # 127 * (0 - 32) = -4064
        blk[nbk // 4: nbk // 2, 0:192] = 0
    return w


# (96, 1024, 70): 9 output tiles, super-blocks across waves; (4096, 512,
# 300): 1280 tiles, 64-token tiles
@pytest.mark.parametrize("n,k,m", [(96, 1024, 70), (4096, 512, 300)])
@pytest.mark.parametrize("wtype", [12, 13, 14])
@pytest.mark.parametrize("epi,t", EPI_TIERS)
def test_matmul_planes_extremes(tier, orc, wtype, epi, t, n, k, m):
    lib = tier
    step(f"planes extremes type={wtype} tier={t} {n}x{k} m={m}")
    lib.set_tier(t)
    w = _extreme_blocks(wtype, n, k, seed=5)
    x = synth.activations(m, k, seed=9)
    x[0] = np.where(np.arange(k) % 2 == 0, 1.0, -1.0)  # quants of +-127: bsums at +-2032
    x[1] = -np.abs(x[1])                               # one sign throughout
    xq = orc.quantize_for(wtype, x)
    planes = lib.pack_planes(wtype, dev(w), n, k)
    got = host(lib.matmul_planes(wtype, planes, n, k, dev(xq), m))
    want = orc.matmul_xq(wtype, w, n, k, xq, m, epi)
    assert_bits_equal(got, want, f"planes extremes {wtype}")


def test_matmul_planes_m2048(lib, orc):
    step("planes config 3 M=2048")
    n, k, m = 3584, 1024, 2048
    w = synth.blocks(12, n, k, seed=0)
    x = synth.activations(m, k, seed=0)
    xq = lib.quantize_q8k(dev(x))
    planes = lib.pack_planes(12, dev(w), n, k)
    got = host(lib.matmul_planes(12, planes, n, k, xq, m))
    want = orc.matmul(12, w, n, k, x, oracle.TIER_EPI[lib.tier()], threads=16)
    assert_bits_equal(got, want, "planes M=2048")


def test_planes_rejects_bad_arguments(lib):
    import torch
    n, k = 64, 512
    w = dev(synth.blocks(12, n, k, seed=1))
    assert lib.planes_bytes(8, n, k) == 0                      # Q8_0 has no planes
    assert lib.planes_bytes(12, n, 300) == 0                   # k not a multiple of 256
    assert lib.planes_bytes(12, n, k) == ((n + 31) // 32) * (k // 256) * 17664
    assert lib.planes_bytes(14, n, k) == ((n + 31) // 32) * (k // 256) * 16640
    planes = torch.empty(lib.planes_bytes(12, n, k), dtype=torch.uint8, device="cuda")
    rc = lib.L.hip_gemm_pack_planes(8, w.data_ptr(), n, k, planes.data_ptr(), None)
    assert rc == 6                                             # QK_ERR_UNSUPPORTED
    rc = lib.L.hip_gemm_pack_planes(12, w.data_ptr(), n, k, w.data_ptr() + 16, None)
    assert rc == 1                                    # planes overlap the weights
    xq = torch.zeros(4 * (k // 256) * 292, dtype=torch.uint8, device="cuda")
    y = torch.empty(4 * n, dtype=torch.float32, device="cuda")
    rc = lib.L.hip_matmul_planes(12, planes.data_ptr(), n, k, xq.data_ptr(), 0, y.data_ptr(), None)
    assert rc == 1                                    # no tokens
    rc = lib.L.hip_matmul_planes(12, planes.data_ptr() + 4, n, k, xq.data_ptr(), 4, y.data_ptr(), None)
    assert rc == 1                                    # misaligned planes
