"""GPU parity of the chunked Gated DeltaNet prefill (hip_deltanet_chunked
and the host-seam body of chunked_ssm_step_f32) against the oracle, which
is pinned to the reference's own chunked_ssm_step_f32: outputs and carried
states bit for bit, one chunk and many, one head and a layer's sixteen."""
import numpy as np
import pytest

from conftest import assert_bits_equal
from test_deltanet_oracle import ssm_inputs

pytestmark = pytest.mark.gpu


def dev(a):
    import torch
    return torch.from_numpy(np.ascontiguousarray(a)).cuda()


def host(t):
    import torch
    torch.cuda.synchronize()
    return t.cpu().numpy()


def step(msg):
    print(f"[gpu] {msg}", flush=True)


def state0(H, kd, vd, seed, zero=False):
    if zero:
        return np.zeros((H, kd, vd), np.float32)
    return (np.random.default_rng(seed).standard_normal((H, kd, vd)) * 0.05).astype(np.float32)


@pytest.mark.parametrize("n", [1, 2, 17, 63, 64])
@pytest.mark.parametrize("zero_rows", [False, True])
def test_deltanet_one_chunk(lib, orc, n, zero_rows):
    step(f"deltanet one chunk n={n} zero_rows={zero_rows}")
    q, k, v, g, b = ssm_inputs(n, seed=n, zero_rows=zero_rows and n > 3)
    for zero in (True, False):
        st = state0(1, 128, 128, n, zero)
        want_o, want_s = orc.chunked_step(q[:, 0], k[:, 0], v[:, 0], g[:, 0], b[:, 0], st[0])
        dst = dev(st)
        out = lib.deltanet_chunked(dev(q), dev(k), dev(v), dev(g), dev(b), dst)
        assert_bits_equal(host(out)[:, 0], want_o, f"out n={n}")
        assert_bits_equal(host(dst)[0], want_s, f"state n={n}")


@pytest.mark.parametrize("n_tok", [64, 200, 512])
def test_deltanet_layer(lib, orc, n_tok):
    """Sixteen heads of 128, the model's shape, over several chunks (512
    tokens: the config-4 prompt)."""
    step(f"deltanet layer n_tok={n_tok} heads=16")
    q, k, v, g, b = ssm_inputs(n_tok, H=16, seed=n_tok)
    st = state0(16, 128, 128, n_tok)
    want_o, want_s = orc.deltanet_chunked(q, k, v, g, b, st)
    dst = dev(st)
    out = lib.deltanet_chunked(dev(q), dev(k), dev(v), dev(g), dev(b), dst)
    assert_bits_equal(host(out), want_o, "out")
    assert_bits_equal(host(dst), want_s, "state")


@pytest.mark.parametrize("H,dim,n_tok", [(64, 32, 300), (300, 16, 130), (16, 128, 1100)])
def test_deltanet_chunk_groups(lib, orc, H, dim, n_tok):
    """Calls whose chunks span several groups of the state-free phases
    (at most 256 (chunk, head) slots per group): 64 heads run 5 chunks as
    4 + 1, 300 heads one chunk per group, 16 heads 18 chunks as 16 + 2."""
    step(f"deltanet chunk groups H={H} dim={dim} n_tok={n_tok}")
    q, k, v, g, b = ssm_inputs(n_tok, H=H, kd=dim, vd=dim, seed=H + n_tok)
    st = state0(H, dim, dim, H)
    want_o, want_s = orc.deltanet_chunked(q, k, v, g, b, st)
    dst = dev(st)
    out = lib.deltanet_chunked(dev(q), dev(k), dev(v), dev(g), dev(b), dst)
    assert_bits_equal(host(out), want_o, "out")
    assert_bits_equal(host(dst), want_s, "state")


@pytest.mark.parametrize("n_tok", [1, 200])
def test_deltanet_layer_host(lib, orc, n_tok):
    """hip_qk_deltanet_layer_host: the layer from host buffers laid out as
    slm_forward_ssm_batch holds them."""
    step(f"deltanet layer host n_tok={n_tok}")
    q, k, v, g, b = ssm_inputs(n_tok, H=16, seed=n_tok + 3, zero_rows=n_tok > 3)
    st = state0(16, 128, 128, n_tok + 3)
    want_o, want_s = orc.deltanet_chunked(q, k, v, g, b, st)
    out, new_st = lib.deltanet_layer_host(q, k, v, g, b, st)
    assert_bits_equal(out, want_o, "out")
    assert_bits_equal(new_st, want_s, "state")


def test_deltanet_other_head_dims(lib, orc):
    step("deltanet kd=64 vd=96 heads=3")
    q, k, v, g, b = ssm_inputs(100, H=3, kd=64, vd=96, seed=5)
    st = state0(3, 64, 96, 5)
    want_o, want_s = orc.deltanet_chunked(q, k, v, g, b, st)
    dst = dev(st)
    out = lib.deltanet_chunked(dev(q), dev(k), dev(v), dev(g), dev(b), dst)
    assert_bits_equal(host(out), want_o, "out")
    assert_bits_equal(host(dst), want_s, "state")


def test_deltanet_ragged_head_dims(lib, orc):
    # v_hd not a multiple of the 8 state columns a workgroup carries, k_hd
    # not a multiple of 4, and a partial last chunk (130 = 2 x 64 + 2)
    step("deltanet kd=40 vd=52 heads=5 n_tok=130")
    q, k, v, g, b = ssm_inputs(130, H=5, kd=40, vd=52, seed=6)
    st = state0(5, 40, 52, 6)
    want_o, want_s = orc.deltanet_chunked(q, k, v, g, b, st)
    dst = dev(st)
    out = lib.deltanet_chunked(dev(q), dev(k), dev(v), dev(g), dev(b), dst)
    assert_bits_equal(host(out), want_o, "out")
    assert_bits_equal(host(dst), want_s, "state")


def test_deltanet_host_seam(lib, orc):
    """The body the seam gives chunked_ssm_step_f32: host buffers, one head."""
    step("deltanet host seam")
    for n in (1, 33, 64):
        q, k, v, g, b = ssm_inputs(n, seed=n + 7)
        st = state0(1, 128, 128, n)[0]
        want = orc.chunked_step(q[:, 0], k[:, 0], v[:, 0], g[:, 0], b[:, 0], st)
        got = lib.deltanet_host(q[:, 0], k[:, 0], v[:, 0], g[:, 0], b[:, 0], st)
        assert_bits_equal(got[0], want[0], f"out n={n}")
        assert_bits_equal(got[1], want[1], f"state n={n}")


def test_deltanet_rejects_bad_shapes(lib):
    import torch
    from conftest import qk
    step("deltanet argument checks")
    n, H, kd = 4, 2, 129                               # head dim past QK_DELTANET_MAX_HD
    q = torch.zeros((n, H, kd), device="cuda")
    gb = torch.zeros((n, H), device="cuda")
    with pytest.raises(qk.QKError):
        lib.deltanet_chunked(q, q, torch.zeros((n, H, 128), device="cuda"), gb, gb,
                             torch.zeros((H, kd, 128), device="cuda"))
    with pytest.raises(qk.QKError):                    # a chunk holds at most 64 tokens
        lib.deltanet_host(np.zeros((65, 128)), np.zeros((65, 128)), np.zeros((65, 128)), np.zeros(65),
                          np.zeros(65), np.zeros((128, 128)))
    q2 = torch.zeros((4, 2, 128), device="cuda")
    g2 = torch.zeros((4, 2), device="cuda")
    with pytest.raises(qk.QKError):                    # out written over v, which later phases still read
        lib.deltanet_chunked(q2, q2, q2, g2, g2, torch.zeros((2, 128, 128), device="cuda"), out=q2)
    buf = torch.zeros(2 * 128 * 128 + 1024, device="cuda")
    with pytest.raises(qk.QKError, match="state overlaps an input"):   # the state is written while k is read
        lib.deltanet_chunked(q2, buf[:1024].view(4, 2, 128), q2, g2, g2, buf[512:512 + 2 * 128 * 128].view(2, 128, 128))
    with pytest.raises(qk.QKError):                    # head dim past QK_DELTANET_MAX_HD, host layer
        lib.deltanet_layer_host(np.zeros((4, 2, 129)), np.zeros((4, 2, 129)), np.zeros((4, 2, 128)),
                                np.zeros((4, 2)), np.zeros((4, 2)), np.zeros((2, 129, 128)))
