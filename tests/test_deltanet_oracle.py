"""The chunked Gated DeltaNet restatement (qko_chunked_step and the chunk
loop of slm_forward_ssm_batch): against the reference's own
chunked_ssm_step_f32 compiled from its sources, against the recurrent
form of the same recurrence in float64, and against the one-token
identity the reference states (slm/chunked.c:45-62)."""
import numpy as np
import pytest


def ssm_inputs(n, H=1, kd=128, vd=128, seed=0, zero_rows=False):
    """Inputs shaped as slm_forward_ssm_batch builds them: q, k L2-normalized
    per head (q also scaled by 1/sqrt(kd)), v after SiLU, g = ssm_a *
    softplus (negative), beta a sigmoid."""
    rng = np.random.default_rng(seed)
    q = rng.standard_normal((n, H, kd))
    k = rng.standard_normal((n, H, kd))
    q = q / np.linalg.norm(q, axis=2, keepdims=True) / np.sqrt(kd)
    k = k / np.linalg.norm(k, axis=2, keepdims=True)
    v = rng.standard_normal((n, H, vd))
    v = v / (1 + np.exp(-v))
    g = -np.log1p(np.exp(rng.standard_normal((n, H)))) * rng.uniform(0.2, 2.0, (n, H))
    beta = 1 / (1 + np.exp(-rng.standard_normal((n, H))))
    if zero_rows:                                      # exercise the reference's zero-coefficient skips
        q[n // 2] = 0
        k[n // 3] = 0
        beta[n // 4] = 0
    f = lambda a: np.asarray(a, np.float32)
    return f(q), f(k), f(v), f(g), f(beta)


def recurrent64(q, k, v, g, beta, state):
    """The Gated DeltaNet recurrence token by token in float64
    (autoregressive_ref, slm/qwen.c:1146-1190): S *= exp(g); kv = S^T k;
    S += k (x) (v - kv) * beta; o = S^T q."""
    n, H, kd = q.shape
    S = state.astype(np.float64).copy()
    out = np.zeros((n, H, v.shape[2]))
    for t in range(n):
        for h in range(H):
            S[h] *= np.exp(np.float64(g[t, h]))
            kv = S[h].T @ k[t, h].astype(np.float64)
            delta = (v[t, h] - kv) * beta[t, h]
            S[h] += np.outer(k[t, h], delta)
            out[t, h] = S[h].T @ q[t, h].astype(np.float64)
    return out, S


@pytest.mark.parametrize("n", [1, 2, 17, 63, 64])
@pytest.mark.parametrize("zero_rows", [False, True])
def test_chunked_step_matches_reference(orc, ref, n, zero_rows):
    q, k, v, g, b = ssm_inputs(n, seed=n, zero_rows=zero_rows and n > 3)
    rng = np.random.default_rng(n + 100)
    for state in (np.zeros((128, 128), np.float32), (rng.standard_normal((128, 128)) * 0.1).astype(np.float32)):
        a = orc.chunked_step(q[:, 0], k[:, 0], v[:, 0], g[:, 0], b[:, 0], state)
        c = ref.chunked_step(q[:, 0], k[:, 0], v[:, 0], g[:, 0], b[:, 0], state)
        assert np.array_equal(a[0].view(np.uint32), c[0].view(np.uint32)), f"out n={n}"
        assert np.array_equal(a[1].view(np.uint32), c[1].view(np.uint32)), f"state n={n}"


def test_chunked_step_other_head_dims(orc, ref):
    q, k, v, g, b = ssm_inputs(40, kd=64, vd=96, seed=9)
    st = np.zeros((64, 96), np.float32)
    a = orc.chunked_step(q[:, 0], k[:, 0], v[:, 0], g[:, 0], b[:, 0], st)
    c = ref.chunked_step(q[:, 0], k[:, 0], v[:, 0], g[:, 0], b[:, 0], st)
    assert np.array_equal(a[0].view(np.uint32), c[0].view(np.uint32))
    assert np.array_equal(a[1].view(np.uint32), c[1].view(np.uint32))


@pytest.mark.parametrize("n", [1, 8, 64, 200])
def test_chunk_loop_is_the_recurrence(orc, n):
    """Chunked (any chunk split) and recurrent forms are the same algebra:
    agreement to float32 accumulation noise over several chunks and heads
    pins every term (a dropped decay, a sign, a transposed product would
    be off by O(1))."""
    q, k, v, g, b = ssm_inputs(n, H=3, seed=n)
    rng = np.random.default_rng(7)
    state = (rng.standard_normal((3, 128, 128)) * 0.05).astype(np.float32)
    out, st = orc.deltanet_chunked(q, k, v, g, b, state)
    ro, rs = recurrent64(q, k, v, g, b, state)
    assert np.max(np.abs(out - ro)) <= 2e-5 * max(1.0, np.max(np.abs(ro)))
    assert np.max(np.abs(st - rs)) <= 2e-5 * max(1.0, np.max(np.abs(rs)))


def test_one_token_identity(orc):
    """slm/chunked.c:45-62: with a zero state, one token gives
    out = (K . Q) V beta and state = K (x) V beta, up to rounding."""
    q, k, v, g, b = ssm_inputs(1, seed=3)
    out, st = orc.chunked_step(q[:, 0], k[:, 0], v[:, 0], g[:, 0], b[:, 0], np.zeros((128, 128), np.float32))
    kq = np.dot(k[0, 0].astype(np.float64), q[0, 0])
    np.testing.assert_allclose(out[0], kq * v[0, 0] * b[0, 0], rtol=1e-5, atol=1e-7)
    np.testing.assert_allclose(st, np.outer(k[0, 0], v[0, 0] * b[0, 0]), rtol=1e-5, atol=1e-7)
