"""The sampler chain: the oracle's restatement of sample_with (plus the
min_new masking and the rng) against the reference's own compiled code,
over random and adversarial logits and every kind of parameter."""
import numpy as np
import pytest

SAMPLERS = [
    dict(temperature=0.7, top_k=40, top_p=0.9, min_p=0.05, repetition_penalty=1.25, repetition_window=64),
    dict(temperature=1.3, top_k=0, top_p=0.0, min_p=0.0, repetition_penalty=1.0, repetition_window=0),
    dict(temperature=0.2, top_k=1, top_p=0.5, min_p=0.2, repetition_penalty=1.1, repetition_window=0),
    dict(temperature=1.0, top_k=256, top_p=0.95, min_p=0.0, repetition_penalty=1.5, repetition_window=8),
    dict(temperature=0.9, top_k=1000, top_p=1.0, min_p=0.5, repetition_penalty=0.8, repetition_window=3),
    dict(temperature=0.0, top_k=40, top_p=0.9, min_p=0.05, repetition_penalty=1.25, repetition_window=64),
    dict(temperature=-1.0, top_k=5, top_p=0.9, min_p=0.05, repetition_penalty=1.0, repetition_window=64),
]


def logit_rows(n, rng):
    """Random logits, coarse ones full of ties, vocab-ordered (every
    element enters topk_collect's slots), and rows with -inf, +inf and NaN."""
    signed_zeros = np.where(rng.random(n) < 0.5, np.float32(0.0), np.float32(-0.0)).astype(np.float32)
    signed_zeros[rng.integers(0, n, max(1, n // 7))] = 1.0
    rows = [(rng.standard_normal(n) * 3).astype(np.float32),
            np.round(rng.standard_normal(n) * 2).astype(np.float32),   # ties, and -0.0 beside +0.0
            np.sort(rng.standard_normal(n)).astype(np.float32),
            np.sort(rng.standard_normal(n))[::-1].astype(np.float32).copy()]
    r = (rng.standard_normal(n) * 3).astype(np.float32)
    r[rng.integers(0, n, max(1, n // 50))] = -np.inf
    rows.append(r)
    r = (rng.standard_normal(n) * 3).astype(np.float32)
    r[rng.integers(0, n, 2)] = np.inf
    rows.append(r)
    r = (rng.standard_normal(n) * 3).astype(np.float32)
    r[rng.integers(0, n, 3)] = np.nan
    rows.append(r)
    r = (rng.standard_normal(n) * 3).astype(np.float32)
    r[0] = np.nan
    rows.append(r)
    rows.append(np.full(n, -np.inf, np.float32))
    rows.append(signed_zeros)                          # -0 and +0 compare equal in every step
    return rows


@pytest.mark.parametrize("n", [1, 2, 39, 40, 41, 300, 5000])
def test_sample_oracle_matches_reference(orc, ref, n):
    rng = np.random.default_rng(n)
    for li, logits in enumerate(logit_rows(n, rng)):
        for si, sp in enumerate(SAMPLERS):
            st = orc.rng_seed(1000 * n + 10 * li + si)
            hist = rng.integers(-2, n + 2, rng.integers(0, 100)).astype(np.int32)
            mask = rng.integers(0, n, rng.integers(0, 3)).astype(np.int32)
            a = orc.sample(logits, sp, st, hist, mask)
            b = ref.sample(logits, sp, st, hist, mask)
            assert a[0] == b[0], (n, li, si)
            assert np.array_equal(a[1].view(np.uint32), b[1].view(np.uint32)), (n, li, si)
            assert np.array_equal(a[2], b[2]), (n, li, si)


def test_sample_oracle_vocab_sequence(orc, ref):
    """A 40-step sampled sequence at the model's vocabulary, history and
    rng carried from step to step as slm_generate_raw does."""
    rng = np.random.default_rng(9)
    sp = SAMPLERS[0]
    st_o = st_r = orc.rng_seed(42)
    hist = []
    for step in range(40):
        logits = (rng.standard_normal(248320) * 2.5).astype(np.float32)
        a = orc.sample(logits, sp, st_o, hist)
        b = ref.sample(logits, sp, st_r, hist)
        assert a[0] == b[0] and np.array_equal(a[2], b[2]), step
        st_o, st_r = a[2], b[2]
        hist.append(a[0])


def test_rng_seed_matches_reference(orc, ref):
    for seed in (0, 1, 42, 2 ** 63, 2 ** 64 - 1):
        assert np.array_equal(orc.rng_seed(seed), ref.rng_seed(seed))


@pytest.mark.parametrize("temperature", [0.0, 0.7])
def test_sample_mask_restore_closed_form(orc, ref, temperature):
    """slm_generate_raw saves the eos / eot logits before masking them and
    puts the saved values back after sample_with (slm/slm.c:309-333): a
    masked id ends at its value from before the mask (the repetition
    penalty never reaches it), an id masked twice ends at -inf (its
    second save), an id out of range is left alone; the other logits are
    penalized as usual."""
    n = 500
    rng = np.random.default_rng(3)
    logits = (rng.standard_normal(n) * 3).astype(np.float32)
    e1, e2 = 17, 311
    hist = np.array([e1, e2, 5, 5, 9], np.int32)
    sp = dict(temperature=temperature, top_k=40, top_p=0.9, min_p=0.05, repetition_penalty=1.25,
              repetition_window=0)
    for impl in (orc, ref):
        _, out, _ = impl.sample(logits, sp, orc.rng_seed(7), hist, np.array([e1, e2], np.int32))
        assert out[e1] == logits[e1] and out[e2] == logits[e2]
        pen = lambda v: v / np.float32(1.25) if v > 0 else v * np.float32(1.25)
        assert out[9] == np.float32(pen(logits[9]))
        _, out, _ = impl.sample(logits, sp, orc.rng_seed(7), hist, np.array([e1, e1], np.int32))
        assert out[e1] == -np.inf
        _, out, _ = impl.sample(logits, sp, orc.rng_seed(7), hist, np.array([-1, n + 5], np.int32))
        assert out[e1] == np.float32(pen(logits[e1]))
