"""GPU parity of the sampler chain (hip_sample) against the oracle's
restatement of sample_with: the token, the penalized logits and the rng
state after every step, bit for bit, over the reference's parameter
space, adversarial logit orders (every logit entering topk_collect's
slots), ties, infinities and NaN, and a sampled sequence at the model's
vocabulary with the history kept on the device."""
import numpy as np
import pytest

from conftest import assert_bits_equal
from test_sampler_oracle import SAMPLERS, logit_rows

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


def check(lib, orc, logits, sp, st, hist, mask, what):
    tok_o, lg_o, st_o = orc.sample(logits, sp, st, hist, mask)
    lg = dev(logits)
    rng = dev(np.asarray(st, np.uint64).view(np.int64))
    h = dev(np.asarray(hist, np.int32)) if len(hist) else None
    tok = lib.sample(lg, sp, rng, h, len(hist), list(int(m) for m in mask))
    assert int(host(tok)[0]) == tok_o, what
    assert_bits_equal(host(lg), lg_o, what + " penalized logits")
    assert np.array_equal(host(rng).view(np.uint64), st_o), what + " rng"


@pytest.mark.parametrize("n", [1, 2, 39, 40, 41, 300, 5000, 1023, 1025, 70000])
def test_sample_matches_oracle(lib, orc, n):
    rng = np.random.default_rng(n)
    step(f"sample n={n}")
    for li, logits in enumerate(logit_rows(n, rng)):
        for si, sp in enumerate(SAMPLERS):
            st = orc.rng_seed(1000 * n + 10 * li + si)
            hist = rng.integers(-2, n + 2, rng.integers(0, 100)).astype(np.int32)
            mask = rng.integers(0, n, rng.integers(0, 3)).astype(np.int32)
            check(lib, orc, logits, sp, st, hist, mask, f"n={n} row={li} sampler={si}")


@pytest.mark.parametrize("window", [0, 5000, 4096, 64])
def test_sample_long_history_windows(lib, orc, window):
    """Windows past the 4096 ids the penalty stages in LDS run over many
    workgroups after the masks: a 12000-id history full of repeats and
    out-of-range ids, masks that are also in the history, and penalties
    that compound (1.3), shrink (0.7) and zero (0: -inf * 0 is NaN, so the
    mask has to land before the penalty)."""
    step(f"sample long history window={window}")
    n = 9000
    rng = np.random.default_rng(window + 1)
    hist = rng.integers(-3, n + 3, 12000).astype(np.int32)
    hist[::7] = 17                                     # one token repeated about 1700 times
    for pen in (1.3, 0.7, 0.0):
        sp = dict(temperature=0.8, top_k=40, top_p=0.9, min_p=0.05, repetition_penalty=pen,
                  repetition_window=window)
        logits = (rng.standard_normal(n) * 2).astype(np.float32)
        logits[17] = 0.5
        check(lib, orc, logits, sp, orc.rng_seed(window + 3), hist, np.array([17, int(hist[5]) % n], np.int32),
              f"window={window} penalty={pen}")


def test_sample_vocab_sequence_on_device(lib, orc):
    """64 steps at vocabulary 248320 with the default sampler: logits from
    a random walk (so later steps see repeated tokens in the window), the
    history appended on the device by pointing the token at its next
    entry, the rng carried in device memory."""
    import torch
    step("sample sequence vocab=248320")
    V, steps = 248320, 64
    sp = SAMPLERS[0]
    rng = np.random.default_rng(5)
    st = orc.rng_seed(77)
    d_rng = dev(st.view(np.int64))
    d_hist = torch.zeros(steps, dtype=torch.int32, device="cuda")
    hist = []
    base = (rng.standard_normal(V) * 2).astype(np.float32)
    for i in range(steps):
        logits = (base + rng.standard_normal(V).astype(np.float32) * 0.5).astype(np.float32)
        tok_o, _, st = orc.sample(logits, sp, st, hist)
        lib.sample(dev(logits), sp, d_rng, d_hist, i, token=d_hist[i:i + 1])
        got = int(host(d_hist[i:i + 1])[0])
        assert got == tok_o, f"step {i}"
        hist.append(tok_o)
    assert np.array_equal(host(d_rng).view(np.uint64), st)
    assert len(set(hist)) > 8


def test_sample_every_logit_enters(lib, orc):
    """Ascending logits: each one enters topk_collect's slots (the longest
    replay); descending: none after the first k; a plateau of equal
    values: ties keep the earlier slot."""
    step("sample adversarial orders")
    sp = dict(SAMPLERS[3])
    for n in (20000, 248320):
        up = np.linspace(-5, 5, n, dtype=np.float32)
        plateau = np.full(n, 1.0, np.float32)
        plateau[n // 3] = 2.0
        for logits in (up, up[::-1].copy(), plateau):
            check(lib, orc, logits, sp, orc.rng_seed(n), [], [], f"n={n}")


def test_sample_rejects_bad_arguments(lib):
    import torch
    from conftest import qk
    step("sample argument checks")
    lg = torch.zeros(100, device="cuda")
    rng = torch.zeros(2, dtype=torch.int64, device="cuda")
    sp = dict(SAMPLERS[0])
    with pytest.raises(qk.QKError):
        lib.sample(lg, sp, rng, mask=[1, 2, 3])           # at most two masked ids
    with pytest.raises(qk.QKError):
        lib.sample(lg, sp, None)                          # sampling needs the rng
    with pytest.raises(qk.QKError):                       # a NaN temperature samples too (slm/sampler.c:140)
        lib.sample(lg, dict(sp, temperature=float("nan")), None)
    lib.sample(lg, dict(sp, temperature=0.0), None)       # greedy does not
