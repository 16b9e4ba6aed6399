"""The allocation-free LM head (hip_lmhead_q6k_argmax_topk_noalloc) against
the allocating entry point, through the C ABI: same logits, argmax and
top-k on two calls in a row, the second with a smaller matrix, with and
without a caller logits buffer."""
import ctypes as C

import numpy as np
import pytest

from conftest import assert_bits_equal, oracle, qk, synth

pytestmark = pytest.mark.gpu


def _bind(lib):
    f = lib.L.hip_lmhead_q6k_argmax_topk_noalloc
    f.argtypes = [C.c_void_p, C.c_int64, C.c_int64, C.c_void_p, C.c_int, C.c_void_p, C.c_void_p,
                  C.c_void_p, C.c_void_p, C.c_void_p]
    return f


def _call(lib, f, w, n, k, xq, topk, logits):
    import torch
    am = torch.full((1,), -1, dtype=torch.int32, device="cuda")
    ti = torch.full((max(topk, 1),), -1, dtype=torch.int32, device="cuda")
    tv = torch.zeros(max(topk, 1), dtype=torch.float32, device="cuda")
    p = lambda t: C.c_void_p(0 if t is None else t.data_ptr())
    rc = f(p(w), n, k, p(xq), topk, p(logits), p(am), p(ti) if topk else None, p(tv) if topk else None,
           C.c_void_p(torch.cuda.current_stream().cuda_stream))
    if rc:
        raise qk.QKError(rc, lib.last_error())
    return am, ti[:topk], tv[:topk]


@pytest.mark.parametrize("with_logits", [True, False])
def test_noalloc_lmhead_matches_allocating(lib, orc, with_logits):
    import torch
    f = _bind(lib)
    k, topk = 1024, 40
    epi = oracle.TIER_EPI[lib.tier()]
    for n, seed in ((248320, 50), (31040, 51)):           # second call smaller
        print(f"[gpu] noalloc lmhead n={n} logits={with_logits}", flush=True)
        w = torch.from_numpy(synth.blocks(14, n, k, seed=seed)).cuda()
        xq = torch.from_numpy(orc.quantize_q8k(synth.activations(1, k, seed=seed))[0]).cuda()
        lg_ref, am_ref, ti_ref, tv_ref = lib.lmhead(w, n, k, xq, topk=topk)
        lg = torch.empty(n, dtype=torch.float32, device="cuda") if with_logits else None
        am, ti, tv = _call(lib, f, w, n, k, xq, topk, lg)
        torch.cuda.synchronize()
        assert int(am.cpu()[0]) == int(am_ref.cpu()[0])
        np.testing.assert_array_equal(ti.cpu().numpy(), ti_ref.cpu().numpy())
        assert_bits_equal(tv.cpu().numpy(), tv_ref.cpu().numpy(), f"topk values n={n}")
        if with_logits:
            assert_bits_equal(lg.cpu().numpy(), lg_ref.cpu().numpy(), f"logits n={n}")
        # and against the CPU oracle's pick
        want = orc.matmul_xq(14, w.cpu().numpy(), n, k, xq.cpu().numpy()[None], 1, epi)[0]
        assert int(am.cpu()[0]) == orc.argmax(want)


def test_noalloc_lmhead_limits(lib):
    import torch
    f = _bind(lib)
    w = torch.zeros(210 * 4, dtype=torch.uint8, device="cuda")
    xq = torch.zeros(292 * 4, dtype=torch.uint8, device="cuda")
    am = torch.zeros(1, dtype=torch.int32, device="cuda")
    p = lambda t: C.c_void_p(t.data_ptr())
    # no logits buffer and more rows than the static scratch holds: refused
    # on the host before any launch
    assert f(p(w), 262145, 1024, p(xq), 0, None, p(am), None, None, None) == 1
    assert "static scratch" in lib.last_error()
    assert f(p(w), 4, 1024, p(xq), 300, None, p(am), None, None, None) == 1      # topk above the maximum


def test_noalloc_lmhead_refuses_overlap_from_another_stream(lib, orc):
    """Two streams calling at once would share the static scratch: a call
    from another stream while the previous call is still queued fails with
    QK_ERR_ARG; once it has finished, or on the same stream, calls go
    through. (Stream a is held busy by a large fp32 matmul first, so the
    first call is certainly still queued when the second arrives.)"""
    import torch
    f = _bind(lib)
    n, k, topk = 31040, 1024, 8
    w = torch.from_numpy(synth.blocks(14, n, k, seed=60)).cuda()
    xq = torch.from_numpy(orc.quantize_q8k(synth.activations(1, k, seed=60))[0]).cuda()
    big = torch.randn(4096, 4096, device="cuda")
    a, b = torch.cuda.Stream(), torch.cuda.Stream()
    torch.cuda.synchronize()
    print("[gpu] noalloc overlap: busy stream a, then a call on a and one on b", flush=True)
    with torch.cuda.stream(a):
        for _ in range(4):
            big = big @ big * 1e-3
        am_a, _, _ = _call(lib, f, w, n, k, xq, topk, None)
    with torch.cuda.stream(b):
        with pytest.raises(qk.QKError) as e:
            _call(lib, f, w, n, k, xq, topk, None)
    assert e.value.rc == 1 and "in flight" in str(e.value)
    with torch.cuda.stream(a):
        am_a2, _, _ = _call(lib, f, w, n, k, xq, topk, None)        # same stream: ordered, allowed
    a.synchronize()
    with torch.cuda.stream(b):
        am_b, _, _ = _call(lib, f, w, n, k, xq, topk, None)         # the other one finished: allowed
    b.synchronize()
    assert int(am_a.cpu()[0]) == int(am_a2.cpu()[0]) == int(am_b.cpu()[0])
