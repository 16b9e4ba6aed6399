"""ctypes front end of the CPU checkers.

TEST INFRASTRUCTURE ONLY: imported by tests/, __graft_entry__.smoke()
and bench.py's cpu_baseline leg, never by the product path.

Two backends with one interface:

* ``Oracle`` -- ``oracle/libqk_oracle.so``, the C restatement
  (qk_oracle.c), always built by ``make -C oracle``.
* ``Ref`` -- ``oracle/_ref/libqkref.so``, the reference's own C compiled
  from its sources (ref_shim.c); present only where it was built.

Byte buffers are numpy uint8 arrays holding raw GGUF / Q8_K blocks.
"""
from __future__ import annotations

import ctypes as C
import os
import subprocess
from concurrent.futures import ThreadPoolExecutor

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
ORACLE_SO = os.path.join(HERE, "libqk_oracle.so")
REF_SO = os.path.join(HERE, "_ref", "libqkref.so")

Q8_0, Q4_K, Q5_K, Q6_K = 8, 12, 13, 14
BLOCK_BYTES = {Q8_0: 34, Q4_K: 144, Q5_K: 176, Q6_K: 210}
BLOCK_ELEMS = {Q8_0: 32, Q4_K: 256, Q5_K: 256, Q6_K: 256}
Q8K_BYTES = 292
EPI_SEPARATE, EPI_FUSED = 0, 1
# reference tier ids (simd/simd.c:208-229) -> oracle epilogue family
TIER_EPI = {0: EPI_SEPARATE, 1: EPI_SEPARATE, 2: EPI_FUSED, 3: EPI_FUSED}

_vp, _fp, _i64, _i32 = C.c_void_p, C.POINTER(C.c_float), C.c_int64, C.c_int32


def _ptr(a):
    return a.ctypes.data_as(C.c_void_p)


def build(quiet=True):
    """make -C oracle (the C restatement, and _ref when REF is present)."""
    out = subprocess.run(["make", "-C", HERE], capture_output=True, text=True)
    if out.returncode != 0:
        raise RuntimeError("oracle build failed:\n" + out.stdout + out.stderr)
    if not quiet:
        print(out.stdout)


def xq_bytes(wtype, k):
    return (k // 32) * 34 if wtype == Q8_0 else (k // 256) * Q8K_BYTES


class Oracle:
    """The C restatement (oracle/qk_oracle.c)."""

    name = "oracle"

    def __init__(self, path=ORACLE_SO):
        if not os.path.exists(path):
            build()
        L = C.CDLL(path)
        self.L = L
        L.qko_f16_to_f32.restype = C.c_float
        L.qko_f16_to_f32.argtypes = [C.c_uint16]
        L.qko_f32_to_f16.restype = C.c_uint16
        L.qko_f32_to_f16.argtypes = [C.c_float]
        L.qko_nearest_int.restype = C.c_int32
        L.qko_nearest_int.argtypes = [C.c_float]
        for f in ("qko_quantize_q8k", "qko_quantize_q8_0"):
            getattr(L, f).argtypes = [_vp, _vp, _i64]
            getattr(L, f).restype = None
        L.qko_scale_min.argtypes = [_vp, C.c_int, _vp, _vp]
        for f in ("qko_q4k_dot", "qko_q5k_dot", "qko_q6k_dot"):
            getattr(L, f).argtypes = [C.c_int, _vp, _vp, C.c_int]
            getattr(L, f).restype = C.c_float
        L.qko_q8_0_dot.argtypes = [_i64, _vp, _vp, C.c_int]
        L.qko_q8_0_dot.restype = C.c_float
        for f in ("qko_q4k_block_ints", "qko_q5k_block_ints", "qko_q6k_block_ints"):
            getattr(L, f).argtypes = [_vp, _vp, _vp, _vp]
        for f in ("qko_dequant_q4k", "qko_dequant_q5k", "qko_dequant_q6k"):
            getattr(L, f).argtypes = [_vp, _i64, _vp]
        L.qko_matmul.argtypes = [C.c_int, _vp, _i64, _i64, _vp, _i64, _vp, C.c_int, _i64, _i64]
        L.qko_matmul_xq.argtypes = L.qko_matmul.argtypes
        L.qko_argmax.argtypes = [_vp, _i64]
        L.qko_argmax.restype = C.c_int32
        L.qko_topk_collect.argtypes = [_vp, _i64, C.c_int32, _vp, _vp]
        L.qko_topk_collect.restype = C.c_int32
        L.qko_add_rmsnorm.argtypes = [_vp, _vp, _vp, C.c_float, _i64, _i64, _vp, _vp]
        L.qko_add_rmsnorm.restype = None
        L.qko_silu.argtypes = [_i64, _vp, _vp]
        L.qko_silu.restype = None
        L.qko_swiglu.argtypes = [_i64, _vp, _vp, _vp]
        L.qko_swiglu.restype = None
        L.qko_chunked_step.argtypes = [C.c_int, C.c_int, C.c_int] + [_vp] * 7
        L.qko_chunked_step.restype = None
        L.qko_deltanet_chunked.argtypes = [_i64, C.c_int, C.c_int, C.c_int] + [_vp] * 7
        L.qko_deltanet_chunked.restype = None
        L.qko_rng_seed.argtypes = [C.c_uint64, _vp]
        L.qko_rng_seed.restype = None
        L.qko_sample.argtypes = [_vp, _i64, C.c_float, C.c_int32, C.c_float, C.c_float, C.c_float, C.c_int32, _vp, _vp, C.c_int32, _vp, C.c_int32]
        L.qko_sample.restype = C.c_int32

    # -- scalars -------------------------------------------------------
    def f16_to_f32(self, h):
        return self.L.qko_f16_to_f32(int(h))

    def f32_to_f16(self, f):
        return self.L.qko_f32_to_f16(float(np.float32(f)))

    def nearest_int(self, v):
        return self.L.qko_nearest_int(float(np.float32(v)))

    def scale_min(self, s12, j):
        s = np.ascontiguousarray(s12, dtype=np.uint8)
        sc, m = C.c_uint8(), C.c_uint8()
        self.L.qko_scale_min(_ptr(s), j, C.byref(sc), C.byref(m))
        return sc.value, m.value

    # -- quantizers ----------------------------------------------------
    def quantize_q8k(self, x):
        x = np.ascontiguousarray(x, dtype=np.float32)
        m, k = x.reshape(-1, x.shape[-1]).shape
        out = np.zeros((m, (k // 256) * Q8K_BYTES), np.uint8)
        for t in range(m):
            self.L.qko_quantize_q8k(_ptr(x.reshape(m, k)[t]), _ptr(out[t]), k)
        return out

    def quantize_q8_0(self, x):
        x = np.ascontiguousarray(x, dtype=np.float32)
        m, k = x.reshape(-1, x.shape[-1]).shape
        out = np.zeros((m, (k // 32) * 34), np.uint8)
        for t in range(m):
            self.L.qko_quantize_q8_0(_ptr(x.reshape(m, k)[t]), _ptr(out[t]), k)
        return out

    def quantize_for(self, wtype, x):
        return self.quantize_q8_0(x) if wtype == Q8_0 else self.quantize_q8k(x)

    # -- dots ----------------------------------------------------------
    def row_dot(self, wtype, wrow, xq, k, epi):
        wrow = np.ascontiguousarray(wrow, np.uint8)
        xq = np.ascontiguousarray(xq, np.uint8)
        nb = k // BLOCK_ELEMS[wtype]
        if wtype == Q8_0:
            return self.L.qko_q8_0_dot(k, _ptr(wrow), _ptr(xq), epi)
        f = {Q4_K: self.L.qko_q4k_dot, Q5_K: self.L.qko_q5k_dot, Q6_K: self.L.qko_q6k_dot}[wtype]
        return f(nb, _ptr(wrow), _ptr(xq), epi)

    def block_ints(self, wtype, wblock, xqblock):
        f = {Q4_K: self.L.qko_q4k_block_ints, Q5_K: self.L.qko_q5k_block_ints,
             Q6_K: self.L.qko_q6k_block_ints}[wtype]
        a, b = C.c_int32(), C.c_int32()
        wb = np.ascontiguousarray(wblock, np.uint8)
        xb = np.ascontiguousarray(xqblock, np.uint8)
        f(_ptr(wb), _ptr(xb), C.byref(a), C.byref(b))
        return a.value, b.value

    def dequant(self, wtype, w, nblocks):
        w = np.ascontiguousarray(w, np.uint8)
        out = np.empty(nblocks * 256, np.float32)
        f = {Q4_K: self.L.qko_dequant_q4k, Q5_K: self.L.qko_dequant_q5k,
             Q6_K: self.L.qko_dequant_q6k}[wtype]
        f(_ptr(w), nblocks, _ptr(out))
        return out

    def _split(self, fn, n, threads):
        threads = max(1, min(threads, n))
        cuts = [n * i // threads for i in range(threads + 1)]
        if threads == 1:
            rc = [fn(0, n)]
        else:
            with ThreadPoolExecutor(threads) as ex:
                rc = list(ex.map(lambda i: fn(cuts[i], cuts[i + 1]), range(threads)))
        if any(rc):
            raise RuntimeError("oracle matmul failed")

    def matmul(self, wtype, w, n, k, x, epi, threads=8):
        """tensor_matmul_* semantics: out[t, j], x is (m, k) fp32."""
        x = np.ascontiguousarray(x, np.float32).reshape(-1, k)
        w = np.ascontiguousarray(w, np.uint8)
        m = x.shape[0]
        out = np.empty((m, n), np.float32)
        self._split(lambda a, b: self.L.qko_matmul(wtype, _ptr(w), n, k, _ptr(x), m,
                                                   _ptr(out), epi, a, b), n, threads)
        return out

    def matmul_xq(self, wtype, w, n, k, xq, m, epi, threads=8):
        w = np.ascontiguousarray(w, np.uint8)
        xq = np.ascontiguousarray(xq, np.uint8)
        out = np.empty((m, n), np.float32)
        self._split(lambda a, b: self.L.qko_matmul_xq(wtype, _ptr(w), n, k, _ptr(xq), m,
                                                      _ptr(out), epi, a, b), n, threads)
        return out

    def argmax(self, v):
        v = np.ascontiguousarray(v, np.float32)
        return self.L.qko_argmax(_ptr(v), v.size)

    def topk_collect(self, v, k):
        v = np.ascontiguousarray(v, np.float32)
        idx = np.zeros(256, np.int32)
        val = np.zeros(256, np.float32)
        f = self.L.qko_topk_collect(_ptr(v), v.size, k, _ptr(idx), _ptr(val))
        return idx[:f].copy(), val[:f].copy()

    # -- decode-chain links (shared by Oracle and Ref) -------------------
    def add_rmsnorm(self, h, delta, w, eps):
        """(h + delta, rms_norm(h + delta) * w) per row; delta may be None."""
        h = np.ascontiguousarray(h, np.float32)
        m, k = h.reshape(-1, h.shape[-1]).shape
        d = None if delta is None else np.ascontiguousarray(delta, np.float32)
        w = np.ascontiguousarray(w, np.float32)
        r = np.empty((m, k), np.float32)
        x = np.empty((m, k), np.float32)
        rc = self._add_rmsnorm(_ptr(h), None if d is None else _ptr(d), _ptr(w), float(np.float32(eps)), m, k,
                               _ptr(r), _ptr(x))
        if rc:
            raise RuntimeError("add_rmsnorm failed")
        return r, x

    def silu(self, x):
        x = np.ascontiguousarray(x, np.float32)
        y = np.empty_like(x)
        self._silu(x.size, _ptr(x), _ptr(y))
        return y

    def swiglu(self, gate, up):
        g = np.ascontiguousarray(gate, np.float32)
        u = np.ascontiguousarray(up, np.float32)
        a = np.empty_like(g)
        if self._swiglu(g.size, _ptr(g), _ptr(u), _ptr(a)):
            raise RuntimeError("swiglu failed")
        return a

    def _add_rmsnorm(self, *a):
        self.L.qko_add_rmsnorm(*a)
        return 0

    def _rng_seed(self, *a):
        self.L.qko_rng_seed(*a)

    def _chunked_step(self, *a):
        self.L.qko_chunked_step(*a)

    def deltanet_chunked(self, q, k, v, g, beta, state):
        """The chunk loop of a layer: q, k [n, H, kd]; v [n, H, vd]; g, beta
        [n, H]; state [H, kd, vd]. Returns (out [n, H, vd], new state)."""
        q = np.ascontiguousarray(q, np.float32)
        n, H, kd = q.shape
        vd = v.shape[2]
        st = np.array(state, np.float32, copy=True)
        out = np.zeros((n, H, vd), np.float32)
        self.L.qko_deltanet_chunked(n, H, kd, vd, _ptr(q), _ptr(np.ascontiguousarray(k, np.float32)),
                                    _ptr(np.ascontiguousarray(v, np.float32)),
                                    _ptr(np.ascontiguousarray(g, np.float32)),
                                    _ptr(np.ascontiguousarray(beta, np.float32)), _ptr(st), _ptr(out))
        return out, st

    # -- chunked Gated DeltaNet (shared by Oracle and Ref) ------------------
    def chunked_step(self, q, k, v, g, beta, state):
        """One chunk of one head: returns (out, new state)."""
        q = np.ascontiguousarray(q, np.float32)
        n, kd = q.shape
        vd = v.shape[1]
        st = np.array(state, np.float32, copy=True)
        out = np.zeros((n, vd), np.float32)
        self._chunked_step(n, kd, vd, _ptr(q), _ptr(np.ascontiguousarray(k, np.float32)),
                           _ptr(np.ascontiguousarray(v, np.float32)), _ptr(np.ascontiguousarray(g, np.float32)),
                           _ptr(np.ascontiguousarray(beta, np.float32)), _ptr(st), _ptr(out))
        return out, st

    def _sample(self, *a):
        return self.L.qko_sample(*a)

    # -- sampler chain (shared by Oracle and Ref) -------------------------
    def rng_seed(self, seed):
        st = np.zeros(2, np.uint64)
        self._rng_seed(C.c_uint64(seed), _ptr(st))
        return st

    def sample(self, logits, sp, st, history=(), mask=()):
        """One step of slm_generate_raw's sampling: returns (token, penalized
        logits, advanced rng state). sp: dict of slm_sampler fields."""
        lg = np.array(logits, np.float32, copy=True)
        st = np.array(st, np.uint64, copy=True)
        h = np.ascontiguousarray(history, np.int32)
        mk = np.ascontiguousarray(mask, np.int32)
        tok = self._sample(_ptr(lg), lg.size, C.c_float(sp["temperature"]), sp["top_k"], C.c_float(sp["top_p"]),
                           C.c_float(sp["min_p"]), C.c_float(sp["repetition_penalty"]), sp["repetition_window"],
                           _ptr(st), _ptr(h) if h.size else None, h.size, _ptr(mk) if mk.size else None, mk.size)
        return tok, lg, st

    def _silu(self, *a):
        self.L.qko_silu(*a)

    def _swiglu(self, *a):
        self.L.qko_swiglu(*a)
        return 0


class Ref:
    """The reference's own C (oracle/_ref/libqkref.so, built from /root/reference)."""

    name = "ref"

    @staticmethod
    def available(path=REF_SO):
        return os.path.exists(path)

    def __init__(self, path=REF_SO):
        L = C.CDLL(path)
        self.L = L
        L.ref_simd_init.restype = None
        L.ref_dispatch_label.restype = C.c_char_p
        L.ref_tiers_available.restype = C.c_int
        for f in ("ref_quantize_q8k", "ref_quantize_q8k_quants_h", "ref_quantize_q8_0"):
            getattr(L, f).argtypes = [_vp, _vp, _i64]
            getattr(L, f).restype = None
        for f in ("ref_q4k_dot", "ref_q5k_dot", "ref_q6k_dot"):
            getattr(L, f).argtypes = [C.c_int, C.c_int, _vp, _vp]
            getattr(L, f).restype = C.c_float
        L.ref_q8_0_dot.argtypes = [C.c_int, _i64, _vp, _vp]
        L.ref_q8_0_dot.restype = C.c_float
        for f in ("ref_dequant_q4k", "ref_dequant_q5k", "ref_dequant_q6k"):
            getattr(L, f).argtypes = [_vp, _i64, _vp]
        L.ref_scale_min.argtypes = [_vp, C.c_int, _vp, _vp]
        L.ref_matmul.argtypes = [C.c_int, _vp, _i64, _i64, _vp, _i64, _vp]
        L.ref_matmul.restype = C.c_int
        L.ref_matmul_threads.argtypes = [C.c_int, _vp, _i64, _i64, _vp, _i64, _vp, C.c_int]
        L.ref_matmul_threads.restype = C.c_int
        L.ref_matmul_pool.argtypes = L.ref_matmul_threads.argtypes
        L.ref_matmul_pool.restype = C.c_int
        L.ref_pool_stop.restype = None
        L.ref_argmax.argtypes = [_vp, _i64]
        L.ref_argmax.restype = C.c_int32
        L.ref_topk_collect.argtypes = [_vp, _i64, C.c_int32, _vp, _vp]
        L.ref_topk_collect.restype = C.c_int32
        L.ref_add_rmsnorm.argtypes = [_vp, _vp, _vp, C.c_float, _i64, _i64, _vp, _vp]
        L.ref_add_rmsnorm.restype = C.c_int
        L.ref_silu.argtypes = [_i64, _vp, _vp]
        L.ref_silu.restype = None
        L.ref_swiglu.argtypes = [_i64, _vp, _vp, _vp]
        L.ref_swiglu.restype = C.c_int
        L.ref_chunked_step.argtypes = [C.c_int, C.c_int, C.c_int] + [_vp] * 7
        L.ref_chunked_step.restype = None
        L.ref_rng_seed.argtypes = [C.c_uint64, _vp]
        L.ref_rng_seed.restype = None
        L.ref_sample.argtypes = [_vp, _i64, C.c_float, C.c_int32, C.c_float, C.c_float, C.c_float, C.c_int32, _vp, _vp, C.c_int32, _vp, C.c_int32]
        L.ref_sample.restype = C.c_int32
        L.ref_simd_init()

    def label(self):
        return self.L.ref_dispatch_label().decode()

    def tiers(self):
        m = self.L.ref_tiers_available()
        return [t for t in range(4) if (m >> t) & 1]

    def dispatched_tier(self):
        return {"scalar": 0, "AVX1": 1, "AVX2-FMA": 2, "AVX-VNNI": 3}.get(self.label(), 0)

    def scale_min(self, s12, j):
        s = np.ascontiguousarray(s12, dtype=np.uint8)
        sc, m = C.c_uint8(), C.c_uint8()
        self.L.ref_scale_min(_ptr(s), j, C.byref(sc), C.byref(m))
        return sc.value, m.value

    def quantize_q8k(self, x, quants_h=False):
        x = np.ascontiguousarray(x, dtype=np.float32)
        m, k = x.reshape(-1, x.shape[-1]).shape
        out = np.zeros((m, (k // 256) * Q8K_BYTES), np.uint8)
        f = self.L.ref_quantize_q8k_quants_h if quants_h else self.L.ref_quantize_q8k
        for t in range(m):
            f(_ptr(x.reshape(m, k)[t]), _ptr(out[t]), k)
        return out

    def quantize_q8_0(self, x):
        x = np.ascontiguousarray(x, dtype=np.float32)
        m, k = x.reshape(-1, x.shape[-1]).shape
        out = np.zeros((m, (k // 32) * 34), np.uint8)
        for t in range(m):
            self.L.ref_quantize_q8_0(_ptr(x.reshape(m, k)[t]), _ptr(out[t]), k)
        return out

    def quantize_for(self, wtype, x):
        return self.quantize_q8_0(x) if wtype == Q8_0 else self.quantize_q8k(x)

    def row_dot(self, wtype, wrow, xq, k, tier=-1):
        wrow = np.ascontiguousarray(wrow, np.uint8)
        xq = np.ascontiguousarray(xq, np.uint8)
        nb = k // BLOCK_ELEMS[wtype]
        if wtype == Q8_0:
            return self.L.ref_q8_0_dot(tier, k, _ptr(wrow), _ptr(xq))
        f = {Q4_K: self.L.ref_q4k_dot, Q5_K: self.L.ref_q5k_dot, Q6_K: self.L.ref_q6k_dot}[wtype]
        return f(tier, nb, _ptr(wrow), _ptr(xq))

    def dequant(self, wtype, w, nblocks):
        w = np.ascontiguousarray(w, np.uint8)
        out = np.empty(nblocks * 256, np.float32)
        f = {Q4_K: self.L.ref_dequant_q4k, Q5_K: self.L.ref_dequant_q5k,
             Q6_K: self.L.ref_dequant_q6k}[wtype]
        f(_ptr(w), nblocks, _ptr(out))
        return out

    def matmul(self, wtype, w, n, k, x, threads=1):
        x = np.ascontiguousarray(x, np.float32).reshape(-1, k)
        w = np.ascontiguousarray(w, np.uint8)
        m = x.shape[0]
        out = np.empty((m, n), np.float32)
        if threads <= 1:
            rc = self.L.ref_matmul(wtype, _ptr(w), n, k, _ptr(x), m, _ptr(out))
        else:
            rc = self.L.ref_matmul_pool(wtype, _ptr(w), n, k, _ptr(x), m, _ptr(out), threads)
        if rc:
            raise RuntimeError("reference matmul failed")
        return out

    def pool_stop(self):
        """End the worker threads of matmul(threads > 1)."""
        self.L.ref_pool_stop()

    def argmax(self, v):
        v = np.ascontiguousarray(v, np.float32)
        return self.L.ref_argmax(_ptr(v), v.size)

    def topk_collect(self, v, k):
        v = np.ascontiguousarray(v, np.float32)
        idx = np.zeros(256, np.int32)
        val = np.zeros(256, np.float32)
        f = self.L.ref_topk_collect(_ptr(v), v.size, k, _ptr(idx), _ptr(val))
        return idx[:f].copy(), val[:f].copy()

    # -- decode-chain links (shared by Oracle and Ref) -------------------
    def add_rmsnorm(self, h, delta, w, eps):
        """(h + delta, rms_norm(h + delta) * w) per row; delta may be None."""
        h = np.ascontiguousarray(h, np.float32)
        m, k = h.reshape(-1, h.shape[-1]).shape
        d = None if delta is None else np.ascontiguousarray(delta, np.float32)
        w = np.ascontiguousarray(w, np.float32)
        r = np.empty((m, k), np.float32)
        x = np.empty((m, k), np.float32)
        rc = self._add_rmsnorm(_ptr(h), None if d is None else _ptr(d), _ptr(w), float(np.float32(eps)), m, k,
                               _ptr(r), _ptr(x))
        if rc:
            raise RuntimeError("add_rmsnorm failed")
        return r, x

    def silu(self, x):
        x = np.ascontiguousarray(x, np.float32)
        y = np.empty_like(x)
        self._silu(x.size, _ptr(x), _ptr(y))
        return y

    def swiglu(self, gate, up):
        g = np.ascontiguousarray(gate, np.float32)
        u = np.ascontiguousarray(up, np.float32)
        a = np.empty_like(g)
        if self._swiglu(g.size, _ptr(g), _ptr(u), _ptr(a)):
            raise RuntimeError("swiglu failed")
        return a

    def _add_rmsnorm(self, *a):
        return self.L.ref_add_rmsnorm(*a)

    def _silu(self, *a):
        self.L.ref_silu(*a)

    def _swiglu(self, *a):
        return self.L.ref_swiglu(*a)

    def _rng_seed(self, *a):
        self.L.ref_rng_seed(*a)

    def _sample(self, *a):
        return self.L.ref_sample(*a)

    # -- sampler chain (shared by Oracle and Ref) -------------------------
    def rng_seed(self, seed):
        st = np.zeros(2, np.uint64)
        self._rng_seed(C.c_uint64(seed), _ptr(st))
        return st

    def sample(self, logits, sp, st, history=(), mask=()):
        """One step of slm_generate_raw's sampling: returns (token, penalized
        logits, advanced rng state). sp: dict of slm_sampler fields."""
        lg = np.array(logits, np.float32, copy=True)
        st = np.array(st, np.uint64, copy=True)
        h = np.ascontiguousarray(history, np.int32)
        mk = np.ascontiguousarray(mask, np.int32)
        tok = self._sample(_ptr(lg), lg.size, C.c_float(sp["temperature"]), sp["top_k"], C.c_float(sp["top_p"]),
                           C.c_float(sp["min_p"]), C.c_float(sp["repetition_penalty"]), sp["repetition_window"],
                           _ptr(st), _ptr(h) if h.size else None, h.size, _ptr(mk) if mk.size else None, mk.size)
        return tok, lg, st

    def _chunked_step(self, *a):
        self.L.ref_chunked_step(*a)

    # -- chunked Gated DeltaNet (shared by Oracle and Ref) ------------------
    def chunked_step(self, q, k, v, g, beta, state):
        """One chunk of one head: returns (out, new state)."""
        q = np.ascontiguousarray(q, np.float32)
        n, kd = q.shape
        vd = v.shape[1]
        st = np.array(state, np.float32, copy=True)
        out = np.zeros((n, vd), np.float32)
        self._chunked_step(n, kd, vd, _ptr(q), _ptr(np.ascontiguousarray(k, np.float32)),
                           _ptr(np.ascontiguousarray(v, np.float32)), _ptr(np.ascontiguousarray(g, np.float32)),
                           _ptr(np.ascontiguousarray(beta, np.float32)), _ptr(st), _ptr(out))
        return out, st
