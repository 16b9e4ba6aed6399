"""ctypes binding of libqk (include/qk.h) for tests and the benchmark.

PyTorch is used only to own device memory and streams: every tensor
passed to the device layer must already live on the GPU, and the call is
enqueued on torch's current stream. The library itself is plain C ABI
(libqk.so next to this file); when it is missing this module raises
instead of falling back to anything else.
"""
from __future__ import annotations

import ctypes as C
import os
import re

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
LIB = os.path.join(HERE, "libqk.so")
HEADER = os.path.join(os.path.dirname(HERE), "include", "qk.h")

Q8_0, Q4_K, Q5_K, Q6_K = 8, 12, 13, 14
BLOCK_BYTES = {Q8_0: 34, Q4_K: 144, Q5_K: 176, Q6_K: 210}
BLOCK_ELEMS = {Q8_0: 32, Q4_K: 256, Q5_K: 256, Q6_K: 256}
Q8K_BYTES = 292
TIER_SCALAR, TIER_AVX1, TIER_AVX2, TIER_AVXVNNI, TIER_AUTO = 0, 1, 2, 3, -1
GROUP_MAX = 16
TOPK_MAX = 256

_vp, _i64, _i32 = C.c_void_p, C.c_int64, C.c_int32


class QKError(RuntimeError):
    def __init__(self, rc, msg):
        super().__init__(f"libqk error {rc}: {msg}")
        self.rc = rc


class Sampler(C.Structure):
    """struct slm_sampler (qk_sampler in include/qk.h)."""
    _fields_ = [("temperature", C.c_float), ("top_k", C.c_int32), ("top_p", C.c_float), ("min_p", C.c_float),
                ("repetition_penalty", C.c_float), ("repetition_window", C.c_int32)]


class GemvDesc(C.Structure):
    _fields_ = [("type", C.c_int32), ("pad_", C.c_int32), ("n", C.c_int64), ("k", C.c_int64),
                ("w", C.c_void_p), ("xq", C.c_void_p), ("y", C.c_void_p)]


def header_functions(path=HEADER):
    """Names of the functions include/qk.h declares."""
    text = open(path).read()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    return sorted(set(re.findall(r"\b(hip_[a-z0-9_]+)\s*\(", text)))


def act_bytes(wtype, k):
    return (k // 32) * 34 if wtype == Q8_0 else (k // 256) * Q8K_BYTES


def _dp(t):
    return C.c_void_p(0 if t is None else t.data_ptr())


def _nbytes(t):
    return t.numel() * t.element_size()


def _need(t, nbytes, what):
    """Refuse a launch whose buffer is smaller than the shape implies (the
    C ABI takes raw pointers and cannot check this itself)."""
    if t is not None and _nbytes(t) < nbytes:
        raise ValueError(f"{what}: buffer of {_nbytes(t)} bytes, shape needs {nbytes}")


def row_bytes(wtype, k):
    return (k // BLOCK_ELEMS[wtype]) * BLOCK_BYTES[wtype] if k % BLOCK_ELEMS[wtype] == 0 else 0


class QK:
    """libqk.so. Device-layer methods take torch CUDA tensors."""

    def __init__(self, path=LIB):
        if not os.path.exists(path):
            raise FileNotFoundError(f"{path} is not built (run __graft_entry__.build())")
        L = C.CDLL(path)
        self.L = L
        L.hip_qk_init.argtypes = [C.c_int]
        L.hip_qk_shutdown.restype = None
        for f in ("hip_qk_device_label", "hip_qk_last_error"):
            getattr(L, f).restype = C.c_char_p
        L.hip_qk_tier_label.restype = C.c_char_p
        L.hip_qk_tier_label.argtypes = [C.c_int]
        L.hip_qk_set_tier.argtypes = [C.c_int]
        for f in ("hip_quantize_q8k", "hip_quantize_q8_0"):
            getattr(L, f).argtypes = [_vp, _i64, _i64, _vp, _vp]
        for f in ("hip_matvec_q4k", "hip_matvec_q5k", "hip_matvec_q6k", "hip_matvec_q8_0"):
            getattr(L, f).argtypes = [_vp, _i64, _i64, _vp, _vp, _vp]
        L.hip_matvec_group.argtypes = [C.POINTER(GemvDesc), C.c_int, _vp]
        L.hip_matvec_group_f32.argtypes = [C.POINTER(GemvDesc), C.c_int, _vp]
        for f in ("hip_matmul_q4k", "hip_matmul_q5k", "hip_matmul_q6k", "hip_matmul_q8_0"):
            getattr(L, f).argtypes = [_vp, _i64, _i64, _vp, _i64, _vp, _vp]
        L.hip_gemm_planes_bytes.argtypes = [C.c_int, _i64, _i64]
        L.hip_gemm_planes_bytes.restype = C.c_size_t
        L.hip_gemm_pack_planes.argtypes = [C.c_int, _vp, _i64, _i64, _vp, _vp]
        L.hip_matmul_planes.argtypes = [C.c_int, _vp, _i64, _i64, _vp, _i64, _vp, _vp]
        for f in ("hip_dequant_q4k", "hip_dequant_q5k", "hip_dequant_q6k"):
            getattr(L, f).argtypes = [_vp, _i64, _vp, _vp]
        L.hip_lmhead_q6k_argmax_topk.argtypes = [_vp, _i64, _i64, _vp, C.c_int, _vp, _vp, _vp, _vp, _vp]
        L.hip_add_rmsnorm_q8k.argtypes = [_vp, _vp, _vp, C.c_float, _i64, _i64, _vp, _vp, _vp, _vp]
        L.hip_silu_f32.argtypes = [_vp, _i64, _vp, _vp]
        L.hip_swiglu_q8k.argtypes = [_vp, _vp, _i64, _i64, _vp, _vp, _vp]
        L.hip_sample.argtypes = [_vp, _i64, C.POINTER(Sampler), _vp, _vp, C.c_int32, _vp, C.c_int32, _vp, _vp]
        L.hip_deltanet_chunked.argtypes = [_vp] * 5 + [_i64, C.c_int, C.c_int, C.c_int, _vp, _vp, _vp]
        L.hip_qk_deltanet_host.argtypes = [C.c_int, C.c_int, C.c_int] + [_vp] * 7
        L.hip_qk_deltanet_layer_host.argtypes = [C.c_int64, C.c_int, C.c_int, C.c_int] + [_vp] * 7
        L.hip_qk_register_weight.argtypes = [_vp, C.c_int, _i64, _i64]
        L.hip_qk_unregister_weight.argtypes = [_vp]
        L.hip_qk_device_weight.argtypes = [_vp]
        L.hip_qk_device_weight.restype = C.c_void_p
        L.hip_qk_matmul_host.argtypes = [_vp, C.c_int, _i64, _i64, _vp, _i64, _vp]
        L.hip_qk_lmhead_host.argtypes = [_vp, _i64, _i64, _vp, C.c_int, _vp, _vp, _vp, _vp]

    # -- plumbing ---------------------------------------------------------
    def _ck(self, rc):
        if rc != 0:
            raise QKError(rc, self.L.hip_qk_last_error().decode())
        return rc

    def last_error(self):
        return self.L.hip_qk_last_error().decode()

    @staticmethod
    def _stream():
        import torch
        return C.c_void_p(torch.cuda.current_stream().cuda_stream)

    def init(self, device=0):
        self._ck(self.L.hip_qk_init(device))
        return self

    def shutdown(self):
        self.L.hip_qk_shutdown()

    def label(self):
        return self.L.hip_qk_device_label().decode()

    def set_tier(self, tier):
        self._ck(self.L.hip_qk_set_tier(tier))

    def tier(self):
        return self.L.hip_qk_get_tier()

    def tier_label(self, tier=None):
        return self.L.hip_qk_tier_label(self.tier() if tier is None else tier).decode()

    # -- device layer ---------------------------------------------------------
    def quantize_q8k(self, x, out=None):
        import torch
        m, k = x.shape
        if out is None:
            out = torch.empty((m, (k // 256) * Q8K_BYTES), dtype=torch.uint8, device=x.device)
        _need(out, m * (k // 256) * Q8K_BYTES, "xq")
        self._ck(self.L.hip_quantize_q8k(_dp(x), m, k, _dp(out), self._stream()))
        return out

    def quantize_q8_0(self, x, out=None):
        import torch
        m, k = x.shape
        if out is None:
            out = torch.empty((m, (k // 32) * 34), dtype=torch.uint8, device=x.device)
        _need(out, m * (k // 32) * 34, "xq")
        self._ck(self.L.hip_quantize_q8_0(_dp(x), m, k, _dp(out), self._stream()))
        return out

    def quantize_for(self, wtype, x, out=None):
        return self.quantize_q8_0(x, out) if wtype == Q8_0 else self.quantize_q8k(x, out)

    def matvec(self, wtype, w, n, k, xq, y=None):
        import torch
        if y is None:
            y = torch.empty(n, dtype=torch.float32, device=w.device)
        f = {Q4_K: self.L.hip_matvec_q4k, Q5_K: self.L.hip_matvec_q5k,
             Q6_K: self.L.hip_matvec_q6k, Q8_0: self.L.hip_matvec_q8_0}[wtype]
        _need(w, n * row_bytes(wtype, k), "w")
        _need(xq, act_bytes(wtype, k), "xq")
        _need(y, 4 * n, "y")
        self._ck(f(_dp(w), n, k, _dp(xq), _dp(y), self._stream()))
        return y

    def matvec_group(self, items):
        """items: list of (wtype, w, n, k, xq, y) with device tensors."""
        arr = (GemvDesc * len(items))()
        for i, (t, w, n, k, xq, y) in enumerate(items):
            _need(w, n * row_bytes(t, k), "w")
            _need(xq, act_bytes(t, k), "xq")
            _need(y, 4 * n, "y")
            arr[i] = GemvDesc(t, 0, n, k, w.data_ptr(), xq.data_ptr(), y.data_ptr())
        self._ck(self.L.hip_matvec_group(arr, len(items), self._stream()))

    def matvec_group_f32(self, items):
        """items: list of (wtype, w, n, k, x, y) with device tensors; x is
        the fp32 activation row (k floats), quantized inside the launch."""
        arr = (GemvDesc * len(items))()
        for i, (t, w, n, k, x, y) in enumerate(items):
            _need(w, n * row_bytes(t, k), "w")
            _need(x, 4 * k, "x")
            _need(y, 4 * n, "y")
            arr[i] = GemvDesc(t, 0, n, k, w.data_ptr(), x.data_ptr(), y.data_ptr())
        self._ck(self.L.hip_matvec_group_f32(arr, len(items), self._stream()))

    def matmul(self, wtype, w, n, k, xq, m, y=None):
        import torch
        if y is None:
            y = torch.empty((m, n), dtype=torch.float32, device=w.device)
        f = {Q4_K: self.L.hip_matmul_q4k, Q5_K: self.L.hip_matmul_q5k, Q6_K: self.L.hip_matmul_q6k,
             Q8_0: self.L.hip_matmul_q8_0}[wtype]
        _need(w, n * row_bytes(wtype, k), "w")
        _need(xq, m * act_bytes(wtype, k), "xq")
        _need(y, 4 * m * n, "y")
        self._ck(f(_dp(w), n, k, _dp(xq), m, _dp(y), self._stream()))
        return y

    def planes_bytes(self, wtype, n, k):
        return int(self.L.hip_gemm_planes_bytes(wtype, n, k))

    def pack_planes(self, wtype, w, n, k, planes=None):
        """Repack a device K-quant matrix into the GEMM's int8 MFMA planes."""
        import torch
        nb = self.planes_bytes(wtype, n, k)
        if planes is None:
            planes = torch.empty(nb, dtype=torch.uint8, device=w.device)
        _need(w, n * row_bytes(wtype, k), "w")
        _need(planes, nb, "planes")
        self._ck(self.L.hip_gemm_pack_planes(wtype, _dp(w), n, k, _dp(planes), self._stream()))
        return planes

    def matmul_planes(self, wtype, planes, n, k, xq, m, y=None):
        import torch
        if y is None:
            y = torch.empty((m, n), dtype=torch.float32, device=planes.device)
        _need(planes, self.planes_bytes(wtype, n, k), "planes")
        _need(xq, m * act_bytes(wtype, k), "xq")
        _need(y, 4 * m * n, "y")
        self._ck(self.L.hip_matmul_planes(wtype, _dp(planes), n, k, _dp(xq), m, _dp(y), self._stream()))
        return y

    def dequant(self, wtype, w, nblocks, y=None):
        import torch
        if y is None:
            y = torch.empty(nblocks * 256, dtype=torch.float32, device=w.device)
        f = {Q4_K: self.L.hip_dequant_q4k, Q5_K: self.L.hip_dequant_q5k, Q6_K: self.L.hip_dequant_q6k}[wtype]
        _need(w, nblocks * BLOCK_BYTES[wtype], "w")
        _need(y, 4 * 256 * nblocks, "y")
        self._ck(f(_dp(w), nblocks, _dp(y), self._stream()))
        return y

    def lmhead(self, w, n, k, xq, topk=0, logits=None, want_logits=True):
        import torch
        dev = w.device
        if logits is None and want_logits:
            logits = torch.empty(n, dtype=torch.float32, device=dev)
        _need(w, n * row_bytes(Q6_K, k), "w")
        _need(xq, act_bytes(Q6_K, k), "xq")
        _need(logits, 4 * n, "logits")
        am = torch.empty(1, dtype=torch.int32, device=dev)
        ti = torch.empty(max(topk, 1), dtype=torch.int32, device=dev)
        tv = torch.empty(max(topk, 1), dtype=torch.float32, device=dev)
        self._ck(self.L.hip_lmhead_q6k_argmax_topk(_dp(w), n, k, _dp(xq), topk, _dp(logits), _dp(am),
                                                    _dp(ti) if topk else None, _dp(tv) if topk else None,
                                                    self._stream()))
        return logits, am, ti[:topk], tv[:topk]

    def add_rmsnorm_q8k(self, h, delta, w, eps, h_out=None, x_out=None, xq=None):
        """h, delta (or None): (m, k) fp32; w: k fp32. Writes h + delta to
        h_out, the normalized rows to x_out and their Q8_K rows to xq (each
        optional; pass the tensors to be filled)."""
        m, k = h.shape
        for t in (delta, h_out, x_out):
            _need(t, 4 * m * k, "row")
        _need(w, 4 * k, "w")
        _need(xq, m * (k // 256) * Q8K_BYTES, "xq")
        self._ck(self.L.hip_add_rmsnorm_q8k(_dp(h), _dp(delta), _dp(w), float(np.float32(eps)), m, k, _dp(h_out),
                                            _dp(x_out), _dp(xq), self._stream()))

    def silu(self, x, y=None):
        import torch
        if y is None:
            y = torch.empty_like(x)
        _need(y, _nbytes(x), "y")
        self._ck(self.L.hip_silu_f32(_dp(x), x.numel(), _dp(y), self._stream()))
        return y

    def swiglu_q8k(self, gate, up, act=None, xq=None):
        """gate, up: (m, k) fp32; writes silu(gate) * up to act and/or its
        Q8_K rows to xq."""
        m, k = gate.shape
        _need(up, 4 * m * k, "up")
        _need(act, 4 * m * k, "act")
        _need(xq, m * (k // 256) * Q8K_BYTES, "xq")
        self._ck(self.L.hip_swiglu_q8k(_dp(gate), _dp(up), m, k, _dp(act), _dp(xq), self._stream()))

    def sample(self, logits, sp, rng, history=None, hist_n=None, mask=(), token=None):
        """One sampling step on device logits (modified in place): sp is a
        dict of slm_sampler fields, rng a device uint64[2] (advanced),
        history a device int32 tensor whose first hist_n ids count.
        Returns the device int32 token tensor."""
        import torch
        if token is None:
            token = torch.empty(1, dtype=torch.int32, device=logits.device)
        if history is not None and hist_n is None:
            hist_n = history.numel()
        hist_n = hist_n or 0
        _need(history, 4 * hist_n, "history")
        s = Sampler(sp["temperature"], sp["top_k"], sp["top_p"], sp["min_p"], sp["repetition_penalty"],
                    sp["repetition_window"])
        m = (C.c_int32 * max(1, len(mask)))(*mask) if len(mask) else None
        self._ck(self.L.hip_sample(_dp(logits), logits.numel(), C.byref(s), _dp(rng),
                                   _dp(history) if hist_n else None, hist_n, m, len(mask), _dp(token),
                                   self._stream()))
        return token

    def deltanet_chunked(self, q, k, v, g, beta, state, out=None):
        """q, k: (n, H, kd); v: (n, H, vd); g, beta: (n, H); state (H, kd, vd)
        updated in place; returns out (n, H, vd). Device tensors."""
        import torch
        n, H, kd = q.shape
        vd = v.shape[2]
        if out is None:
            out = torch.empty((n, H, vd), dtype=torch.float32, device=q.device)
        for t, want in ((k, n * H * kd), (v, n * H * vd), (g, n * H), (beta, n * H), (state, H * kd * vd),
                        (out, n * H * vd)):
            _need(t, 4 * want, "deltanet operand")
        self._ck(self.L.hip_deltanet_chunked(_dp(q), _dp(k), _dp(v), _dp(g), _dp(beta), n, H, kd, vd, _dp(state),
                                             _dp(out), self._stream()))
        return out

    def deltanet_host(self, q, k, v, g, beta, state):
        """One head, one chunk, numpy in and out: returns (out, new state)."""
        q = np.ascontiguousarray(q, np.float32)
        n, kd = q.shape
        vd = v.shape[1]
        st = np.array(state, np.float32, copy=True)
        out = np.empty((n, vd), np.float32)
        arrs = [np.ascontiguousarray(a, np.float32) for a in (k, v, g, beta)]
        self._ck(self.L.hip_qk_deltanet_host(n, kd, vd, q.ctypes.data_as(_vp), *[a.ctypes.data_as(_vp) for a in arrs],
                                             st.ctypes.data_as(_vp), out.ctypes.data_as(_vp)))
        return out, st

    def deltanet_layer_host(self, q, k, v, g, beta, state):
        """One layer, numpy in and out (q, k [n][H][kd], v [n][H][vd], g,
        beta [n][H], state [H][kd][vd]): returns (out, new state)."""
        q = np.ascontiguousarray(q, np.float32)
        n, H, kd = q.shape
        vd = v.shape[2]
        st = np.array(state, np.float32, copy=True)
        out = np.empty((n, H, vd), np.float32)
        arrs = [np.ascontiguousarray(a, np.float32) for a in (k, v, g, beta)]
        self._ck(self.L.hip_qk_deltanet_layer_host(n, H, kd, vd, q.ctypes.data_as(_vp),
                                                   *[a.ctypes.data_as(_vp) for a in arrs],
                                                   st.ctypes.data_as(_vp), out.ctypes.data_as(_vp)))
        return out, st

    # -- host seam --------------------------------------------------------------
    def matmul_host(self, wtype, w_np, out_f, k, x_np):
        x = np.ascontiguousarray(x_np, np.float32).reshape(-1, k)
        out = np.empty((x.shape[0], out_f), np.float32)
        self._ck(self.L.hip_qk_matmul_host(w_np.ctypes.data_as(_vp), wtype, out_f, k,
                                           x.ctypes.data_as(_vp), x.shape[0], out.ctypes.data_as(_vp)))
        return out

    def lmhead_host(self, w_np, n, k, x_np, topk=0):
        x = np.ascontiguousarray(x_np, np.float32).reshape(k)
        logits = np.empty(n, np.float32)
        am = np.zeros(1, np.int32)
        ti = np.zeros(max(topk, 1), np.int32)
        tv = np.zeros(max(topk, 1), np.float32)
        self._ck(self.L.hip_qk_lmhead_host(w_np.ctypes.data_as(_vp), n, k, x.ctypes.data_as(_vp), topk,
                                           logits.ctypes.data_as(_vp), am.ctypes.data_as(_vp),
                                           ti.ctypes.data_as(_vp), tv.ctypes.data_as(_vp)))
        return logits, int(am[0]), ti[:topk], tv[:topk]

    def register_weight(self, w_np, wtype, k, n):
        self._ck(self.L.hip_qk_register_weight(w_np.ctypes.data_as(_vp), wtype, k, n))

    def unregister_weight(self, w_np):
        self._ck(self.L.hip_qk_unregister_weight(w_np.ctypes.data_as(_vp)))
