"""Deterministic synthetic GGUF blocks and activations for the benchmark
configurations (the reference has no generator; its tests fabricate
random bytes, simd/simd.c:508-531).

Counter-based splitmix64: value i of stream s under seed S depends only
on (S, s, i), so any slice can be regenerated independently. N(0,1)
comes from Box-Muller in float64, rounded once to float32. fp16 fields
use numpy's IEEE round-to-nearest-even conversion.

Block recipes (one per GGUF type):
  Q4_K  d = fp16(|N|*2e-3), dmin = fp16(|N|*1e-3), 8 scales and 8 mins
        U[0,63] packed into 12 bytes, 128 B of uniform 4-bit pairs;
  Q5_K  as Q4_K plus 32 B of uniform qh;
  Q6_K  d = fp16(|N|*2e-3), int8 scales U[-32,31], uniform ql and qh;
  Q8_0  d = fp16(|N|*2e-3), int8 quants U[-127,127].
"""
from __future__ import annotations

import numpy as np

Q8_0, Q4_K, Q5_K, Q6_K = 8, 12, 13, 14
BLOCK_BYTES = {Q8_0: 34, Q4_K: 144, Q5_K: 176, Q6_K: 210}
BLOCK_ELEMS = {Q8_0: 32, Q4_K: 256, Q5_K: 256, Q6_K: 256}

_M64 = np.uint64(0xFFFFFFFFFFFFFFFF)
_GOLD = np.uint64(0x9E3779B97F4A7C15)


def _mix(z):
    z = (z ^ (z >> np.uint64(30))) * np.uint64(0xBF58476D1CE4E5B9)
    z = (z ^ (z >> np.uint64(27))) * np.uint64(0x94D049BB133111EB)
    return z ^ (z >> np.uint64(31))


def u64(seed: int, stream: int, n: int, start: int = 0) -> np.ndarray:
    """n splitmix64 outputs of (seed, stream) starting at counter `start`."""
    with np.errstate(over="ignore"):
        key = _mix(np.uint64(seed & 0xFFFFFFFFFFFFFFFF) * _GOLD + np.uint64(stream + 1))
        ctr = np.arange(start + 1, start + n + 1, dtype=np.uint64)
        return _mix(key + ctr * _GOLD)


def uniform01(seed, stream, n):
    return (u64(seed, stream, n) >> np.uint64(11)).astype(np.float64) * (1.0 / 9007199254740992.0)


def normal(seed, stream, n) -> np.ndarray:
    """N(0,1) as float32 (Box-Muller on two uniform streams)."""
    u1 = uniform01(seed, 2 * stream, n)
    u2 = uniform01(seed, 2 * stream + 1, n)
    u1 = np.where(u1 <= 0.0, 2.0 ** -53, u1)
    z = np.sqrt(-2.0 * np.log(u1)) * np.cos(2.0 * np.pi * u2)
    return z.astype(np.float32)


def ubytes(seed, stream, n) -> np.ndarray:
    return (u64(seed, stream, n) & np.uint64(0xFF)).astype(np.uint8)


def uint_range(seed, stream, n, lo, hi) -> np.ndarray:
    """Integers uniform in [lo, hi] (inclusive)."""
    span = np.uint64(hi - lo + 1)
    return ((u64(seed, stream, n) % span).astype(np.int64) + lo)


def pack_scales_mins(sc: np.ndarray, mn: np.ndarray) -> np.ndarray:
    """Inverse of q4k_get_scale_min (simd/quants.h:215-224): (nb, 8) six-bit
    scales and mins -> (nb, 12) bytes."""
    sc = sc.astype(np.uint8)
    mn = mn.astype(np.uint8)
    s = np.zeros((sc.shape[0], 12), np.uint8)
    s[:, 0:4] = (sc[:, 0:4] & 63) | ((sc[:, 4:8] >> 4) << 6)
    s[:, 4:8] = (mn[:, 0:4] & 63) | ((mn[:, 4:8] >> 4) << 6)
    s[:, 8:12] = (sc[:, 4:8] & 15) | ((mn[:, 4:8] & 15) << 4)
    return s


def _f16_bytes(v: np.ndarray) -> np.ndarray:
    return v.astype(np.float16).view(np.uint8).reshape(-1, 2)


def blocks(wtype: int, n_rows: int, k: int, seed: int = 0, tag: int = 0) -> np.ndarray:
    """(n_rows, k/elems * bytes) uint8 matrix of random blocks."""
    nb = n_rows * (k // BLOCK_ELEMS[wtype])
    base = 64 * tag
    out = np.zeros((nb, BLOCK_BYTES[wtype]), np.uint8)
    if wtype in (Q4_K, Q5_K):
        out[:, 0:2] = _f16_bytes(np.abs(normal(seed, base + 0, nb)) * np.float32(2e-3))
        out[:, 2:4] = _f16_bytes(np.abs(normal(seed, base + 1, nb)) * np.float32(1e-3))
        sc = uint_range(seed, base + 4, nb * 8, 0, 63).reshape(nb, 8)
        mn = uint_range(seed, base + 5, nb * 8, 0, 63).reshape(nb, 8)
        out[:, 4:16] = pack_scales_mins(sc, mn)
        if wtype == Q4_K:
            out[:, 16:144] = ubytes(seed, base + 6, nb * 128).reshape(nb, 128)
        else:
            out[:, 16:48] = ubytes(seed, base + 7, nb * 32).reshape(nb, 32)
            out[:, 48:176] = ubytes(seed, base + 6, nb * 128).reshape(nb, 128)
    elif wtype == Q6_K:
        out[:, 0:128] = ubytes(seed, base + 8, nb * 128).reshape(nb, 128)
        out[:, 128:192] = ubytes(seed, base + 9, nb * 64).reshape(nb, 64)
        out[:, 192:208] = uint_range(seed, base + 10, nb * 16, -32, 31).astype(np.int8).view(np.uint8).reshape(nb, 16)
        out[:, 208:210] = _f16_bytes(np.abs(normal(seed, base + 11, nb)) * np.float32(2e-3))
    elif wtype == Q8_0:
        out[:, 0:2] = _f16_bytes(np.abs(normal(seed, base + 12, nb)) * np.float32(2e-3))
        out[:, 2:34] = uint_range(seed, base + 13, nb * 32, -127, 127).astype(np.int8).view(np.uint8).reshape(nb, 32)
    else:
        raise ValueError(f"unsupported type {wtype}")
    return out.reshape(n_rows, -1)


def activations(m: int, k: int, seed: int = 0, tag: int = 0) -> np.ndarray:
    """(m, k) float32 ~ N(0,1)."""
    return normal(seed, 64 * tag + 40, m * k).reshape(m, k)
