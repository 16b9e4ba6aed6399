"""Deterministic activation rows that exercise the quantizers' edge cases."""
import numpy as np


def edge_rows(k):
    """(m, k) float32 rows; each 256-element (or 32-element) block of a row
    carries the same pattern so both quantizers see it."""
    rows = []
    rng = np.random.default_rng(1234)
    def tile(block):
        return np.resize(np.asarray(block, np.float32), k)
    z = np.zeros(256, np.float32)
    rows.append(tile(z))                                   # all zero -> d = 0
    t = rng.normal(0, 0.1, 256).astype(np.float32)
    t[5], t[77] = -3.0, 3.0                                # |x| tie, opposite signs
    rows.append(tile(t))
    t = rng.normal(0, 0.1, 256).astype(np.float32)
    t[9], t[3] = 3.0, -3.0                                 # tie, first one negative
    rows.append(tile(t))
    h = (np.arange(256, dtype=np.float32) % 254) - 126.5   # x.5 under iscale = 1
    h[0] = -127.0
    rows.append(tile(h))
    h = -h
    rows.append(tile(h))
    c = np.full(256, 2.0, np.float32)                      # constant block
    rows.append(tile(c))
    big = rng.normal(0, 1, 256).astype(np.float32) * np.float32(1e37)
    rows.append(tile(big))
    tiny = rng.normal(0, 1, 256).astype(np.float32) * np.float32(1e-39)   # subnormal inputs
    rows.append(tile(tiny))
    last = rng.normal(0, 1, 256).astype(np.float32)
    last[255] = 50.0                                       # max at the last index
    last[0:8] = -0.0
    rows.append(tile(last))
    q = (np.arange(32, dtype=np.float32) - 16) + 0.5       # Q8_0 halves: amax 127 -> id 1
    q[0] = 127.0
    rows.append(tile(q))
    small = rng.normal(0, 1, 256).astype(np.float32) * np.float32(1e-3)
    rows.append(tile(small))
    return np.stack(rows).astype(np.float32)


def special_rows(k):
    """(m, k) float32 rows with NaN and infinity entries and |x| ties across
    lanes, each 256-element block carrying the same pattern."""
    rows = []
    rng = np.random.default_rng(4321)
    def tile(block):
        return np.resize(np.asarray(block, np.float32), k)
    t = rng.normal(0, 1, 256).astype(np.float32)
    t[3], t[100] = np.nan, np.nan                          # NaN never chosen; quantizes to 0
    t[200] = 7.0
    rows.append(tile(t))
    t = rng.normal(0, 1, 256).astype(np.float32)
    t[10] = np.inf                                         # amax = inf: d = -inf, q = 0
    rows.append(tile(t))
    t = rng.normal(0, 1, 256).astype(np.float32)
    t[20], t[200] = -4.0, 4.0                              # tie across lanes: the first wins
    rows.append(tile(t))
    t = rng.normal(0, 1, 256).astype(np.float32)
    t[63], t[64] = 4.0, -4.0                               # tie across a 16-lane row boundary
    rows.append(tile(t))
    t = np.full(256, np.nan, np.float32)                   # all NaN: amax 0, d = 0
    rows.append(tile(t))
    return np.stack(rows).astype(np.float32)
