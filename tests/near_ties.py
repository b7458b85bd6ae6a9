"""Tokens whose RMSNorm output sits almost exactly on a float rounding midpoint.

RMSNorm (engine.cpp:723-740) sums x*x in double in index order, then rounds
x*scale*gain to float. A parallel sum differs from the in-order one in its
last bits, which moves x*scale*gain by a few parts in 1e15: harmless unless
the double value lies that close to the midpoint between two floats. These
helpers search for tokens where it does, so a test can check that the device
keeps the in-order result there too.

The search varies the last element c of a token: the in-order sum is then
S + c*c with S the fixed sum of the other elements, so every candidate costs
one vector of products.
"""
from __future__ import annotations

import numpy as np


def midpoint_distance(yd: np.ndarray) -> np.ndarray:
    """Relative distance from each double to the nearest midpoint between the
    float it rounds to and that float's neighbours."""
    f = yd.astype(np.float32)
    up = np.nextafter(f, np.float32(np.inf))
    dn = np.nextafter(f, np.float32(-np.inf))
    f64 = f.astype(np.float64)
    hi = (f64 + up.astype(np.float64)) * 0.5
    lo = (f64 + dn.astype(np.float64)) * 0.5
    d = np.minimum(np.abs(yd - lo), np.abs(hi - yd))
    with np.errstate(divide="ignore", invalid="ignore"):
        return np.where(yd != 0, d / np.abs(yd), np.inf)


def in_order_rmsnorm_double(x: np.ndarray, w: np.ndarray, eps: float) -> np.ndarray:
    """x*scale*gain in double, the sum of squares taken in index order."""
    x64 = x.astype(np.float64)
    ss = np.cumsum(x64 * x64)[-1]
    scale = 1.0 / np.sqrt(ss / x.size + eps)
    return (x64 * scale) * w.astype(np.float32).astype(np.float64)


def craft(x: np.ndarray, w: np.ndarray, eps: float, rel: float = 2e-15, batch: int = 512,
          max_candidates: int = 400_000) -> tuple[np.ndarray, int, float]:
    """A copy of token x (float32, [H]) with its last element changed so that
    some element's in-order x*scale*gain lies within `rel` (relative) of a
    float midpoint. Returns (token, element index, distance)."""
    H = x.size
    x = x.astype(np.float32).copy()
    x64 = x.astype(np.float64)
    g64 = w.astype(np.float32).astype(np.float64)
    S = np.cumsum(x64[:-1] * x64[:-1])[-1]
    base = float(x[-1]) if x[-1] != 0 else 0.5
    for start in range(0, max_candidates, batch):
        i = np.arange(start, start + batch, dtype=np.float64)
        c = (base * (1.0 + i * 2.0 ** -13)).astype(np.float32)
        c64 = c.astype(np.float64)
        ss = S + c64 * c64
        scale = 1.0 / np.sqrt(ss / H + eps)
        xs = np.broadcast_to(x64, (batch, H)).copy()
        xs[:, -1] = c64
        yd = (xs * scale[:, None]) * g64[None, :]
        dist = midpoint_distance(yd)
        j = int(np.argmin(dist))
        b, k = divmod(j, H)
        if dist[b, k] < rel:
            x[-1] = c[b]
            return x, k, float(dist[b, k])
    raise RuntimeError("no near-tie token found")
