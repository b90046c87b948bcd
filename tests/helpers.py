"""Shared test helpers: seeded inputs, tolerances, golden loading."""
from __future__ import annotations

import json
import os

import numpy as np

GOLDEN = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden")

# fp32 attention outputs: |a - b| <= ATOL + RTOL * |b|  (BASELINE.json north_star)
ATOL = 1e-5
RTOL = 1e-4


def assert_close(got, want, atol=ATOL, rtol=RTOL, what=""):
    got = np.asarray(got, np.float64)
    want = np.asarray(want, np.float64)
    assert got.shape == want.shape, (got.shape, want.shape)
    err = np.abs(got - want)
    bound = atol + rtol * np.abs(want)
    bad = err > bound
    if bad.any():
        i = int(np.argmax(err - bound))
        raise AssertionError(
            f"{what}: {int(bad.sum())}/{bad.size} elements out of tolerance; worst index {i} "
            f"got {got.flat[i]!r} want {want.flat[i]!r} (err {err.flat[i]:.3e})")


def rng(seed: int) -> np.random.Generator:
    return np.random.default_rng(seed)


def normal(seed: int, *shape) -> np.ndarray:
    return rng(seed).standard_normal(shape, dtype=np.float32)


class Lcg:
    """tests/kv_int8_test.cpp:24-31: uniform [-1, 1) from a 64-bit LCG."""

    def __init__(self, seed: int):
        self.s = seed & 0xFFFFFFFFFFFFFFFF

    def next(self) -> np.float32:
        self.s = (self.s * 6364136223846793005 + 1442695040888963407) & 0xFFFFFFFFFFFFFFFF
        hi = self.s >> 32
        return np.float32(np.float32(hi) / np.float32(2147483648.0) - np.float32(1.0))

    def fill(self, n: int, mul: float = 1.0) -> np.ndarray:
        return np.array([self.next() * np.float32(mul) for _ in range(n)], np.float32)


def load_golden(name: str) -> np.ndarray:
    man = json.load(open(os.path.join(GOLDEN, "manifest.json")))
    entry = next(t for t in man["tensors"] if t["name"] == name)
    a = np.fromfile(os.path.join(GOLDEN, entry["file"]), dtype="<f4")
    return a.reshape(entry["shape"])


def softmax64(s: np.ndarray) -> np.ndarray:
    s = s - s.max()
    e = np.exp(s)
    return e / e.sum()


def rope64(x: np.ndarray, pos: int, theta: float) -> np.ndarray:
    """NeoX rope of one head vector in float64 (pairs j, j + hd/2)."""
    hd = x.shape[-1]
    half = hd // 2
    j = np.arange(half, dtype=np.float64)
    ang = pos * np.power(np.float64(theta), -2.0 * j / hd)
    c, s = np.cos(ang), np.sin(ang)
    a, b = x[..., :half].astype(np.float64), x[..., half:].astype(np.float64)
    return np.concatenate([a * c - b * s, b * c + a * s], axis=-1)


def attention64(q: np.ndarray, keys: np.ndarray, vals: np.ndarray, scale: float) -> np.ndarray:
    """Textbook single-query attention in float64: q [hd], keys/vals [n][hd]."""
    s = keys.astype(np.float64) @ q.astype(np.float64) * scale
    return softmax64(s) @ vals.astype(np.float64)
