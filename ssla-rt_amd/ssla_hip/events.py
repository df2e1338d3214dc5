"""Synthetic event and ring-record streams for the drain path.

Each generator is seeded and returns plain numpy arrays.  Ring records are
post-stage-1 events at s2 coordinates (x, y on the H/4 x W/4 grid) with a
24-float feature, laid out with abi.INPUT_DTYPE by `to_records`.

  p1_replica        the P1 correctness workload: the random-draw order of
                    orin/orin/hybrid_common.py:152-211 (four random layers
                    with N(0, 0.05^2) initial hidden state) followed by
                    orin/bench_s2_s3_head_celled.py:131-134 (t, x, y, feat1),
                    which reproduces the published pass counts 50124 / 12562
                    at n = 200000, seed 1 (docs/archive/STATUS.md:1384-1385)
  raw_uniform       raw sensor events: x, y uniform, polarity +-1, Exp
                    inter-arrival (the CPU reference workload)
  blob_records      ring records from moving Gaussian blobs plus uniform
                    background (the offline-drain workload)
  edge_blob_records ring records at 640x480 from elongated moving blobs
                    plus hot-pixel bursts (the scaled-resolution workload)
"""
from __future__ import annotations

from dataclasses import dataclass
from typing import List, Optional

import numpy as np

from .abi import C1, C2, C3, INPUT_DTYPE

# (in, out) of the four GPU layers L4..L7, all K = 3
GPU_LAYER_IO = ((C1, C2), (C2, C2), (C2, C3), (C3, C3))


@dataclass
class RawLayer:
    """Unfused weights of one SSLA layer as stored in weights.npz."""
    W_in_cat: np.ndarray          # (in, 9*out)
    W_out_cat: np.ndarray         # (9*out, out)
    qW: np.ndarray
    vW: np.ndarray
    gW: np.ndarray
    oW: np.ndarray
    input_proj: Optional[np.ndarray]   # (out, in) or None
    ln_gamma: np.ndarray
    ln_beta: np.ndarray


@dataclass
class Records:
    t: np.ndarray       # float32 (n,)
    x: np.ndarray       # uint16 (n,) s2 x
    y: np.ndarray       # uint16 (n,) s2 y
    feat1: np.ndarray   # float32 (n, 24)


@dataclass
class P1Workload:
    layers: List[RawLayer]
    h_init: List[np.ndarray]      # (cells, out) float32 per layer
    rec: Records
    H2: int
    W2: int


def p1_replica(n: int = 200_000, seed: int = 1, H2: int = 16, W2: int = 20) -> P1Workload:
    rng = np.random.default_rng(seed)
    H3, W3 = H2 >> 1, W2 >> 1
    f32 = np.float32
    layers, h_init = [], []
    for li, (i, o) in enumerate(GPU_LAYER_IO):
        Win = rng.normal(scale=0.3, size=(i, 9 * o)).astype(f32)
        Wout = rng.normal(scale=0.3, size=(9 * o, o)).astype(f32)
        qW = rng.normal(scale=0.3, size=(o, o)).astype(f32)
        vW = rng.normal(scale=0.3, size=(o, o)).astype(f32)
        gW = rng.normal(scale=0.3, size=(o, o)).astype(f32)
        oW = rng.normal(scale=0.3, size=(o, o)).astype(f32)
        ip = rng.normal(scale=0.3, size=(o, i)).astype(f32) if i != o else None
        gamma = (rng.normal(scale=0.1, size=o) + 1.0).astype(f32)
        beta = rng.normal(scale=0.1, size=o).astype(f32)
        cells = H2 * W2 if li < 2 else H3 * W3
        h_init.append(rng.normal(scale=0.05, size=(cells, o)).astype(f32))
        layers.append(RawLayer(Win, Wout, qW, vW, gW, oW, ip, gamma, beta))
    t = rng.uniform(0, 1, n).astype(f32)
    x = rng.integers(0, W2, n).astype(np.uint16)
    y = rng.integers(0, H2, n).astype(np.uint16)
    feat1 = rng.normal(scale=0.5, size=(n, C1)).astype(f32)
    return P1Workload(layers, h_init, Records(t, x, y, feat1), H2, W2)


def raw_uniform(n: int = 50_000, seed: int = 1, height: int = 64, width: int = 80,
                rate_mev: float = 2.0) -> np.ndarray:
    """(n, 4) float32 [t_us, x, y, p] with p = +-1 and monotone t."""
    rng = np.random.default_rng(seed)
    x = rng.integers(0, width, n)
    y = rng.integers(0, height, n)
    p = np.where(rng.random(n) < 0.5, -1.0, 1.0)
    dt = rng.exponential(1.0 / rate_mev, n)
    t = np.cumsum(dt) - dt[0]
    return np.stack([t, x, y, p], axis=1).astype(np.float32)


def _reflect(v: np.ndarray, hi: float) -> np.ndarray:
    """Fold positions into [0, hi] as a point bouncing between the walls."""
    period = 2.0 * hi
    m = np.mod(v, period)
    return np.where(m > hi, period - m, m)


def blob_records(n: int = 200_000, seed: int = 1, height: int = 64, width: int = 80,
                 n_blobs: int = 8, sigma: float = 3.0, bg_frac: float = 0.1,
                 rec_rate_hz: float = 2.0e6 / 16) -> Records:
    """Ring records from n_blobs Gaussian blobs (sigma in sensor pixels)
    moving at 0.5-2 px/ms with reflection at the borders, plus bg_frac
    uniform background.  Sensor coordinates are mapped to s2 with >> 2."""
    rng = np.random.default_rng(seed)
    dt = rng.exponential(1e6 / rec_rate_hz, n)           # microseconds
    t_us = np.cumsum(dt) - dt[0]
    start = rng.uniform([0, 0], [width - 1, height - 1], size=(n_blobs, 2))
    speed = rng.uniform(0.5, 2.0, n_blobs) / 1000.0      # px per microsecond
    ang = rng.uniform(0, 2 * np.pi, n_blobs)
    vel = np.stack([np.cos(ang), np.sin(ang)], axis=1) * speed[:, None]
    which = rng.integers(0, n_blobs, n)
    from_bg = rng.random(n) < bg_frac
    cx = _reflect(start[which, 0] + vel[which, 0] * t_us, width - 1)
    cy = _reflect(start[which, 1] + vel[which, 1] * t_us, height - 1)
    px = np.rint(cx + rng.normal(0, sigma, n))
    py = np.rint(cy + rng.normal(0, sigma, n))
    ux = rng.integers(0, width, n)
    uy = rng.integers(0, height, n)
    px = np.where(from_bg, ux, np.clip(px, 0, width - 1)).astype(np.int64)
    py = np.where(from_bg, uy, np.clip(py, 0, height - 1)).astype(np.int64)
    rng.random(n)                                        # polarity draw (unused at s2)
    feat1 = rng.normal(scale=0.5, size=(n, C1)).astype(np.float32)
    return Records(t_us.astype(np.float32), (px >> 2).astype(np.uint16),
                   (py >> 2).astype(np.uint16), feat1)


def edge_blob_records(n: int, seed: int = 1, height: int = 480, width: int = 640,
                      n_blobs: int = 64, hot_frac: float = 0.05,
                      hot_pixel_frac: float = 0.01,
                      rec_rate_hz: float = 20e6 / 16) -> Records:
    """Ring records of a full-resolution sensor: elongated blobs (edges,
    sigma 8 x 1.5 px, random orientation) moving at 0.5-2 px/ms, plus
    hot_frac of records from a fixed set of hot pixels (hot_pixel_frac of
    the sensor).  Mapped to s2 with >> 2."""
    rng = np.random.default_rng(seed)
    dt = rng.exponential(1e6 / rec_rate_hz, n)
    t_us = np.cumsum(dt) - dt[0]
    start = rng.uniform([0, 0], [width - 1, height - 1], size=(n_blobs, 2))
    speed = rng.uniform(0.5, 2.0, n_blobs) / 1000.0
    ang = rng.uniform(0, 2 * np.pi, n_blobs)
    vel = np.stack([np.cos(ang), np.sin(ang)], axis=1) * speed[:, None]
    orient = rng.uniform(0, np.pi, n_blobs)
    which = rng.integers(0, n_blobs, n)
    a = rng.normal(0, 8.0, n)
    b = rng.normal(0, 1.5, n)
    co, so = np.cos(orient[which]), np.sin(orient[which])
    cx = _reflect(start[which, 0] + vel[which, 0] * t_us, width - 1) + a * co - b * so
    cy = _reflect(start[which, 1] + vel[which, 1] * t_us, height - 1) + a * so + b * co
    n_hot = max(1, int(hot_pixel_frac * width * height))
    hot = rng.integers(0, width * height, n_hot)
    is_hot = rng.random(n) < hot_frac
    hp = hot[rng.integers(0, n_hot, n)]
    px = np.where(is_hot, hp % width, np.clip(np.rint(cx), 0, width - 1)).astype(np.int64)
    py = np.where(is_hot, hp // width, np.clip(np.rint(cy), 0, height - 1)).astype(np.int64)
    feat1 = rng.normal(scale=0.5, size=(n, C1)).astype(np.float32)
    return Records(t_us.astype(np.float32), (px >> 2).astype(np.uint16),
                   (py >> 2).astype(np.uint16), feat1)


def to_records(r: Records) -> np.ndarray:
    """Pack into abi.INPUT_DTYPE ring records (seq_done = slot + 1)."""
    n = r.x.size
    out = np.zeros(n, dtype=INPUT_DTYPE)
    out["seq_done"] = np.arange(1, n + 1, dtype=np.uint64)
    out["t"] = r.t
    out["x"] = r.x
    out["y"] = r.y
    out["feat1"] = r.feat1
    return out
