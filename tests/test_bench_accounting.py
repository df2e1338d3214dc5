"""bench.py's work accounting against the measurement's per-record formulas.

The bench line's FLOP and byte figures come from per-layer aggregates
(`bench.algorithmic_work`, `bench.compulsory_bytes`).  These tests evaluate
the per-record formulas of the unit of work instead, record by record, with
the 3x3 patch counts taken by brute force:

    MAC   = n2 (5760 + 4608) + 1152 + P2 (n2 4608 + n3 (23040 + 18432) + 4608)
            + P2 P3 (n3 18432 + owner 19104)
    bytes = 128 + n2 48 8 2 + P2 n3 96 8 2 + 392 + 2

(n2, n3: in-bounds patches at s2 and s3; P2, P3: pass flags; off-grid
records do no layer work).  The per-pair terms follow the layer shapes of
`ssla_ref.py:17-93` (L4 24 -> 48, L5 48 -> 48, L6 48 -> 96, L7 96 -> 96,
head 96 -> 2 x 96 -> 7).
"""
import numpy as np
import pytest

import bench

H2, W2 = 16, 20


def _patches(x, y, H, W):
    n = 0
    for dy in (-1, 0, 1):
        for dx in (-1, 0, 1):
            if 0 <= x + dx < W and 0 <= y + dy < H:
                n += 1
    return n


def _records(seed, n=600):
    rng = np.random.default_rng(seed)
    x = rng.integers(0, W2, n).astype(np.uint16)
    y = rng.integers(0, H2, n).astype(np.uint16)
    # border-heavy and off-grid records
    x[:40] = 0
    y[40:80] = H2 - 1
    x[80:90] = W2
    y[90:95] = 0xFFFF
    p2 = (rng.random(n) < 0.3).astype(np.int8)
    p3 = (p2 & (rng.random(n) < 0.3)).astype(np.int8)
    owner = (rng.random(n) < 0.8).astype(np.int32)
    return x, y, p2, p3, owner


def _per_record(x, y, p2, p3, owner):
    mac = hid = 0
    for xi, yi, a, b, o in zip(x.tolist(), y.tolist(), p2.tolist(), p3.tolist(), owner.tolist()):
        if not (xi < W2 and yi < H2):
            continue
        n2 = _patches(xi, yi, H2, W2)
        n3 = _patches(xi >> 1, yi >> 1, H2 >> 1, W2 >> 1)
        P2, P3 = int(a == 1), int(b == 1)
        mac += (n2 * (5760 + 4608) + 1152 + P2 * (n2 * 4608 + n3 * (23040 + 18432) + 4608)
                + P2 * P3 * (n3 * 18432 + o * 19104))
        hid += n2 * 48 * 8 * 2 + P2 * n3 * 96 * 8 * 2
    return mac, hid


@pytest.mark.parametrize("seed", [1, 2, 3])
def test_macs_match_per_record_formula(seed):
    x, y, p2, p3, owner = _records(seed)
    flops, byts, iface, total_mac = bench.algorithmic_work(x, y, p2, p3, owner, H2, W2)
    want, _ = _per_record(x, y, p2, p3, owner)
    assert total_mac == want
    # every MAC phase's FLOPs are twice its MACs; the recurrences add their own
    mac_phases = [k for k in flops if not k.endswith(".apply")]
    assert sum(flops[k] for k in mac_phases) == 2 * want


@pytest.mark.parametrize("seed", [1, 2])
def test_recurrence_bytes_are_the_hidden_state_rmw(seed):
    x, y, p2, p3, owner = _records(seed)
    flops, byts, iface, _ = bench.algorithmic_work(x, y, p2, p3, owner, H2, W2)
    _, hid = _per_record(x, y, p2, p3, owner)
    assert sum(byts[f"L{i}.apply"] for i in (4, 5, 6, 7)) == hid
    # a recurrence's interface (v, g rows in, h rows out) exceeds its algorithmic bytes
    for i in (4, 5, 6, 7):
        assert iface[f"L{i}.apply"] > byts[f"L{i}.apply"]


@pytest.mark.parametrize("seed", [1, 2])
def test_compulsory_bytes_match_per_record_formula(seed):
    x, y, p2, p3, owner = _records(seed)
    _, hid = _per_record(x, y, p2, p3, owner)
    want = x.size * (128 + 392 + 2) + hid
    assert bench.compulsory_bytes(x, y, p2, H2, W2) == want


def test_a_dropped_term_is_seen():
    """The per-record formula distinguishes the layers: dropping the head's
    term (all records non-owners) changes the total by 19104 MAC per owned
    pass-3 record."""
    x, y, p2, p3, owner = _records(4)
    _, _, _, full = bench.algorithmic_work(x, y, p2, p3, owner, H2, W2)
    _, _, _, none = bench.algorithmic_work(x, y, p2, p3, np.zeros_like(owner), H2, W2)
    ok = (x < W2) & (y < H2)
    assert full - none == 19104 * int((ok & (p3 == 1) & (owner == 1)).sum())
