"""Pins the composition of the oracle's drain schedule (oracle_s2s3_run).

The schedule follows orin/bench_s2_s3_head_celled.py:53-86 (and the kernel's
masks, orin/kernels/ssla_s2_s3_head_celled.cuh:1020-1064): L4 and L5 for
every record (L5's output is consumed only by pass-2 records), tdrop_s2 at
the record's s2 cell after L5, then -- for pass-2 records only -- pooling
to the s3 cell, L6, L7 and tdrop_s3 at the s3 cell after L7; s3_feat is the
L7 output of pass-3 records.

Each layer is pinned elsewhere (test_oracle_layer.py); here the chaining is
checked against an independent chain of the unfused per-patch module
forward (module_layer, written from the unfused weights, not from the
oracle's fused tensors), and against invariants a misplaced mask or gate
would break:
  - a record dropped at s2 changes the L4/L5 state and leaves L6/L7 alone;
  - a pass-2 record dropped at s3 still advances the L6/L7 state and the
    s3 counter;
  - the s3 gate keys on the pooled cell, so two s2 cells of one s3 cell
    share its counter.
"""
import numpy as np
import pytest

from oracle import oracle as O
from test_oracle_layer import _raw, module_layer

IO = ((24, 48), (48, 48), (48, 96), (96, 96))


def state_close(a, b):
    """Hidden states grow to |h| ~ 10-20; the fused weights are rounded to
    fp32 while the module chain multiplies the unfused ones in fp64, so the
    states agree to ~2e-6 of their magnitude."""
    return np.abs(a - b).max() <= 1e-5 * max(1.0, float(np.abs(b).max()))


def _model(seed):
    rng = np.random.default_rng(seed)
    raws, ips, gammas, betas, layers = [], [], [], [], []
    for i, D in IO:
        raw = _raw(rng, i, D, 9, 9)
        ip = rng.normal(0, 0.3, (D, i)).astype(np.float32) if i != D else None
        g = (1 + rng.normal(0, 0.1, D)).astype(np.float32)
        b = rng.normal(0, 0.1, D).astype(np.float32)
        qvg, go = O.reshape(**raw)
        raws.append(raw)
        ips.append(ip)
        gammas.append(g)
        betas.append(b)
        layers.append(O.Layer(qvg, go, ip, g, b, 3))
    return raws, ips, gammas, betas, layers


def module_chain(model, xs, ys, feats, H2, W2, window):
    """The drain schedule written out on the unfused module forward."""
    raws, ips, gammas, betas, _ = model
    H3, W3 = H2 >> 1, W2 >> 1
    H = [np.zeros((H2 * W2, 48), np.float32), np.zeros((H2 * W2, 48), np.float32),
         np.zeros((H3 * W3, 96), np.float32), np.zeros((H3 * W3, 96), np.float32)]
    td2 = np.zeros(H2 * W2, np.uint8)
    td3 = np.zeros(H3 * W3, np.uint8)
    n = len(xs)
    p2 = np.zeros(n, np.int8)
    p3 = np.zeros(n, np.int8)
    feat = np.zeros((n, 96), np.float32)

    def gate(td, cell):
        pre = int(td[cell])
        td[cell] = (pre + 1) & 255
        return window <= 1 or pre % window == 0

    for k in range(n):
        x, y = int(xs[k]), int(ys[k])
        lay = lambda li, v, cx, cy, hl, wl: module_layer(raws[li], ips[li], gammas[li], betas[li],
                                                         v, H[li], cx, cy, hl, wl)
        y4 = lay(0, feats[k], x, y, H2, W2)
        y5 = lay(1, y4, x, y, H2, W2)
        if not gate(td2, y * W2 + x):
            continue
        p2[k] = 1
        x3, y3 = x >> 1, y >> 1
        y6 = lay(2, y5, x3, y3, H3, W3)
        y7 = lay(3, y6, x3, y3, H3, W3)
        if gate(td3, y3 * W3 + x3):
            p3[k] = 1
            feat[k] = y7
    return p2, p3, feat, H, td2, td3


def _oracle(model, xs, ys, feats, H2, W2, window):
    st = O.S2S3(model[4], H2, W2, window)
    p2, p3, feat, _ = st.run(np.asarray(xs), np.asarray(ys), np.asarray(feats, np.float32))
    return p2, p3, feat, st


# A hand-made sequence on a 6 x 4 s2 grid (3 x 2 at s3), window 2:
#   0 (2,1) pass2, pass3 at s3 (1,0)       1 (2,1) dropped at s2
#   2 (3,1) pass2, s3 (1,0) dropped        3 (2,1) pass2, s3 (1,0) pass3
#   4 (3,0) pass2, s3 (1,0) dropped        5 (0,0) corner   6 (5,3) corner
#   7 (5,3) dropped at s2                  8 (4,2) pass2, s3 (2,1) dropped
#                                            (record 6 reached s3 (2,1) first)
HAND = [(2, 1), (2, 1), (3, 1), (2, 1), (3, 0), (0, 0), (5, 3), (5, 3), (4, 2)]
HAND_P2 = [1, 0, 1, 1, 1, 1, 1, 0, 1]
HAND_P3 = [1, 0, 0, 1, 0, 1, 1, 0, 0]


def test_hand_sequence_decisions_and_values():
    model = _model(21)
    rng = np.random.default_rng(4)
    xs, ys = [p[0] for p in HAND], [p[1] for p in HAND]
    feats = rng.normal(0, 0.5, (len(HAND), 24)).astype(np.float32)
    p2, p3, feat, st = _oracle(model, xs, ys, feats, 4, 6, 2)
    assert p2.tolist() == HAND_P2 and p3.tolist() == HAND_P3
    r2, r3, rfeat, rH, rtd2, rtd3 = module_chain(model, xs, ys, feats, 4, 6, 2)
    assert r2.tolist() == HAND_P2 and r3.tolist() == HAND_P3
    assert np.abs(feat - rfeat).max() < 1e-4
    for li in range(4):
        assert state_close(st.H[li], rH[li]), li
    assert np.array_equal(st.td2, rtd2) and np.array_equal(st.td3, rtd3)
    # the shared s3 cells: (1,0) saw records 0, 2, 3, 4 (s2 cells (2,1),
    # (3,1), (3,0)); (2,1) saw records 6 and 8 (s2 cells (5,3), (4,2))
    assert int(st.td3[0 * 3 + 1]) == 4 and int(st.td3[1 * 3 + 2]) == 2


def test_dropped_records_touch_only_their_layers():
    model = _model(22)
    rng = np.random.default_rng(5)
    xs, ys = [p[0] for p in HAND], [p[1] for p in HAND]
    feats = rng.normal(0, 0.5, (len(HAND), 24)).astype(np.float32)
    states = []
    for k in range(len(HAND) + 1):
        _, _, _, st = _oracle(model, xs[:k], ys[:k], feats[:k], 4, 6, 2)
        states.append(st)
    for k in range(len(HAND)):
        a, b = states[k], states[k + 1]
        # every record advances L4 and L5 and its s2 counter
        assert not np.array_equal(a.H[0], b.H[0]) and not np.array_equal(a.H[1], b.H[1]), k
        assert int(b.td2.sum()) == int(a.td2.sum()) + 1
        if HAND_P2[k]:
            # pass-2 records advance L6 and L7 and the s3 counter, whether or
            # not they pass tdrop_s3
            assert not np.array_equal(a.H[2], b.H[2]) and not np.array_equal(a.H[3], b.H[3]), k
            assert int(b.td3.sum()) == int(a.td3.sum()) + 1
        else:
            assert np.array_equal(a.H[2], b.H[2]) and np.array_equal(a.H[3], b.H[3]), k
            assert np.array_equal(a.td3, b.td3)


@pytest.mark.parametrize("window", [1, 2, 3])
def test_random_sequence_matches_module_chain(window):
    model = _model(30 + window)
    rng = np.random.default_rng(window)
    n = 40
    xs = rng.integers(0, 6, n)
    ys = rng.integers(0, 4, n)
    feats = rng.normal(0, 0.5, (n, 24)).astype(np.float32)
    p2, p3, feat, st = _oracle(model, xs, ys, feats, 4, 6, window)
    r2, r3, rfeat, rH, rtd2, rtd3 = module_chain(model, xs, ys, feats, 4, 6, window)
    assert np.array_equal(p2, r2) and np.array_equal(p3, r3)
    if window == 1:
        assert p2.all() and p3.all()
    else:
        assert 0 < p2.sum() < n and 0 < p3.sum() < p2.sum()
    assert np.abs(feat - rfeat).max() < 1e-4
    for li in range(4):
        assert state_close(st.H[li], rH[li]), li
    assert np.array_equal(st.td2, rtd2) and np.array_equal(st.td3, rtd3)
