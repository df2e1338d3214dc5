"""Pins the oracle's YOLOX head (raw [reg0..3, obj, cls0, cls1] of
...celled.cuh:841-902, BN fold of hybrid_common.py:327-349) against the
reference's own CPU head: openeva::heads::load_yolox_level (BN fold,
async_yolox.h:81-143) + decode_yolox_cell_ct (async_yolox.h:203-254),
compiled into oracle/_ref.  The reference decodes boxes, so its raw outputs
are recovered as reg0 = cx/stride - gx, reg1 = cy/stride - gy,
reg2 = log(w/stride), reg3 = log(h/stride); obj and cls are raw logits.
"""
import ctypes

import numpy as np
import pytest

from oracle import oracle as O


def test_bn_fold_closed_form():
    rng = np.random.default_rng(2)
    W = rng.normal(0, 0.1, (96, 96)).astype(np.float32)
    g = (1 + rng.normal(0, 0.05, 96)).astype(np.float32)
    b = rng.normal(0, 0.05, 96).astype(np.float32)
    mu = rng.normal(0, 0.1, 96).astype(np.float32)
    var = rng.uniform(0.5, 2.0, 96).astype(np.float32)
    cb = rng.normal(0, 0.1, 96).astype(np.float32)
    Wf, bf = O.fuse_conv_bn(W, cb, g, b, mu, var)
    x = rng.normal(0, 1, 96)
    # conv then eval-mode BN equals the folded conv
    y = W.astype(np.float64) @ x + cb
    bn = (y - mu) / np.sqrt(var.astype(np.float64) + 1e-5) * g + b
    assert np.abs(Wf.astype(np.float64) @ x + bf - bn).max() < 1e-5
    # absent conv bias is zero
    _, bf0 = O.fuse_conv_bn(W, None, g, b, mu, var)
    assert np.abs(bf0 - (b - g / np.sqrt(var + 1e-5) * mu)).max() < 1e-6


def test_head_matches_reference_decode(stub_dir, stub_npz):
    L = O.load_ref()
    if L is None:
        pytest.skip("oracle/_ref not built (reference checkout absent)")
    head = O.head_from_npz(stub_npz)
    rng = np.random.default_rng(4)
    fp = lambda a: a.ctypes.data_as(ctypes.POINTER(ctypes.c_float))
    stride = 8.0
    for k in range(20):
        x = rng.normal(0, 1.0, 96).astype(np.float32)
        gx, gy = int(rng.integers(0, 10)), int(rng.integers(0, 8))
        row = np.zeros(7, np.float32)
        assert L.ref_head_decode(stub_dir.encode(), gx, gy, fp(x), fp(row)) == 7
        raw = np.array([row[0] / stride - gx, row[1] / stride - gy,
                        np.log(row[2] / stride), np.log(row[3] / stride),
                        row[4], row[5], row[6]])
        for prec in (64, 32):
            ours = O.head_raw(head, x, prec)
            assert np.abs(ours - raw).max() < 2e-5, (k, prec, ours, raw)


# ---- single-linear head (...celled.cuh:1476-1481) ----------------------------

def _linear_head(seed=7):
    rng = np.random.default_rng(seed)
    W = rng.normal(0, 0.1, (96, 7)).astype(np.float32)
    b = rng.normal(0, 0.1, 7).astype(np.float32)
    return W, b, O.Head.linear(W, b)


def test_linear_head_closed_forms():
    """The device layout is (IN, OUT) = (96, 7), read as head_W[i*7 + o]
    (matvec_w, orin/kernels/proto_layer_pair.cuh:39-58): a one-hot feature
    e_i returns row i of head_W plus head_b, the zero feature head_b, and the
    map is affine.  Reading the weights as (7, 96) fails the one-hot case."""
    W, b, head = _linear_head()
    for prec in (64, 32):
        assert np.array_equal(O.head_raw(head, np.zeros(96, np.float32), prec), b)
        for i in range(96):
            e = np.zeros(96, np.float32)
            e[i] = 2.0
            assert np.abs(O.head_raw(head, e, prec) - (2.0 * W[i] + b)).max() < 1e-6, (prec, i)
    rng = np.random.default_rng(8)
    x, y = rng.normal(0, 1, (2, 96)).astype(np.float32)
    fx, fy = O.head_raw(head, x) - b, O.head_raw(head, y) - b
    fxy = O.head_raw(head, (0.5 * x - 1.5 * y).astype(np.float32)) - b
    assert np.abs(fxy - (0.5 * fx - 1.5 * fy)).max() < 1e-5


def test_linear_head_matches_reference_matvec():
    """Against the reference's own prim::matvec_ct<96, 7> (vendor/openeva/prim/
    linear.h:80-91, (OUT, IN) weights) built into oracle/_ref, fed head_W
    transposed: sums and bias."""
    L = O.load_ref()
    if L is None or not hasattr(L, "ref_matvec96x7"):
        pytest.skip("oracle/_ref not built (reference checkout absent)")
    W, b, head = _linear_head(9)
    Wt = np.ascontiguousarray(W.T)
    fp = lambda a: a.ctypes.data_as(ctypes.POINTER(ctypes.c_float))
    rng = np.random.default_rng(10)
    for k in range(20):
        x = rng.normal(0, 2.0, 96).astype(np.float32)
        ref = np.zeros(7, np.float32)
        assert L.ref_matvec96x7(fp(x), fp(Wt), fp(b), fp(ref)) == 0
        for prec in (64, 32):
            assert np.abs(O.head_raw(head, x, prec) - ref).max() < 1e-5, (k, prec)


def test_schedule_with_linear_head(stub_npz):
    """The drain schedule writes the single-linear head's raw outputs for
    owned pass-3 records (from their L7 output) and zeros elsewhere."""
    from ssla_hip import events
    W, b, head = _linear_head(11)
    rec = events.blob_records(3000, seed=4)
    own = (np.arange(3000) % 5 != 0).astype(np.uint8)
    st = O.S2S3(O.layers_from_npz(stub_npz), 16, 20, 4, head=head)
    p2, p3, feat, h7 = st.run(rec.x, rec.y, rec.feat1, owner=own, want_head=True)
    m = (p3 == 1) & (own == 1)
    assert m.sum() > 50 and ((p3 == 1) & (own == 0)).sum() > 5
    exp = feat[m].astype(np.float64) @ W.astype(np.float64) + b
    assert np.abs(h7[m] - exp).max() < 1e-5
    assert np.all(h7[~m] == 0)
