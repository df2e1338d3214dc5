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
