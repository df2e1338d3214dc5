"""Pins the oracle's weight reshape and layer step.

- Reshape (weights_ssla.py:24-88): the fused per-position tensors must
  reproduce the per-position module forward on the unfused weights
  (u = x W_in_cat[:, p]; q, v, g = u qW^T, u vW^T, u gW^T; h = s(g) h + v;
  out += (q h) oW^T W_out_cat[p]) -- the identity of
  orin/tests/test_weights_ssla.py:29-112, restated here in fp64 numpy.
- Layer step (ssla_ref.py:17-93): against the same unfused module forward
  plus residual and LayerNorm, on interior, edge and corner events, with
  the patch offset convention delta = (1-dy)*3 + (1-dx) (ssla_ref.py:85).
- Primitives: the oracle's LayerNorm / LRU numerics against the reference's
  own C++ primitives (vendor/openeva/prim/layernorm.h, rnn.h) compiled into
  oracle/_ref, and the reshape products against the reference's prim::mm.
"""
import ctypes

import numpy as np
import pytest

from oracle import oracle as O


def _raw(rng, i, D, a_in, a_out):
    f = np.float32
    return dict(W_in_cat=rng.normal(0, 0.3, (i, a_in * D)).astype(f),
                W_out_cat=rng.normal(0, 0.3, (a_out * D, D)).astype(f),
                qW=rng.normal(0, 0.3, (D, D)).astype(f), vW=rng.normal(0, 0.3, (D, D)).astype(f),
                gW=rng.normal(0, 0.3, (D, D)).astype(f), oW=rng.normal(0, 0.3, (D, D)).astype(f))


def module_patch(raw, x, h, p):
    """One patch of the unfused module forward in fp64; returns (out, h_new)."""
    D = raw["qW"].shape[0]
    n_in = raw["W_in_cat"].shape[1] // D
    n_out = raw["W_out_cat"].shape[0] // D
    pin = 0 if n_in == 1 else p
    pout = 0 if n_out == 1 else p
    d = lambda a: a.astype(np.float64)
    u = d(x) @ d(raw["W_in_cat"][:, pin * D:(pin + 1) * D])
    q, v, g = u @ d(raw["qW"]).T, u @ d(raw["vW"]).T, u @ d(raw["gW"]).T
    hn = 1.0 / (1.0 + np.exp(-g)) * d(h) + v
    o = (q * hn) @ d(raw["oW"]).T
    return o @ d(raw["W_out_cat"][pout * D:(pout + 1) * D, :]), hn


@pytest.mark.parametrize("in_dim,D,a_in,a_out", [
    (2, 12, 1, 1),      # K = 1 (SSLA-S layer 0)
    (2, 12, 9, 9),
    (24, 48, 9, 9),     # L4
    (96, 96, 9, 9),     # L7
    (12, 24, 9, 1),     # scatter-only positions
    (12, 24, 1, 9),     # gather-only positions
])
def test_reshape_identity(in_dim, D, a_in, a_out):
    rng = np.random.default_rng(in_dim * 1000 + D + a_in * 7 + a_out)
    raw = _raw(rng, in_dim, D, a_in, a_out)
    qvg, go = O.reshape(**raw)
    A = max(a_in, a_out)
    assert qvg.shape == (A, 3 * D, in_dim) and go.shape == (A, D, D)
    x = rng.normal(0, 0.5, in_dim).astype(np.float32)
    h0 = rng.normal(0, 0.3, (A, D)).astype(np.float32)
    for p in range(A):
        ref_out, ref_h = module_patch(raw, x, h0[p], p)
        qv = qvg[p].astype(np.float64) @ x.astype(np.float64)
        q, v, g = qv[:D], qv[D:2 * D], qv[2 * D:]
        hn = 1.0 / (1.0 + np.exp(-g)) * h0[p].astype(np.float64) + v
        out = go[p].astype(np.float64) @ (q * hn)
        atol = 16 * 1.2e-7 * D * A * max(1.0, np.abs(ref_out).max())
        assert np.abs(out - ref_out).max() < atol
        assert np.abs(hn - ref_h).max() < atol


def module_layer(raws, ip, gamma, beta, x, H, ev_x, ev_y, Hl, Wl):
    """Residual + sum over in-bounds patches + fp64 LayerNorm, unfused weights."""
    D = raws["qW"].shape[0]
    res = (ip.astype(np.float64) @ x.astype(np.float64)) if ip is not None else x.astype(np.float64)
    acc = np.zeros(D)
    for dy in (-1, 0, 1):
        for dx in (-1, 0, 1):
            py, px = ev_y + dy, ev_x + dx
            if not (0 <= py < Hl and 0 <= px < Wl):
                continue
            p = (1 - dy) * 3 + (1 - dx)
            o, hn = module_patch(raws, x, H[py * Wl + px], p)
            H[py * Wl + px] = hn.astype(np.float32)
            acc += o
    y = acc + res
    mu = y.mean()
    inv = 1.0 / np.sqrt(((y - mu) ** 2).mean() + 1e-5)
    return ((y - mu) * inv * gamma + beta).astype(np.float32)


@pytest.mark.parametrize("in_dim,D", [(24, 48), (48, 48), (48, 96), (96, 96)])
@pytest.mark.parametrize("pos", [(3, 2), (0, 0), (4, 0), (5, 3), (0, 2)])
def test_layer_step_matches_module_forward(in_dim, D, pos):
    rng = np.random.default_rng(in_dim + 3 * D + 11 * pos[0] + 17 * pos[1])
    Hl, Wl = 4, 6
    raw = _raw(rng, in_dim, D, 9, 9)
    ip = rng.normal(0, 0.3, (D, in_dim)).astype(np.float32) if in_dim != D else None
    gamma = (1 + rng.normal(0, 0.1, D)).astype(np.float32)
    beta = rng.normal(0, 0.1, D).astype(np.float32)
    qvg, go = O.reshape(**raw)
    layer = O.Layer(qvg, go, ip, gamma, beta, 3)
    H = rng.normal(0, 0.3, (Hl * Wl, D)).astype(np.float32)
    H_ref = H.copy()
    # three events in a row at the same place exercise the state update
    for k in range(3):
        x = rng.normal(0, 0.5, in_dim).astype(np.float32)
        out = O.layer_step(layer, x, H, pos[0], pos[1], Hl, Wl, precision=64)
        ref = module_layer(raw, ip, gamma, beta, x, H_ref, pos[0], pos[1], Hl, Wl)
        assert np.abs(out - ref).max() < 1e-4, k
        assert np.abs(H - H_ref).max() < 1e-5, k
        # cells outside the 3x3 neighbourhood are untouched by construction
    far = [c for c in range(Hl * Wl) if abs(c % Wl - pos[0]) > 1 or abs(c // Wl - pos[1]) > 1]
    assert np.array_equal(H[far], H_ref[far])


def test_layer_step_f32_close_to_f64():
    rng = np.random.default_rng(5)
    raw = _raw(rng, 48, 96, 9, 9)
    qvg, go = O.reshape(**raw)
    ip = rng.normal(0, 0.3, (96, 48)).astype(np.float32)
    layer = O.Layer(qvg, go, ip, np.ones(96, np.float32), np.zeros(96, np.float32), 3)
    H64 = rng.normal(0, 0.3, (8 * 10, 96)).astype(np.float32)
    H32 = H64.copy()
    for k in range(50):
        x = rng.normal(0, 0.5, 48).astype(np.float32)
        ex, ey = int(rng.integers(0, 10)), int(rng.integers(0, 8))
        a = O.layer_step(layer, x, H64, ex, ey, 8, 10, 64)
        b = O.layer_step(layer, x, H32, ex, ey, 8, 10, 32)
        assert np.abs(a - b).max() < 5e-5


def test_layer_step_f64_same_on_both_weight_layouts():
    """The fp64 step runs its dot products over input-major copies of qvgIn
    and goW when the layer struct carries them; each sum keeps its terms and
    their order, so outputs and states equal the row-major run bit for bit."""
    rng = np.random.default_rng(9)
    for in_dim, D in ((24, 48), (48, 96), (96, 96)):
        raw = _raw(rng, in_dim, D, 9, 9)
        qvg, go = O.reshape(**raw)
        ip = rng.normal(0, 0.3, (D, in_dim)).astype(np.float32) if in_dim != D else None
        layer = O.Layer(qvg, go, ip, np.ones(D, np.float32), np.zeros(D, np.float32), 3)
        Ha = rng.normal(0, 0.3, (6 * 7, D)).astype(np.float32)
        Hb = Ha.copy()
        fn = O.load().oracle_layer_step_f64
        for k in range(20):
            x = rng.normal(0, 0.5, in_dim).astype(np.float32)
            ex, ey = int(rng.integers(0, 7)), int(rng.integers(0, 6))
            La = layer.c()
            Lb = layer.c()
            Lb.qvgInT = None
            Lb.goWT = None
            assert La.qvgInT and La.goWT
            oa, ob = np.zeros(D, np.float32), np.zeros(D, np.float32)
            fn(ctypes.byref(La), O._fp(x), O._fp(Ha), ex, ey, 6, 7, O._fp(oa))
            fn(ctypes.byref(Lb), O._fp(x), O._fp(Hb), ex, ey, 6, 7, O._fp(ob))
            assert np.array_equal(oa, ob) and np.array_equal(Ha, Hb), (in_dim, D, k)


def test_zero_weights_reduce_to_layernorm_of_residual():
    D, i = 48, 24
    z = lambda *s: np.zeros(s, np.float32)
    rng = np.random.default_rng(1)
    ip = rng.normal(0, 0.3, (D, i)).astype(np.float32)
    g = (1 + rng.normal(0, 0.1, D)).astype(np.float32)
    b = rng.normal(0, 0.1, D).astype(np.float32)
    layer = O.Layer(z(9, 3 * D, i), z(9, D, D), ip, g, b, 3)
    H = rng.normal(0, 1, (12, D)).astype(np.float32)
    H0 = H.copy()
    x = rng.normal(0, 0.5, i).astype(np.float32)
    out = O.layer_step(layer, x, H, 1, 1, 3, 4, 64)
    r = ip.astype(np.float64) @ x
    ref = (r - r.mean()) / np.sqrt(r.var() + 1e-5) * g + b
    assert np.abs(out - ref).max() < 1e-5
    # zero gates: sigmoid(0) = 1/2 halves every touched hidden cell, v = 0
    touched = [0, 1, 2, 4, 5, 6, 8, 9, 10]
    assert np.allclose(H[touched], H0[touched] * 0.5)
    assert np.array_equal(H[[3, 7, 11]], H0[[3, 7, 11]])


def _ref():
    L = O.load_ref()
    if L is None:
        pytest.skip("oracle/_ref not built (reference checkout absent)")
    return L


def test_primitives_match_reference_cpp():
    L = _ref()
    rng = np.random.default_rng(3)
    fp = lambda a: a.ctypes.data_as(ctypes.POINTER(ctypes.c_float))
    for D in (48, 96):
        # LayerNorm: the oracle's fp64 LN, reached through a zero-weight
        # layer with identity residual, equals prim::layernorm_ct.
        x = rng.normal(0, 2, D).astype(np.float32)
        g = (1 + rng.normal(0, 0.1, D)).astype(np.float32)
        b = rng.normal(0, 0.1, D).astype(np.float32)
        ref = x.copy()
        assert L.ref_layernorm(fp(ref), D, fp(g), fp(b)) == 0
        z = np.zeros
        layer = O.Layer(z((9, 3 * D, D), np.float32), z((9, D, D), np.float32), None, g, b, 3)
        out = O.layer_step(layer, x, np.zeros((9, D), np.float32), 1, 1, 3, 3, 64)
        assert np.array_equal(out, ref)
        # LRU step: h = sigmoid(g) h + v; y = q h  (prim::lru_step, fp32)
        gg, v, q = (rng.normal(0, 1, D).astype(np.float32) for _ in range(3))
        h = rng.normal(0, 1, D).astype(np.float32)
        h_ref, y_ref = h.copy(), np.zeros(D, np.float32)
        assert L.ref_lru_step(fp(gg), fp(v), fp(q), fp(h_ref), fp(y_ref), D) == 0
        hn = 1 / (1 + np.exp(-gg.astype(np.float64))) * h + v
        assert np.abs(hn - h_ref).max() < 1e-5 and np.abs(q * hn - y_ref).max() < 1e-5


def test_reshape_products_match_reference_mm():
    L = _ref()
    rng = np.random.default_rng(9)
    raw = _raw(rng, 24, 48, 9, 9)
    qvg, go = O.reshape(**raw)
    fp = lambda a: a.ctypes.data_as(ctypes.POINTER(ctypes.c_float))
    for p in (0, 4, 8):
        scatter = np.ascontiguousarray(raw["W_in_cat"][:, p * 48:(p + 1) * 48].T)
        gather = np.ascontiguousarray(raw["W_out_cat"][p * 48:(p + 1) * 48, :].T)
        for part, W in enumerate((raw["qW"], raw["vW"], raw["gW"])):
            C = np.zeros((48, 24), np.float32)
            assert L.ref_mm(fp(W), 48, 48, fp(scatter), 24, fp(C)) == 0
            assert np.array_equal(qvg[p, part * 48:(part + 1) * 48], C)
        C = np.zeros((48, 48), np.float32)
        assert L.ref_mm(fp(gather), 48, 48, fp(raw["oW"]), 48, fp(C)) == 0
        assert np.array_equal(go[p], C)
