"""Host-side prediction-grid consumer of libssla_hip.so (no GPU needed).

Pins:
  - decode (async_yolox.h:189-196) and the host head row against the
    reference's own load_yolox_level + decode_yolox_cell_ct compiled into
    oracle/_ref, plus closed forms (zero raw row -> cell corner and stride
    sized box; exp/offset terms with known values);
  - box collection (hybrid_runner_multi.py:163-207) against hand-computed
    boxes: centre offset +4, 8x scaling, clipping to [2, W_full], the >=
    threshold, block order and topo in s2 units;
  - the OEVA format and diff (include/oracle.h) byte-for-byte and
    report-for-report against deploy::OracleRecorder / deploy::diff_dumps
    compiled into oracle/_ref;
  - torn-free snapshots under a concurrent writer.
"""
import ctypes
import threading
import time
import types

import numpy as np
import pytest

from oracle import oracle as O
from ssla_hip import abi, grid, lib

BUSY = abi.PRED_BUSY


def fp(a):
    return a.ctypes.data_as(ctypes.POINTER(ctypes.c_float))


def sig32(x):
    return np.float32(1.0) / (np.float32(1.0) + np.exp(np.float32(-x), dtype=np.float32))


# ---- decode -----------------------------------------------------------------

def test_decode_closed_form():
    raw = np.zeros((6, 7), np.float32)
    raw[:, 4] = [-1, 0, 1, 2, 3, 4]
    raw[:, 5] = 0.5
    raw[:, 6] = -0.5
    out = grid.decode_cells(raw, grid_w=3, gx0=2, gy0=5, stride_w=8, stride_h=4)
    gx = 2 + np.arange(6) % 3
    gy = 5 + np.arange(6) // 3
    assert np.array_equal(out[:, 0], gx * 8.0)
    assert np.array_equal(out[:, 1], gy * 4.0)
    assert np.all(out[:, 2] == 8.0) and np.all(out[:, 3] == 4.0)
    assert np.array_equal(out[:, 4:], raw[:, 4:])       # logits stay raw
    raw[:, 0], raw[:, 1] = 0.5, -0.25
    raw[:, 2], raw[:, 3] = np.log(2.0), -np.log(4.0)
    out = grid.decode_cells(raw, grid_w=3, gx0=2, gy0=5, stride_w=8, stride_h=4)
    assert np.allclose(out[:, 0], (gx + 0.5) * 8.0, rtol=0, atol=1e-5)
    assert np.allclose(out[:, 1], (gy - 0.25) * 4.0, rtol=0, atol=1e-5)
    assert np.allclose(out[:, 2], 16.0, rtol=1e-6) and np.allclose(out[:, 3], 1.0, rtol=1e-6)


def test_decode_rejects_bad_shapes():
    with pytest.raises(ValueError):
        grid.decode_cells(np.zeros((3, 4), np.float32), grid_w=3)
    with pytest.raises(lib.SslaHipError):
        grid.decode_cells(np.zeros((3, 7), np.float32), grid_w=0)


def test_head_row_and_decode_match_reference(stub_dir):
    L = O.load_ref()
    if L is None:
        pytest.skip("oracle/_ref not built (reference checkout absent)")
    rng = np.random.default_rng(11)
    for k in range(24):
        x = np.zeros(96, np.float32) if k == 0 else rng.normal(0, 1.0, 96).astype(np.float32)
        gx, gy = int(rng.integers(0, 10)), int(rng.integers(0, 8))
        ref = np.zeros(7, np.float32)
        assert L.ref_head_decode(stub_dir.encode(), gx, gy, fp(x), fp(ref)) == 7
        raw = grid.head_row(stub_dir, x)
        ours = grid.decode_cells(raw[None], grid_w=10, gx0=gx, gy0=gy)[0]
        assert np.allclose(ours, ref, rtol=1e-5, atol=2e-5), (k, ours, ref)


def test_head_row_errors(tmp_path):
    with pytest.raises(lib.SslaHipError):
        grid.head_row(str(tmp_path / "missing"))


# ---- snapshot -----------------------------------------------------------------

def test_snapshot_copies_and_flags_busy_cells():
    rng = np.random.default_rng(3)
    preds = rng.normal(0, 1, (50, 7)).astype(np.float32)
    version = rng.integers(0, 1000, 50).astype(np.uint32)
    p, v, torn = grid.snapshot(preds, version)
    assert torn == 0 and np.array_equal(p, preds) and np.array_equal(v, version)
    version[[3, 17]] |= BUSY
    p, v, torn = grid.snapshot(preds, version, max_tries=3)
    assert torn == 2
    assert set(np.nonzero(v & BUSY)[0]) == {3, 17}
    ok = (v & BUSY) == 0
    assert np.array_equal(p[ok], preds[ok]) and np.array_equal(v[ok], version[ok])
    with pytest.raises(ValueError):
        grid.snapshot(preds[:, :3].copy(), version[:10].copy())


def test_snapshot_never_returns_a_torn_cell_under_a_writer():
    """A writer thread rewrites cells as version|BUSY, 7 values, version;
    every cell a snapshot returns without the busy bit is whole."""
    n = 8
    preds = np.zeros((n, 7), np.float32)
    version = np.zeros(n, np.uint32)
    stop = threading.Event()

    def writer():
        k = 1
        while not stop.is_set() and k < (1 << 22):
            c = k % n
            version[c] = np.uint32(int(version[c]) | BUSY)
            preds[c, :] = float(k)
            version[c] = np.uint32(k)
            k += 1

    t = threading.Thread(target=writer)
    t.start()
    checked = 0
    try:
        t_end = time.monotonic() + 1.0
        while time.monotonic() < t_end:
            p, v, torn = grid.snapshot(preds, version, max_tries=4)
            ok = (v & BUSY) == 0
            assert torn == int((~ok).sum())
            assert np.all(p[ok] == v[ok, None].astype(np.float32)), (p[ok], v[ok])
            checked += int(ok.sum())
    finally:
        stop.set()
        t.join()
    assert checked > 0


# ---- whole-grid decode -----------------------------------------------------------

def test_grid_decode_fills_unwritten_and_unowned_cells():
    H3, W3 = 4, 6
    cfg = abi.HybridS2S3Config()
    cfg.H3, cfg.W3, cfg.n_blocks = H3, W3, 2
    boxes = [(0, 3, 0, 4), (3, 5, 1, 4)]   # s3 x_lo, x_hi, y_lo, y_hi; column 5 unowned
    rng = np.random.default_rng(5)
    keep = []
    for b, (xl, xh, yl, yh) in enumerate(boxes):
        s = cfg.strip[b]
        s.s3_owned_lo, s.s3_owned_hi, s.s3_owned_y_lo, s.s3_owned_y_hi = xl, xh, yl, yh
        n = (xh - xl) * (yh - yl)
        p = rng.normal(0, 0.5, (n, 7)).astype(np.float32)
        v = rng.integers(0, 3, n).astype(np.uint32)
        keep += [p, v]
        cfg.preds[b] = p.ctypes.data
        cfg.version[b] = v.ctypes.data
    zero = np.array([0.1, -0.2, 0.3, -0.4, -3.0, 1.0, -1.0], np.float32)
    out, torn = grid.grid_decode(cfg, zero, 8, 8)
    assert torn == 0
    raw = np.tile(zero, (H3 * W3, 1))
    for b, (xl, xh, yl, yh) in enumerate(boxes):
        p, v = keep[2 * b], keep[2 * b + 1]
        w = xh - xl
        for i in np.nonzero(v)[0]:
            raw[(yl + i // w) * W3 + xl + i % w] = p[i]
    want = grid.decode_cells(raw, grid_w=W3)
    assert np.array_equal(out, want)
    # a busy cell is reported and left at the zero row
    keep[1][0] |= BUSY
    out, torn = grid.grid_decode(cfg, zero, 8, 8, max_tries=2)
    assert torn == 1
    assert np.array_equal(out[0], grid.decode_cells(zero[None], grid_w=W3)[0])
    # an owned box outside the grid is an error
    cfg.strip[1].s3_owned_hi = W3 + 1
    with pytest.raises(lib.SslaHipError):
        grid.grid_decode(cfg, zero)


# ---- box collection ------------------------------------------------------------------

def test_collect_boxes_known_answer():
    s3w, s3h, x_lo, y_lo = 3, 2, 2, 1
    raw = np.zeros((s3w * s3h, 7), np.float32)
    raw[:, 4] = -5.0
    raw[4] = [0.25, -0.5, np.log(3.0), np.log(0.1), 2.0, 0.0, 0.0]   # s3 (x=3, y=2)
    strip = abi.HybridStrip()
    strip.s3_owned_lo, strip.s3_owned_hi = x_lo, x_lo + s3w
    strip.s3_owned_y_lo, strip.s3_owned_y_hi = y_lo, y_lo + s3h
    boxes, scores, mx = grid.collect_bboxes([raw], [strip], 0, 0, 1.5, 0.3, 80, 64)
    # cx = 3*8 + 4 + 0.25*8 = 30, cy = 2*8 + 4 - 4 = 16, w = 24, h = clip(0.8) = 2
    assert len(boxes) == 1
    assert np.allclose(boxes[0], [(30 - 12) * 1.5, (16 - 1) * 1.5, 36.0, 3.0], atol=1e-5)
    assert scores[0] == pytest.approx(float(sig32(2.0)), abs=1e-7)
    assert mx == pytest.approx(float(sig32(2.0)), abs=1e-7)


def test_collect_boxes_threshold_clip_order_and_topo():
    raw = np.zeros((4, 7), np.float32)          # 2x2 box, all obj logits 0 -> 0.5
    raw[1, 2] = 10.0                            # exp(10)*8 -> clipped to W_full
    raw[2, 3] = 10.0                            # -> clipped to H_full
    topo = [types.SimpleNamespace(owned_x_lo=4, owned_x_hi=8, owned_y_lo=2, owned_y_hi=6),
            types.SimpleNamespace(owned_x_lo=8, owned_x_hi=8, owned_y_lo=0, owned_y_hi=4),
            types.SimpleNamespace(owned_x_lo=0, owned_x_hi=4, owned_y_lo=0, owned_y_hi=4)]
    raw_b2 = raw.copy()
    raw_b2[:, 4] = [1.0, -1.0, 1.0, -1.0]
    views = [raw, np.zeros((0, 7), np.float32), raw_b2]
    boxes, scores, mx = grid.collect_bboxes(views, topo, 0, 0, 1.0, 0.5, 80, 64)
    # block 0: every cell (0.5 >= 0.5); block 1 empty; block 2: cells 0 and 2
    assert len(boxes) == 6 and scores[:4] == [0.5] * 4
    assert mx == pytest.approx(float(sig32(1.0)))
    b = np.array(boxes)
    # block 0 sits at s3 (2, 1): cell 0 centre (2*8+4, 1*8+4) = (20, 12), 8x8
    assert np.allclose(b[0], [16, 8, 8, 8])
    assert b[1, 2] == 80.0 and b[2, 3] == 64.0
    # block 2 at s3 (0, 0): cell 2 (0, 1) keeps the copied h = 64 clip, cy = 12
    assert np.allclose(b[4], [0, 0, 8, 8]) and np.allclose(b[5], [0, 12 - 32, 8, 64])
    # strictly above 0.5 drops the logit-0 cells
    boxes, _, _ = grid.collect_bboxes(views, topo, 0, 0, 1.0, float(np.nextafter(np.float32(0.5),
                                                                             np.float32(1))),
                                      80, 64)
    assert len(boxes) == 2
    with pytest.raises(ValueError):
        grid.collect_bboxes([raw[:3]], topo[:1], 0, 0, 1.0, 0.5, 80, 64)


# ---- OEVA dumps -----------------------------------------------------------------------

def _cps(rng, n, na=12, cols=7):
    return [rng.normal(0, 10, (na, cols)).astype(np.float32) for _ in range(n)]


def test_oeva_roundtrip_and_errors(tmp_path):
    rng = np.random.default_rng(1)
    preds = _cps(rng, 3)
    path = tmp_path / "a.oeva"
    grid.write_dump(path, 12, 7, [0, 5, 10], preds)
    raw = path.read_bytes()
    assert raw[:20] == np.array([0x4F455641, 1, 12, 7, 3], "<u4").tobytes()
    assert len(raw) == 20 + 3 * (8 + 12 * 7 * 4)
    idx, got = grid.read_dump(path)
    assert list(idx) == [0, 5, 10] and np.array_equal(got, np.stack(preds))
    # truncated body: the short read keeps the 25 floats it got, the rest
    # of that checkpoint and every later one stay zero (fread semantics)
    (tmp_path / "t.oeva").write_bytes(raw[:20 + 8 + 12 * 7 * 4 + 8 + 100])
    idx, got = grid.read_dump(tmp_path / "t.oeva")
    assert np.array_equal(got[0], preds[0])
    assert np.array_equal(got[1].reshape(-1)[:25], preds[1].reshape(-1)[:25])
    assert not got[1].reshape(-1)[25:].any() and not got[2].any() and list(idx) == [0, 5, 0]
    bad = bytearray(raw)
    bad[0] ^= 1
    (tmp_path / "b.oeva").write_bytes(bytes(bad))
    with pytest.raises(lib.SslaHipError, match="magic"):
        grid.read_dump(tmp_path / "b.oeva")
    (tmp_path / "s.oeva").write_bytes(raw[:12])
    with pytest.raises(lib.SslaHipError, match="header"):
        grid.read_dump(tmp_path / "s.oeva")
    # a corrupt header (2^32 - 1 checkpoints of 12 x 7) is refused before
    # anything is allocated from it
    huge = np.array([0x4F455641, 1, 12, 7, 0xFFFFFFFF], "<u4").tobytes() + raw[20:]
    (tmp_path / "h.oeva").write_bytes(huge)
    with pytest.raises(lib.SslaHipError, match="implausible"):
        grid.read_dump(tmp_path / "h.oeva")
    with pytest.raises(lib.SslaHipError, match="cannot open"):
        grid.diff_dumps(path, tmp_path / "missing.oeva")


def test_recorder_policy(tmp_path):
    rec = grid.OracleRecorder(4, 7, 3, str(tmp_path / "r.oeva"))
    p = np.ones((4, 7), np.float32)
    for i in range(8):
        rec.record(i, p * i)
    rec.record(9, np.ones(5, np.float32))     # wrong size: head not ready, skipped
    rec.record(12, None)
    assert rec.num_checkpoints() == 3
    rec.save()
    idx, got = grid.read_dump(tmp_path / "r.oeva")
    assert list(idx) == [0, 3, 6] and got[2][0, 0] == 6.0
    off = grid.OracleRecorder(4, 7, 0, str(tmp_path / "o.oeva"))
    off.record(0, p)
    assert off.num_checkpoints() == 0
    with pytest.raises(ValueError):
        grid.OracleRecorder(0, 7, 1, "x")


def test_oeva_file_matches_reference_recorder(tmp_path):
    L = O.load_ref()
    if L is None or not hasattr(L, "ref_oeva_record"):
        pytest.skip("oracle/_ref not built (reference checkout absent)")
    rng = np.random.default_rng(2)
    na, cols, every = 10, 7, 3
    events = [0, 1, 2, 3, 5, 6, 9, 10, 12]
    preds = _cps(rng, len(events), na, cols)
    sizes = [na * cols] * len(events)
    sizes[5] = na * cols - 1                 # event 6: head not ready -> skipped
    ref_path = tmp_path / "ref.oeva"
    idx = (ctypes.c_ulonglong * len(events))(*events)
    body = np.concatenate([p.reshape(-1) for p in preds])
    sz = (ctypes.c_int * len(events))(*sizes)
    kept = L.ref_oeva_record(str(ref_path).encode(), na, cols, every, len(events), idx, fp(body), sz)
    assert kept == 4                          # events 0, 3, 9, 12
    rec = grid.OracleRecorder(na, cols, every, str(tmp_path / "ours.oeva"))
    for e, p, s in zip(events, preds, sizes):
        rec.record(e, p.reshape(-1)[:s])
    rec.save()
    assert (tmp_path / "ours.oeva").read_bytes() == ref_path.read_bytes()


def test_oeva_diff_matches_reference(tmp_path):
    L = O.load_ref()
    if L is None or not hasattr(L, "ref_oeva_diff"):
        pytest.skip("oracle/_ref not built (reference checkout absent)")
    rng = np.random.default_rng(3)
    base = _cps(rng, 4)
    a = tmp_path / "a.oeva"
    grid.write_dump(a, 12, 7, [0, 4, 8, 12], base)
    cases = {}
    cases["same"] = ([0, 4, 8, 12], base)
    pert = [p.copy() for p in base]
    pert[1][3, 2] += 5e-5
    pert[2][0, 0] -= 2e-3
    pert[3][11, 6] += 0.5
    cases["perturbed"] = ([0, 4, 8, 12], pert)
    nan = [p.copy() for p in base]
    nan[0][1, 1] = np.nan
    cases["nan"] = ([0, 4, 8, 12], nan)
    cases["index"] = ([0, 4, 9, 12], pert)
    cases["count"] = ([0, 4, 8], base[:3])
    cases["truncated"] = ([0, 4, 8, 12], base)
    for name, (idx, preds) in cases.items():
        b = tmp_path / f"{name}.oeva"
        grid.write_dump(b, 12, 7, idx, preds)
        if name == "truncated":
            b.write_bytes(b.read_bytes()[:-40])
        for tol in (1e-4, 1e-2):
            ours = grid.diff_dumps(a, b, tol)
            ref = (ctypes.c_double * 4)()
            assert L.ref_oeva_diff(str(a).encode(), str(b).encode(), tol, ref) == 0
            got = (float(ours.ok), float(ours.n_cp), ours.max_abs_delta,
                   float(ours.n_mismatched_cp))
            assert got == tuple(ref), (name, tol, got, tuple(ref))
    shape = tmp_path / "shape.oeva"
    grid.write_dump(shape, 6, 14, [0, 4, 8, 12], base)
    ours = grid.diff_dumps(a, shape)
    assert not ours.ok and ours.max_abs_delta == 0.0
    r = grid.diff_dumps(a, tmp_path / "perturbed.oeva", 1e-4)
    assert r.ok and r.n_mismatched_cp == 2
    assert r.max_abs_delta == pytest.approx(0.5, abs=1e-5)
