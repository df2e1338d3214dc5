"""GPU parity of the group drains: G workgroups per block, each owning
16-channel slices of every layer and exchanging partial pre-LayerNorm sums
(libssla_hip.so C ABI, SslaHipDrainOpts.group / SslaHipLiveOpts.group),
against the fp64 oracle, with the bars of test_live_gpu.py.

The batch mode gives per-record outputs (pass flags, s3_feat, head rows);
the live mode is checked like the one-workgroup live drain (timing-slot
owner flags, counters, hidden state, prediction grid).
"""
import ctypes

import numpy as np
import pytest

from oracle import oracle as O
from ssla_hip import abi, events, lib
from test_live_gpu import (FEAT_TOL, HEAD_TOL, _produce, _wait_done, check_preds, hidden_close,
                           oracle_run, say)

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def H():
    from ssla_hip import hybrid, lib
    lib.load()
    return hybrid


@pytest.mark.parametrize("group,batch", [(6, 32), (6, 1), (6, 8), (3, 32), (4, 17), (5, 32)])
def test_group_batch_matches_oracle(H, stub_dir, stub_npz, group, batch):
    n = 6000 if batch > 1 else 1500
    say("group batch drain", group, batch, n)
    rec = events.blob_records(n, seed=11)
    with H.Drain.from_weights_dir(stub_dir) as d:
        (out,), (h7,) = d.drain([events.to_records(rec)], want_head=True, batch=batch, group=group)
        st, p2, p3, feat, ref7 = oracle_run(stub_npz, rec)
        assert np.array_equal(out["pass2"], p2.astype(np.int32))
        assert np.array_equal(out["pass3"], p3.astype(np.int32))
        m = p3 == 1
        df = np.abs(out["s3_feat"][m] - feat[m]).max()
        dh = np.abs(h7[m] - ref7[m]).max()
        say(f"group {group} batch {batch}: s3_feat max|d| {df:.3g}, head max|d| {dh:.3g}")
        assert df <= FEAT_TOL and dh <= HEAD_TOL
        for li in range(4):
            assert hidden_close(d.hidden(0, li), st.H[li]), li
        td2, td3 = d.counters(0)
        assert np.array_equal(td2, st.td2) and np.array_equal(td3, st.td3)
        check_preds(*d.preds(0), rec, p3, ref7)


def test_group_batch_continues_state(H, stub_dir, stub_npz):
    """Two calls in a row continue one state (the counter copies of members
    1..G-1 are taken from the block's counters at each call)."""
    rec = events.blob_records(4000, seed=21)
    say("group batch drain, two calls")
    with H.Drain.from_weights_dir(stub_dir) as d:
        recs = events.to_records(rec)
        (o1,), _ = d.drain([recs[:2500]], batch=32, group=6)
        (o2,), _ = d.drain([recs[2500:]], batch=32, group=6)
        st, p2, p3, feat, _ = oracle_run(stub_npz, rec, head=False)
        assert np.array_equal(np.concatenate([o1["pass2"], o2["pass2"]]), p2.astype(np.int32))
        assert np.array_equal(np.concatenate([o1["pass3"], o2["pass3"]]), p3.astype(np.int32))
        for li in range(4):
            assert hidden_close(d.hidden(0, li), st.H[li]), li
        td2, td3 = d.counters(0)
        assert np.array_equal(td2, st.td2) and np.array_equal(td3, st.td3)


def test_group_batch_repeated_calls(H, stub_dir, stub_npz):
    """Three group batch drains in a row, each on the resources the first
    one sized (they are kept per device), continue one state: the
    concatenated outputs equal the oracle run on all records."""
    rec = events.blob_records(3000, seed=23)
    recs = events.to_records(rec)
    with H.Drain.from_weights_dir(stub_dir) as d:
        outs = []
        for lo in (0, 1000, 2000):
            d.load_rings([recs[lo:lo + 1000]])
            # a device-wide sync before each call marks the call boundaries
            # in a HIP API trace of this test
            lib.check(lib.load().ssla_hip_device_synchronize())
            d.run(batch=32, group=6)
            outs.append(d.results()[0][0])
        st, p2, p3, feat, _ = oracle_run(stub_npz, rec, head=False)
        o = np.concatenate(outs)
        assert np.array_equal(o["pass2"], p2.astype(np.int32))
        assert np.array_equal(o["pass3"], p3.astype(np.int32))
        for li in range(4):
            assert hidden_close(d.hidden(0, li), st.H[li]), li


@pytest.mark.parametrize("group", [0, 6])
def test_batch_head_with_full_batches(H, stub_w1_dir, group):
    """Tdrop window 1: every record passes both gates and is owned, so the
    head runs on every record of each 32-record batch (two 16-record row
    tiles of the head's MFMA items) -- raw head rows, s3_feat, flags, state
    and prediction grid against the oracle."""
    rec = events.blob_records(2000, seed=27)
    npz = O.load_npz(stub_w1_dir)
    say(f"batch head with full batches, group {group}")
    with H.Drain.from_weights_dir(stub_w1_dir) as d:
        (out,), (h7,) = d.drain([events.to_records(rec)], want_head=True, batch=32, group=group)
        st = O.S2S3(O.layers_from_npz(npz), 16, 20, 1, head=O.head_from_npz(npz))
        p2, p3, feat, ref7 = st.run(rec.x, rec.y, rec.feat1, want_head=True)
        assert np.all(p3 == 1)
        assert np.array_equal(out["pass2"], p2.astype(np.int32))
        assert np.array_equal(out["pass3"], p3.astype(np.int32))
        df = np.abs(out["s3_feat"] - feat).max()
        dh = np.abs(h7 - ref7).max()
        say(f"group {group}: s3_feat max|d| {df:.3g}, head max|d| {dh:.3g}")
        assert df <= FEAT_TOL and dh <= HEAD_TOL
        for li in range(4):
            assert hidden_close(d.hidden(0, li), st.H[li]), li
        check_preds(*d.preds(0), rec, p3, ref7)


def test_group_bad_sizes(H, stub_dir):
    rec = events.to_records(events.blob_records(64, seed=3))
    with H.Drain.from_weights_dir(stub_dir) as d:
        d.load_rings([rec])
        for g in (2, 7):
            with pytest.raises(lib.SslaHipError):
                d.run(batch=8, group=g)
        with pytest.raises(lib.SslaHipError):
            d.run(batch=0, group=6)          # the whole-ring drain has no groups


@pytest.mark.parametrize("group,stages", [(6, 1), (3, 1), (6, 2), (3, 2)])
def test_live_group_single_stream(H, stub_dir, stub_npz, group, stages):
    """One stream drained by a group (stages 1) or by two groups in a
    pipeline (stages 2: L4-L5 of a batch beside L6-head of the previous
    one, the batch handed over through device memory)."""
    n = 3000
    say("live group single stream", group, stages, n)
    rec = events.blob_records(n, seed=13)
    recs = events.to_records(rec)
    with H.Drain.from_weights_dir(stub_dir) as d:
        d.alloc_timing(4096)
        rings = H.HostRings(1, capacity=1024)
        live = H.LiveDrain(d, rings, idle_timeout_ms=15000, group=group, stages=stages,
                           profile=True)
        try:
            _produce(rings, 0, recs)
            _wait_done(rings, 0, n)
        finally:
            status = live.stop()
        assert status == 0
        assert int(rings.done[0]) == n
        st, p2, p3, feat, ref7 = oracle_run(stub_npz, rec)
        ts = d.timing(0)[:n]
        assert np.array_equal(ts["seq"], np.arange(n, dtype=np.uint32))
        assert np.array_equal(ts["owner"], (p3 == 1).astype(np.uint32))
        assert np.all(ts["t_done_clk"] >= ts["t_pop_clk"])
        for li in range(4):
            assert hidden_close(d.hidden(0, li), st.H[li]), li
        td2, td3 = d.counters(0)
        assert np.array_equal(td2, st.td2) and np.array_equal(td3, st.td3)
        check_preds(*d.preds(0), rec, p3, ref7)
        khz = ctypes.c_int()
        lib.check(lib.load().ssla_hip_wall_clock_khz(ctypes.byref(khz)))
        lat_us = (ts["t_done_clk"] - ts["t_pop_clk"]).astype(np.float64) / khz.value * 1e3
        ph = live.phase_us
        nbat = max(1.0, ph[abi.BATCH_PHASES.index("batches")])
        per = {k: round(ph[i] / nbat, 2) for i, k in enumerate(abi.BATCH_PHASES)
               if k not in ("batches", "records")}
        say(f"live group {group} x {stages}: per-batch kernel time p50 {np.median(lat_us):.1f} us, "
            f"max {lat_us.max():.1f} us; {nbat:.0f} batches of "
            f"{ph[abi.BATCH_PHASES.index('records')] / nbat:.1f} records; per batch (us) {per}")
        rings.free()


@pytest.mark.parametrize("group,stages", [(0, 1), (6, 1), (6, 2)])
def test_live_off_grid_records(H, stub_dir, stub_npz, group, stages):
    """Records outside the s2 grid in the live drains, including the two-
    stage hand-off: x = W2, x = 4095, y = 4096 and 0xFFFF (whose bits would
    reach the hand-off's flag bits if the coordinates were not masked).  They
    change no state and produce nothing; the rest equals the oracle, which
    skips such records."""
    n = 3000
    say("live off-grid records", group, stages, n)
    rec = events.blob_records(n, seed=17)
    bad = [(20, 3), (4095, 10), (5, 4096), (5, 0xFFFF), (0xFFFF, 0xFFFF), (19, 16)]
    idx = np.arange(11, n, 37)
    for k, i in enumerate(idx):
        rec.x[i], rec.y[i] = bad[k % len(bad)]
    recs = events.to_records(rec)
    with H.Drain.from_weights_dir(stub_dir) as d:
        d.alloc_timing(4096)
        rings = H.HostRings(1, capacity=1024)
        live = H.LiveDrain(d, rings, idle_timeout_ms=15000, group=group, stages=stages)
        try:
            _produce(rings, 0, recs)
            _wait_done(rings, 0, n)
        finally:
            status = live.stop()
        assert status == 0 and int(rings.done[0]) == n
        st, p2, p3, feat, ref7 = oracle_run(stub_npz, rec)
        assert np.all(p2[idx] == -2)
        ts = d.timing(0)[:n]
        assert np.array_equal(ts["owner"], (p3 == 1).astype(np.uint32))
        for li in range(4):
            assert hidden_close(d.hidden(0, li), st.H[li]), li
        td2, td3 = d.counters(0)
        assert np.array_equal(td2, st.td2) and np.array_equal(td3, st.td3)
        check_preds(*d.preds(0), rec, p3, ref7)
        say(f"off-grid: {idx.size} records outside the grid, group {group} stages {stages}: "
            "state and predictions match")
        rings.free()


@pytest.mark.parametrize("group", [0, 6])
def test_clock_handshake(H, stub_dir, group):
    """The live kernels answer the host's clock ping with their wall clock:
    two handshakes 0.2 s apart give the 100 MHz constant-rate clock to
    better than 0.1 %, each bracketed by the host within 1 ms."""
    import time
    from ssla_hip import live as LV
    khz = ctypes.c_int()
    lib.check(lib.load().ssla_hip_wall_clock_khz(ctypes.byref(khz)))
    with H.Drain.from_weights_dir(stub_dir) as d:
        d.alloc_timing(1024)
        rings = H.HostRings(1, capacity=256)
        live = H.LiveDrain(d, rings, idle_timeout_ms=10000, group=group)
        try:
            p0 = LV.clock_pair(d, 0)
            time.sleep(0.2)
            p1 = LV.clock_pair(d, 0)
        finally:
            status = live.stop()
        assert status == 0 and p0 is not None and p1 is not None
        assert p0[2] < 1e6 and p1[2] < 1e6
        ns_per_tick = (p1[0] - p0[0]) / (p1[1] - p0[1])
        say(f"clock handshake group {group}: {ns_per_tick:.5f} ns/tick, brackets {p0[2]}, {p1[2]} ns")
        assert abs(ns_per_tick * khz.value / 1e6 - 1.0) < 1e-3
        rings.free()


def test_two_stages_bad_sizes(H, stub_dir):
    """Two stages need a group, and n_blocks x group x 2 workgroups on the
    device at once."""
    with H.Drain.from_weights_dir(stub_dir) as d:
        rings = H.HostRings(1, capacity=256)
        for g, st in ((0, 2), (6, 3)):
            with pytest.raises(lib.SslaHipError):
                H.LiveDrain(d, rings, idle_timeout_ms=2000, group=g, stages=st)
        rings.free()
