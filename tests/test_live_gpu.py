"""GPU parity of the in-kernel batch drain and the persistent live drain
(libssla_hip.so C ABI) against the fp64 oracle.

The batch drain takes records in batches of 1..32 inside one workgroup per
block; the reference's drain_n contract (8-record batches with a clock pair
per batch) is ssla_hip_drain_n with batch_clks.  The live drain polls rings
in fine-grained host memory; here the test itself is the producer (records
written, then their seq_done tags), so the check is deterministic: pass
flags (through the timing slots' owner flag), counters, hidden state, and
the prediction grid against the oracle.  Bars are those of
test_drain_gpu.py.
"""
import ctypes
import time

import numpy as np
import pytest

from oracle import oracle as O
from ssla_hip import abi, events

pytestmark = pytest.mark.gpu

FEAT_TOL = 1e-4
HEAD_TOL = 5e-5
HIDDEN_REL_TOL = 2e-5


def say(*a):
    print("[gpu-case]", *a, flush=True)


@pytest.fixture(scope="module")
def H():
    from ssla_hip import hybrid, lib
    lib.load()
    return hybrid


def hidden_close(a, b):
    return np.abs(a - b).max() <= HIDDEN_REL_TOL * max(1.0, float(np.abs(b).max()))


def oracle_run(npz, rec, head=True):
    st = O.S2S3(O.layers_from_npz(npz), 16, 20, 4, head=O.head_from_npz(npz) if head else None)
    p2, p3, feat, h7 = st.run(rec.x, rec.y, rec.feat1, want_head=head)
    return st, p2, p3, feat, h7


def check_preds(preds, version, rec, p3, ref7):
    m = p3 == 1
    c3 = (rec.y.astype(int) >> 1) * 10 + (rec.x >> 1)
    for cell in range(80):
        k = np.nonzero(m & (c3 == cell))[0]
        assert version[cell] == k.size, cell
        if k.size:
            assert np.abs(preds[cell] - ref7[k[-1]]).max() <= HEAD_TOL, cell


@pytest.mark.parametrize("batch", [1, 8, 17, 32])
def test_batch_mode_matches_oracle(H, stub_dir, stub_npz, batch):
    n = 6000
    say("batch_mode", batch, n)
    rec = events.blob_records(n, seed=11)
    with H.Drain.from_weights_dir(stub_dir) as d:
        (out,), (h7,) = d.drain([events.to_records(rec)], want_head=True, batch=batch)
        st, p2, p3, feat, ref7 = oracle_run(stub_npz, rec)
        assert np.array_equal(out["pass2"], p2.astype(np.int32))
        assert np.array_equal(out["pass3"], p3.astype(np.int32))
        m = p3 == 1
        df = np.abs(out["s3_feat"][m] - feat[m]).max()
        dh = np.abs(h7[m] - ref7[m]).max()
        say(f"batch {batch}: s3_feat max|d| {df:.3g}, head max|d| {dh:.3g}")
        assert df <= FEAT_TOL and dh <= HEAD_TOL
        for li in range(4):
            assert hidden_close(d.hidden(0, li), st.H[li]), li
        td2, td3 = d.counters(0)
        assert np.array_equal(td2, st.td2) and np.array_equal(td3, st.td3)
        check_preds(*d.preds(0), rec, p3, ref7)


def test_drain_n_with_batch_clocks(H, stub_dir, stub_npz):
    n = 3001                       # partial last batch
    say("drain_n batch_clks", n)
    rec = events.blob_records(n, seed=12)
    with H.Drain.from_weights_dir(stub_dir) as d:
        (out,), (clk,) = d.drain_with_clocks([events.to_records(rec)])
        _, p2, p3, feat, _ = oracle_run(stub_npz, rec, head=False)
        assert np.array_equal(out["pass2"], p2.astype(np.int32))
        assert np.array_equal(out["pass3"], p3.astype(np.int32))
        m = p3 == 1
        assert np.abs(out["s3_feat"][m] - feat[m]).max() <= FEAT_TOL
        assert clk.shape == ((n + 7) // 8, 2)
        assert np.all(clk[:, 1] >= clk[:, 0]) and np.all(clk[:, 0] > 0)
        assert np.all(np.diff(clk[:, 0].astype(np.int64)) >= 0)


def _produce(rings, blk, recs, timeout_s=30.0, chunk=97):
    """Publish records in chunks, never more than the ring holds ahead."""
    t0 = time.time()
    k = 0
    while k < recs.size:
        free = rings.capacity - int(rings.head[blk] - rings.tail[blk])
        if free >= chunk or recs.size - k <= free:
            m = min(chunk, recs.size - k, free)
            rings.push(blk, recs[k:k + m])
            k += m
        elif time.time() - t0 > timeout_s:
            raise TimeoutError("live drain stopped consuming")
        else:
            time.sleep(0.0002)


def _wait_done(rings, blk, n, timeout_s=30.0):
    t0 = time.time()
    while int(rings.tail[blk]) < n:
        if time.time() - t0 > timeout_s:
            raise TimeoutError(f"block {blk}: tail {int(rings.tail[blk])} of {n}")
        time.sleep(0.001)


def test_live_single_stream(H, stub_dir, stub_npz):
    n = 3000
    say("live single stream", n)
    rec = events.blob_records(n, seed=13)
    recs = events.to_records(rec)
    with H.Drain.from_weights_dir(stub_dir) as d:
        d.alloc_timing(4096)
        rings = H.HostRings(1, capacity=1024)
        live = H.LiveDrain(d, rings, idle_timeout_ms=15000)
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
        k0, k1 = d.kernel_clocks(0)
        assert 0 < k0 <= int(ts["t_pop_clk"].min()) and k1 >= int(ts["t_done_clk"].max())
        for li in range(4):
            assert hidden_close(d.hidden(0, li), st.H[li]), li
        td2, td3 = d.counters(0)
        assert np.array_equal(td2, st.td2) and np.array_equal(td3, st.td3)
        check_preds(*d.preds(0), rec, p3, ref7)
        from ssla_hip import lib
        khz = ctypes.c_int()
        lib.check(lib.load().ssla_hip_wall_clock_khz(ctypes.byref(khz)))
        lat_us = (ts["t_done_clk"] - ts["t_pop_clk"]).astype(np.float64) / khz.value * 1e3
        say(f"live: per-batch kernel time p50 {np.median(lat_us):.1f} us, max {lat_us.max():.1f} us")
        rings.free()


def test_live_preds_read_while_running(H, stub_dir, stub_npz):
    """The host reads the prediction grid between pushes while the live
    kernel writes it: every snapshot is whole (no cell stays busy), versions
    never go back, and the last snapshot matches the oracle."""
    n = 3000
    say("live preds read while running", n)
    rec = events.blob_records(n, seed=17)
    recs = events.to_records(rec)
    with H.Drain.from_weights_dir(stub_dir) as d:
        rings = H.HostRings(1, capacity=1024)
        live = H.LiveDrain(d, rings, idle_timeout_ms=15000)
        snaps = 0
        try:
            prev = np.zeros(80, np.uint32)
            for lo in range(0, n, 150):
                _produce(rings, 0, recs[lo:lo + 150])
                preds, version = d.preds(0)      # raises if a cell stays busy
                assert np.all(version >= prev)
                assert np.all(np.isfinite(preds[version > 0]))
                prev = version
                snaps += 1
            _wait_done(rings, 0, n)
        finally:
            status = live.stop()
        assert status == 0 and snaps == 20
        st, p2, p3, feat, ref7 = oracle_run(stub_npz, rec)
        check_preds(*d.preds(0), rec, p3, ref7)
        rings.free()


def test_live_four_streams(H, stub_dir, stub_npz):
    n = 1500
    say("live four streams", n)
    recs = [events.blob_records(n, seed=20 + b) for b in range(4)]
    with H.Drain.from_weights_dir(stub_dir, n_blocks=4) as d:
        rings = H.HostRings(4, capacity=512)
        live = H.LiveDrain(d, rings, idle_timeout_ms=15000)
        try:
            packed = [events.to_records(r) for r in recs]
            for k in range(0, n, 100):
                for b in range(4):
                    _produce(rings, b, packed[b][k:k + 100])
            for b in range(4):
                _wait_done(rings, b, n)
        finally:
            status = live.stop()
        assert status == 0
        for b in range(4):
            st, p2, p3, feat, ref7 = oracle_run(stub_npz, recs[b])
            for li in range(4):
                assert hidden_close(d.hidden(b, li), st.H[li]), (b, li)
            td2, td3 = d.counters(b)
            assert np.array_equal(td2, st.td2) and np.array_equal(td3, st.td3)
            check_preds(*d.preds(b), recs[b], p3, ref7)
        rings.free()


def test_live_two_ring_legacy_entry(H, stub_dir, stub_npz):
    """The legacy two-ring persistent entry (ssla_hip_persistent_start2, the
    signature of orin/kernels/ssla_s2_s3_head_celled.cuh:1271-1281): two
    rings fed in turns, each block's state, counters, timing slots and
    prediction grid equal the oracle run over its ring."""
    n = 1500
    say("live two-ring legacy entry", n)
    recs = [events.blob_records(n, seed=30 + b) for b in range(2)]
    with H.Drain.from_weights_dir(stub_dir, n_blocks=2) as d:
        d.alloc_timing(2048)
        rings = H.HostRings(2, capacity=512)
        live = H.LiveDrain(d, rings, idle_timeout_ms=15000, two_ring=True)
        try:
            packed = [events.to_records(r) for r in recs]
            for k in range(0, n, 100):
                for b in range(2):
                    _produce(rings, b, packed[b][k:k + 100])
            for b in range(2):
                _wait_done(rings, b, n)
        finally:
            status = live.stop()
        assert status == 0
        for b in range(2):
            assert int(rings.done[b]) == n
            st, p2, p3, feat, ref7 = oracle_run(stub_npz, recs[b])
            ts = d.timing(b)[:n]
            assert np.array_equal(ts["owner"], (p3 == 1).astype(np.uint32)), b
            for li in range(4):
                assert hidden_close(d.hidden(b, li), st.H[li]), (b, li)
            td2, td3 = d.counters(b)
            assert np.array_equal(td2, st.td2) and np.array_equal(td3, st.td3)
            check_preds(*d.preds(b), recs[b], p3, ref7)
        rings.free()


def test_live_two_ring_entry_rejects_other_block_counts(H, stub_dir):
    from ssla_hip import lib
    with H.Drain.from_weights_dir(stub_dir, n_blocks=1) as d:
        rings = H.HostRings(2, capacity=64)
        with pytest.raises(lib.SslaHipError):
            H.LiveDrain(d, rings, two_ring=True)
        rings.free()


def test_live_idle_timeout_exits(H, stub_dir):
    say("live idle timeout")
    with H.Drain.from_weights_dir(stub_dir) as d:
        rings = H.HostRings(1, capacity=64)
        live = H.LiveDrain(d, rings, idle_timeout_ms=300)
        status = live.wait(timeout_ms=20000)
        assert status == 3
        rings.free()


def test_live_fed_by_producer_matches_oracle(H, stub_dir, stub_npz):
    """Raw events -> host producer (one shard) -> fine-grained ring ->
    persistent kernel; the ring's records then drive the oracle, whose state,
    flags and predictions the kernel must match."""
    from ssla_hip import producer as P
    n_ev = 40000
    say("live fed by producer", n_ev)
    rng = np.random.default_rng(5)
    ev = P.events_array(np.arange(n_ev), rng.integers(0, 80, n_ev), rng.integers(0, 64, n_ev),
                        np.where(rng.random(n_ev) < 0.5, -1.0, 1.0))
    with H.Drain.from_weights_dir(stub_dir) as d:
        d.alloc_timing(1 << 14)
        rings = H.HostRings(1, capacity=1 << 14)
        api = P.S01gAPI()
        api.init(stub_dir, 1, 2, -1, 4096)
        live = None
        try:
            api.attach_multi([rings.bufs[0].ptr], rings.head_ptrs(), rings.capacity - 1, 20, 16,
                             [0], [20], [0], [16])
            live = H.LiveDrain(d, rings, idle_timeout_ms=20000)
            assert api.submit(ev) == n_ev
            st_p = api.wait_processed(n_ev, 0)
            n = int(rings.head[0])
            assert n == st_p[14] and 0 < n < rings.capacity
            _wait_done(rings, 0, n)
        finally:
            status = live.stop() if live is not None else -1
            api.shutdown()
        assert status == 0
        recs = rings.rings[0][:n].copy()
        assert np.array_equal(recs["seq_done"], np.arange(1, n + 1, dtype=np.uint64))
        rec = events.Records(recs["t"], recs["x"], recs["y"], recs["feat1"])
        st, p2, p3, feat, ref7 = oracle_run(stub_npz, rec)
        ts = d.timing(0)[:n]
        assert np.array_equal(ts["owner"], (p3 == 1).astype(np.uint32))
        assert np.all(ts["t_push_ns"] >= ts["t_emit_ns"]) and np.all(ts["t_emit_ns"] > 0)
        for li in range(4):
            assert hidden_close(d.hidden(0, li), st.H[li]), li
        td2, td3 = d.counters(0)
        assert np.array_equal(td2, st.td2) and np.array_equal(td3, st.td3)
        check_preds(*d.preds(0), rec, p3, ref7)
        rings.free()


def test_live_eight_blocks_fed_by_producer(H, stub_dir, stub_npz):
    """The reference's default live topology: 8 owned strips (2 x 4) with a
    2-cell halo, one ring and workgroup each, fed by two producer shards.
    Each ring's records (in ring order) drive an oracle with that block's
    ownership mask; state, flags and predictions must match per block."""
    from ssla_hip import producer as P
    from ssla_hip.topology import grid_topology
    n_ev = 40000
    say("live eight blocks fed by producer", n_ev)
    rng = np.random.default_rng(6)
    ev = P.events_array(np.arange(n_ev), rng.integers(0, 80, n_ev), rng.integers(0, 64, n_ev),
                        np.where(rng.random(n_ev) < 0.5, -1.0, 1.0))
    topo = grid_topology(8, 20, 16)
    with H.Drain.from_weights_dir(stub_dir, n_blocks=8, strips=[t.owned for t in topo]) as d:
        d.alloc_timing(1 << 14)
        rings = H.HostRings(8, capacity=1 << 14)
        api = P.S01gAPI()
        api.init(stub_dir, 2, 2, -1, 4096)
        live = None
        try:
            api.attach_multi([rings.bufs[b].ptr for b in range(8)], rings.head_ptrs(),
                             rings.capacity - 1, 20, 16,
                             [t.proc_x_lo for t in topo], [t.proc_x_hi for t in topo],
                             [t.proc_y_lo for t in topo], [t.proc_y_hi for t in topo])
            live = H.LiveDrain(d, rings, idle_timeout_ms=20000)
            assert api.submit(ev) == n_ev
            api.wait_processed(n_ev, 0)
            ns = [int(rings.head[b]) for b in range(8)]
            assert all(0 < n < rings.capacity for n in ns)
            for b in range(8):
                _wait_done(rings, b, ns[b])
        finally:
            status = live.stop() if live is not None else -1
            api.shutdown()
        assert status == 0
        head = O.head_from_npz(stub_npz)
        layers = O.layers_from_npz(stub_npz)
        for b, t in enumerate(topo):
            recs = rings.rings[b][:ns[b]].copy()
            assert np.array_equal(recs["seq_done"], np.arange(1, ns[b] + 1, dtype=np.uint64))
            x, y = recs["x"].astype(int), recs["y"].astype(int)
            assert np.all((x >= t.proc_x_lo) & (x < t.proc_x_hi) & (y >= t.proc_y_lo)
                          & (y < t.proc_y_hi))
            own = (x >= t.owned_x_lo) & (x < t.owned_x_hi) & (y >= t.owned_y_lo) & (y < t.owned_y_hi)
            st = O.S2S3(layers, 16, 20, 4, head=head)
            p2, p3, feat, ref7 = st.run(recs["x"], recs["y"], recs["feat1"], owner=own,
                                        want_head=True)
            ts = d.timing(b)[:ns[b]]
            assert np.array_equal(ts["owner"], (own & (p3 == 1)).astype(np.uint32)), b
            for li in range(4):
                assert hidden_close(d.hidden(b, li), st.H[li]), (b, li)
            td2, td3 = d.counters(b)
            assert np.array_equal(td2, st.td2) and np.array_equal(td3, st.td3), b
            # predictions: owned pass-3 records whose s3 cell is in the block's s3 box
            x3l, x3h, y3l, y3h = (t.owned_x_lo >> 1, t.owned_x_hi >> 1, t.owned_y_lo >> 1,
                                  t.owned_y_hi >> 1)
            w3 = x3h - x3l
            preds, version = d.preds(b)
            hit = own & (p3 == 1) & ((x >> 1) >= x3l) & ((x >> 1) < x3h) \
                & ((y >> 1) >= y3l) & ((y >> 1) < y3h)
            cell = ((y >> 1) - y3l) * w3 + ((x >> 1) - x3l)
            for c in range(version.size):
                k = np.nonzero(hit & (cell == c))[0]
                assert version[c] == k.size, (b, c)
                if k.size:
                    assert np.abs(preds[c] - ref7[k[-1]]).max() <= HEAD_TOL, (b, c)
        say("eight blocks: records per ring", ns)
        rings.free()


@pytest.mark.parametrize("group,stages", [(0, 1), (6, 2)])
def test_live_back_pressure_small_ring(H, stub_dir, stub_npz, group, stages):
    """A 128-slot ring and a burst of 40000 events: with back-pressure the
    producer waits for the kernel's tail instead of lapping it, so the
    kernel sees every record once, in order (no overrun exit), and its drop
    counters match the oracle's over the published positions.  Also with
    two pipelined groups, whose first stage frees ring slots while the
    second still works on earlier batches."""
    from ssla_hip import producer as P
    n_ev = 40000
    say("live back-pressure small ring", n_ev, "group", group, "stages", stages)
    rng = np.random.default_rng(9)
    ev = P.events_array(np.arange(n_ev), rng.integers(0, 80, n_ev), rng.integers(0, 64, n_ev),
                        np.where(rng.random(n_ev) < 0.5, -1.0, 1.0))
    with H.Drain.from_weights_dir(stub_dir) as d:
        d.alloc_timing(1 << 14)
        rings = H.HostRings(1, capacity=128)
        api = P.S01gAPI()
        api.init(stub_dir, 1, 2, -1, 1 << 16)
        live = None
        try:
            api.attach_multi([rings.bufs[0].ptr], rings.head_ptrs(), rings.capacity - 1, 20, 16,
                             [0], [20], [0], [16])
            api.set_ring_tails(rings.tail_ptrs(), timeout_ms=10000)
            live = H.LiveDrain(d, rings, idle_timeout_ms=20000, group=group, stages=stages)
            assert api.submit(ev) == n_ev
            st_p = api.wait_processed(n_ev, 0)
            n = int(rings.head[0])
            assert n == st_p[14] and n > 10 * rings.capacity
            _wait_done(rings, 0, n)
        finally:
            status = live.stop() if live is not None else -1
            api.shutdown()
        assert status == 0
        # one workgroup: the producer waits for the tail; two stages free
        # the slots as soon as the first stage holds a batch and the
        # producer may never wait -- either way no wait times out
        assert st_p[30] == 0 and (stages == 2 or st_p[28] > 0)
        say(f"back-pressure: {n} records, {int(st_p[28])} waits, "
            f"{st_p[29] / max(1, st_p[28]) / 1e3:.1f} us mean wait")
        ts = d.timing(0)[:n]
        assert np.array_equal(ts["seq"], np.arange(n, dtype=np.uint32))
        # the one shard publishes in event order: the oracle's stage 0+1
        # schedule gives the published positions
        sh = O.S01(O.layers_from_npz(stub_npz, first=0), 64, 80, 4)
        a0, a1, f1, x2, y2 = sh.run(ev, precision=32)
        m = a1 == 1
        assert m.sum() == n
        st = O.S2S3(O.layers_from_npz(stub_npz), 16, 20, 4)
        st.run(x2[m], y2[m], f1[m])
        td2, td3 = d.counters(0)
        assert np.array_equal(td2, st.td2) and np.array_equal(td3, st.td3)
        rings.free()


def test_run_live_short(stub_dir):
    """The live pipeline end to end at a low rate: nothing lost, latencies
    measured for output-producing records."""
    from ssla_hip import live as LV
    say("run_live 0.2 Mev/s 1 s")
    r = LV.run_live(stub_dir, rate_mev=0.2, duration_s=1.0, n_shards=2, halo=2,
                    timing_capacity=1 << 16)
    say(f"run_live: status {r.status} ring {r.ring_records} drained {r.drained} "
        f"out {r.output_records} lat {r.lat_us}")
    assert r.status == 0
    assert r.drained == r.ring_records > 0 and r.output_records > 0
    assert 0 < r.lat_us["emit_to_push_p50"] <= r.lat_us["emit_to_done_p50"]
    assert r.lat_us["kernel_p50"] > 0


def test_run_live_sixteen_blocks(stub_dir):
    """The 4 x 4 strip topology (16 rings, 16 workgroups of one persistent
    kernel) fed by the host producer: every published record (halo copies
    included) is drained and output-producing records carry latencies."""
    from ssla_hip import live as LV
    say("run_live 0.5 Mev/s 1 s, 16 blocks")
    r = LV.run_live(stub_dir, rate_mev=0.5, duration_s=1.0, n_shards=2, halo=2,
                    timing_capacity=1 << 16, gpu_blocks=16)
    say(f"run_live 16: status {r.status} ring {r.ring_records} drained {r.drained} "
        f"out {r.output_records}")
    assert r.status == 0 and r.gpu_blocks == 16
    assert r.drained == r.ring_records > 0 and r.output_records > 0
    assert r.lat_us["kernel_p50"] > 0


def test_replay_four_streams_live(stub_dir, stub_npz):
    """Four streams replayed into four rings of one persistent kernel: every
    record drained, drop drift 0 per stream against the oracle's schedule."""
    from ssla_hip import live as LV
    n = 3000
    say("replay four streams", n)
    recs = [events.blob_records(n, seed=40 + s) for s in range(4)]
    expect = [O.decisions(r.x, r.y, 16, 20, 4)[1] for r in recs]
    res = LV.run_replay(stub_dir, [events.to_records(r) for r in recs], 50_000.0,
                        ring_capacity=1 << 12, timing_capacity=1 << 12, expect_p3=expect)
    say("replay:", res.status, [(s["drained"], s["drop_drift"], round(s["push_to_done_p50"], 1))
                                for s in res.streams])
    assert res.status == 0
    for s in res.streams:
        assert s["drained"] == n and s["drop_drift"] == 0
        assert s["output_records"] > 0 and 0 < s["push_to_done_p50"] < 1e5


def _oracle_rings(stub_npz, jobs, H2=16, W2=20):
    """Runs the fp64 oracle (with head) over several rings at once, one
    thread each (the C oracle keeps no global state and ctypes releases the
    GIL).  jobs: (x, y, feat1, owner-or-None); returns (state, p2, p3, ref7)."""
    from concurrent.futures import ThreadPoolExecutor
    layers, head = O.layers_from_npz(stub_npz), O.head_from_npz(stub_npz)

    def one(job):
        x, y, f, own = job
        st = O.S2S3(layers, H2, W2, 4, head=head)
        p2, p3, _, ref7 = st.run(x, y, f, owner=own, want_head=True)
        return st, p2, p3, ref7

    with ThreadPoolExecutor(max_workers=min(16, len(jobs))) as ex:
        return list(ex.map(one, jobs))


def _check_block_preds(preds, version, x, y, own, p3, ref7, owned):
    """Prediction cells of a block's owned s3 box: version = owned pass-3
    records of the cell, values = the last one's head outputs."""
    x3l, x3h, y3l, y3h = owned[0] >> 1, owned[1] >> 1, owned[2] >> 1, owned[3] >> 1
    w3 = x3h - x3l
    hit = own & (p3 == 1) & ((x >> 1) >= x3l) & ((x >> 1) < x3h) & ((y >> 1) >= y3l) \
        & ((y >> 1) < y3h)
    cell = ((y >> 1) - y3l) * w3 + ((x >> 1) - x3l)
    for c in range(version.size):
        k = np.nonzero(hit & (cell == c))[0]
        assert version[c] == k.size, c
        if k.size:
            assert np.abs(preds[c] - ref7[k[-1]]).max() <= HEAD_TOL, c


@pytest.mark.parametrize("gpu_blocks,group,stages",
                         [(1, 0, 1), (8, 0, 1), (1, 6, 1), (8, 6, 1), (1, 6, 2), (8, 6, 2)])
def test_config2_live_two_mev_six_shards(stub_dir, stub_npz, gpu_blocks, group, stages):
    """The live configuration: the producer's paced blob source at
    2.0 Mev/s -> 6 host shards for stages 0 + 1 (halo 2) -> fine-grained
    rings -> the persistent kernel, 2 s per parametrisation
    (orin/hybrid_runner_multi.py:314-754).
    One ownership domain (1 block) and the reference's 8-strip topology,
    one workgroup per block; one domain drained by a group of 6 workgroups
    (channel slices, exact: no halo); the 8 strips drained by a group of 6
    each (48 workgroups); and both with two pipelined groups per block
    (stages 2: 12 and 96 workgroups).
    Every published record is drained with no overrun, and each ring's
    contents, run through the oracle with that block's ownership, give the
    kernel's pass flags (timing-slot owner flags), tdrop counters, final
    hidden state and prediction grid."""
    _config2(stub_dir, stub_npz, gpu_blocks, group, stages, 2.0,
             1 << 19 if gpu_blocks == 1 else 1 << 18)


def test_config2_headline_eight_seconds(stub_dir, stub_npz):
    """Config 2's headline run as stated: one ownership domain drained by
    two pipelined groups of 6 workgroups, 2.0 Mev/s for 8 s (about 1M ring
    records), every ring record checked against the oracle as above."""
    _config2(stub_dir, stub_npz, 1, 6, 2, 8.0, 1 << 21)


def _config2(stub_dir, stub_npz, gpu_blocks, group, stages, duration, cap):
    from ssla_hip import live as LV
    say(f"config 2: 2.0 Mev/s, 6 shards, halo 2, {duration:g} s, {gpu_blocks} GPU block(s), "
        f"group {group}, stages {stages}")
    seen = {}

    def inspect(drain, rings, heads, topo):
        jobs, meta = [], []
        for b, t in enumerate(topo):
            n = heads[b]
            assert 0 < n <= rings.capacity, (b, n)
            assert int(rings.done[b]) == n, b
            recs = rings.rings[b][:n].copy()
            assert np.array_equal(recs["seq_done"], np.arange(1, n + 1, dtype=np.uint64)), b
            x, y = recs["x"].astype(int), recs["y"].astype(int)
            own = (x >= t.owned_x_lo) & (x < t.owned_x_hi) & (y >= t.owned_y_lo) \
                & (y < t.owned_y_hi)
            jobs.append((recs["x"], recs["y"], recs["feat1"], own))
            meta.append((b, t, x, y, own, drain.timing(b)[:n],
                         [drain.hidden(b, li) for li in range(4)], drain.counters(b),
                         drain.preds(b)))
        say(f"config 2: records per ring {heads}; running the oracle")
        for (st, p2, p3, ref7), (b, t, x, y, own, ts, hid, (td2, td3), (pr, ver)) in zip(
                _oracle_rings(stub_npz, jobs), meta):
            assert np.array_equal(ts["owner"], (own & (p3 == 1)).astype(np.uint32)), b
            for li in range(4):
                assert hidden_close(hid[li], st.H[li]), (b, li)
            assert np.array_equal(td2, st.td2) and np.array_equal(td3, st.td3), b
            _check_block_preds(pr, ver, x, y, own, p3, ref7, t.owned)
        seen["blocks"] = len(topo)

    r = LV.run_live(stub_dir, rate_mev=2.0, duration_s=duration, n_shards=6, halo=2,
                    gpu_blocks=gpu_blocks, ring_capacity=cap, timing_capacity=cap,
                    group=group, stages=stages, inspect=inspect)
    say(f"config 2: status {r.status}, {r.synth_events} events "
        f"({r.synth_events / r.duration_s / 1e6:.2f} Mev/s achieved), {r.ring_records} ring records, "
        f"{r.drained} drained, {r.output_records} output-producing, "
        f"emit->prediction p50 {r.lat_us['emit_to_done_p50']:.1f} us "
        f"p99 {r.lat_us['emit_to_done_p99']:.1f} us")
    assert r.status == 0 and seen.get("blocks") == gpu_blocks
    assert r.drained == r.ring_records > 0 and r.output_records > 0
    # the paced source asks for 2 Mev/s; the run must reach at least 1.8
    assert r.synth_events >= 1.8e6 * r.duration_s, r.synth_events / r.duration_s


@pytest.mark.parametrize("group,stages", [(0, 1), (6, 1), (6, 2)])
def test_config4_sixteen_rings_one_persistent_kernel(stub_dir, stub_npz, group, stages):
    """Config 4: 16 independent 80x64 instances sharing the stub weights in
    one persistent kernel (...celled.cuh:82 MAX_BLOCKS = 16, :1547), each fed
    its own seeded blob stream (seeds 1..16) through its own ring at 125k
    records/s (2.0 Mev/s raw / 16).  Per stream: every record drained, drop
    drift 0, tdrop counters, final hidden state and prediction grid equal to
    the oracle's."""
    from ssla_hip import live as LV
    n = 40_000
    say(f"config 4: 16 rings x {n} records at 125k records/s each, group {group}, "
        f"stages {stages}")
    recs = [events.blob_records(n, seed=1 + s) for s in range(16)]
    expect = [O.decisions(r.x, r.y, 16, 20, 4)[1] for r in recs]
    state = {}

    def inspect(drain):
        for b in range(16):
            state[b] = ([drain.hidden(b, li) for li in range(4)], drain.counters(b),
                        drain.preds(b))

    res = LV.run_replay(stub_dir, [events.to_records(r) for r in recs], 125_000.0,
                        ring_capacity=1 << 16, timing_capacity=1 << 16, expect_p3=expect,
                        group=group, stages=stages, inspect=inspect)
    say("config 4: status", res.status, "per stream (drained, drift, p50 us, p99 us):",
        [(s["drained"], s["drop_drift"], round(s["push_to_done_p50"], 1),
          round(s["push_to_done_p99"], 1)) for s in res.streams])
    assert res.status == 0 and len(state) == 16
    for s in res.streams:
        assert s["drained"] == n and s["drop_drift"] == 0
    got = _oracle_rings(stub_npz, [(r.x, r.y, r.feat1, None) for r in recs])
    for b, (st, p2, p3, ref7) in enumerate(got):
        hid, (td2, td3), (pr, ver) = state[b]
        assert np.array_equal(p3, expect[b])
        for li in range(4):
            assert hidden_close(hid[li], st.H[li]), (b, li)
        assert np.array_equal(td2, st.td2) and np.array_equal(td3, st.td3), b
        check_preds(pr, ver, recs[b], p3, ref7)


@pytest.mark.parametrize("stages", [1, 2])
def test_640x480_strips_live_group(stub_640, stages):
    """The 640x480 stream live in the reference's multi-block form: the
    full-resolution records split into 16 owned strips (4 x 4, halo 2), each
    strip's processed-window records (halo copies included) replayed by
    record time into its own ring of one persistent kernel, each ring
    drained by a group of 6 workgroups (96 workgroups).  Per strip, against
    the fp64 oracle run on that ring with the strip's ownership: every record
    drained, owner flags (drop drift 0), tdrop counters, final hidden state
    and the owned box's prediction cells."""
    from ssla_hip import live as LV
    from ssla_hip.topology import grid_topology
    n = 40_000
    say(f"640x480 live: {n} edge-blob records over 16 strips, group 6, stages {stages}")
    npz = O.load_npz(stub_640)
    rec = events.edge_blob_records(n, seed=3)
    full = events.to_records(rec)
    x, y = rec.x.astype(np.int64), rec.y.astype(np.int64)
    topo = grid_topology(16, 160, 120)
    rings, jobs = [], []
    for t in topo:
        m = (x >= t.proc_x_lo) & (x < t.proc_x_hi) & (y >= t.proc_y_lo) & (y < t.proc_y_hi)
        rings.append(full[m])
        xs, ys = x[m], y[m]
        own = (xs >= t.owned_x_lo) & (xs < t.owned_x_hi) & (ys >= t.owned_y_lo) \
            & (ys < t.owned_y_hi)
        jobs.append((rec.x[m], rec.y[m], rec.feat1[m], own))
    got = _oracle_rings(npz, jobs, H2=120, W2=160)
    expect = [(j[3] & (g[2] == 1)).astype(np.int8) for j, g in zip(jobs, got)]
    state = {}

    def inspect(drain):
        for b in range(len(topo)):
            state[b] = ([drain.hidden(b, li) for li in range(4)], drain.counters(b),
                        drain.preds(b))

    res = LV.run_replay(stub_640, rings, 0.0, strips=[t.owned for t in topo], speed=1.0,
                        ring_capacity=1 << 14, timing_capacity=1 << 14, expect_p3=expect,
                        group=6, stages=stages, inspect=inspect)
    say("640x480 live: status", res.status, "per strip (drained, drift, p50 us):",
        [(s["drained"], s["drop_drift"], round(s["push_to_done_p50"], 1)) for s in res.streams])
    assert res.status == 0 and len(state) == len(topo)
    for b, (s, r, (st, p2, p3, ref7), (xs, ys, _, own)) in enumerate(
            zip(res.streams, rings, got, jobs)):
        assert s["drained"] == r.size and s["drop_drift"] == 0, b
        hid, (td2, td3), (pr, ver) = state[b]
        for li in range(4):
            assert hidden_close(hid[li], st.H[li]), (b, li)
        assert np.array_equal(td2, st.td2) and np.array_equal(td3, st.td3), b
        _check_block_preds(pr, ver, xs.astype(int), ys.astype(int), own, p3, ref7,
                           topo[b].owned)
