"""GPU parity of the single-linear head (cfg.head_W / head_b, used when
head_cls_conv_W is not set: orin/kernels/ssla_s2_s3_head_celled.cuh:
1462-1500, 1715-1751) in every drain form -- whole ring, in-kernel batches,
group batches, the persistent live kernel with one workgroup, a group of 6
and two pipelined groups of 6 -- and the live runner's fallback for weight
directories without head keys (orin/hybrid_runner_multi.py:395-423).

Against the fp64 oracle with the same head (oracle.Head.linear): raw head
rows of owned pass-3 records within HEAD_TOL, zeros elsewhere; the
prediction grid holds the last pass-3 record's row per s3 cell and a version
equal to the cell's pass-3 count; flags, counters and hidden state as in
test_live_gpu.py.
"""
import numpy as np
import pytest

from oracle import oracle as O
from ssla_hip import events, lib
from test_live_gpu import (FEAT_TOL, HEAD_TOL, _produce, _wait_done, check_preds, hidden_close,
                           say)

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def H():
    from ssla_hip import hybrid
    lib.load()
    return hybrid


def linear_weights(H, seed=5):
    return H.build_head_weights(np.random.default_rng(seed))


def oracle_linear(npz, rec, W, b):
    st = O.S2S3(O.layers_from_npz(npz), 16, 20, 4, head=O.Head.linear(W, b))
    p2, p3, feat, h7 = st.run(rec.x, rec.y, rec.feat1, want_head=True)
    return st, p2, p3, feat, h7


def check_drain(d, out, h7, st, p2, p3, feat, ref7, rec, tag):
    assert np.array_equal(out["pass2"], p2.astype(np.int32)), tag
    assert np.array_equal(out["pass3"], p3.astype(np.int32)), tag
    m = p3 == 1
    df = np.abs(out["s3_feat"][m] - feat[m]).max()
    dh = np.abs(h7[m] - ref7[m]).max()
    say(f"{tag}: {int(m.sum())} pass-3 records, s3_feat max|d| {df:.3g}, "
        f"linear head max|d| {dh:.3g}")
    assert df <= FEAT_TOL and dh <= HEAD_TOL
    assert np.all(h7[~m] == 0)
    for li in range(4):
        assert hidden_close(d.hidden(0, li), st.H[li]), (tag, li)
    td2, td3 = d.counters(0)
    assert np.array_equal(td2, st.td2) and np.array_equal(td3, st.td3), tag
    check_preds(*d.preds(0), rec, p3, ref7)


@pytest.mark.parametrize("batch,group", [(0, 0), (8, 0), (32, 0), (32, 6), (17, 3)])
def test_linear_head_drains(H, headless_dir, stub_npz, batch, group):
    """Whole-ring drain (batch 0), batches of 8 and 32 in one workgroup,
    group batches (6 and 3 workgroups per block)."""
    n = 20_000 if batch == 0 else 6000
    say("linear head drain", n, "batch", batch, "group", group)
    rec = events.blob_records(n, seed=31)
    W, b = linear_weights(H)
    with H.Drain.from_weights_dir(headless_dir, linear_head=(W, b)) as d:
        assert d.cfg.head_W and d.cfg.head_b and not d.cfg.head_cls_conv_W
        assert np.array_equal(d.zero_row(), b)
        (out,), (h7,) = d.drain([events.to_records(rec)], want_head=True, batch=batch,
                                group=group)
        st, p2, p3, feat, ref7 = oracle_linear(stub_npz, rec, W, b)
        check_drain(d, out, h7, st, p2, p3, feat, ref7, rec, f"batch {batch} group {group}")


def test_linear_head_replaces_two_branch_head(H, stub_dir, stub_npz):
    """bind_linear_head on a model that has the two-branch head: the
    configuration then carries only head_W / head_b, and the drain computes
    the single-linear head."""
    n = 6000
    rec = events.blob_records(n, seed=32)
    W, b = linear_weights(H, seed=6)
    with H.Drain.from_weights_dir(stub_dir) as d:
        assert d.cfg.head_cls_conv_W
        d.bind_linear_head(W, b)
        assert not d.cfg.head_cls_conv_W and d.cfg.head_W
        (out,), (h7,) = d.drain([events.to_records(rec)], want_head=True)
        st, p2, p3, feat, ref7 = oracle_linear(stub_npz, rec, W, b)
        check_drain(d, out, h7, st, p2, p3, feat, ref7, rec, "rebound head")


def test_linear_head_without_bias_is_refused(H, headless_dir):
    rec = events.to_records(events.blob_records(64, seed=3))
    W, b = linear_weights(H)
    with H.Drain.from_weights_dir(headless_dir, linear_head=(W, b)) as d:
        d.cfg.head_b = None
        d.load_rings([rec])
        for batch in (0, 8):
            with pytest.raises(lib.SslaHipError, match="head_b"):
                d.run(batch=batch)


@pytest.mark.parametrize("group,stages", [(0, 1), (6, 1), (6, 2)])
def test_linear_head_live(H, headless_dir, stub_npz, group, stages):
    """The persistent kernel with the single-linear head (the test is the
    producer): timing-slot owner flags, counters, hidden state and the
    prediction grid against the oracle."""
    n = 3000
    say("linear head live", n, "group", group, "stages", stages)
    rec = events.blob_records(n, seed=33)
    recs = events.to_records(rec)
    W, b = linear_weights(H, seed=7)
    with H.Drain.from_weights_dir(headless_dir, linear_head=(W, b)) as d:
        d.alloc_timing(4096)
        rings = H.HostRings(1, capacity=1024)
        live = H.LiveDrain(d, rings, idle_timeout_ms=15000, group=group, stages=stages)
        try:
            _produce(rings, 0, recs)
            _wait_done(rings, 0, n)
        finally:
            status = live.stop()
        assert status == 0 and int(rings.done[0]) == n
        st, p2, p3, feat, ref7 = oracle_linear(stub_npz, rec, W, b)
        ts = d.timing(0)[:n]
        assert np.array_equal(ts["owner"], (p3 == 1).astype(np.uint32))
        for li in range(4):
            assert hidden_close(d.hidden(0, li), st.H[li]), li
        td2, td3 = d.counters(0)
        assert np.array_equal(td2, st.td2) and np.array_equal(td3, st.td3)
        check_preds(*d.preds(0), rec, p3, ref7)
        say(f"linear head live group {group} stages {stages}: {int((p3 == 1).sum())} "
            "prediction writes match")
        rings.free()


def test_run_live_headless_dir_uses_linear_head(H, headless_dir, stub_npz):
    """The live runner on a directory without head keys: the producer's
    paced blob source at 2.0 Mev/s -> 6 shards -> one ring -> two pipelined
    groups of 6; the prediction grid comes from the random single-linear head
    drawn from the run's seed, as the reference's runner does."""
    from ssla_hip import live as LV
    seed = 3
    W, b = linear_weights(H, seed=seed)
    seen = {}

    def inspect(drain, rings, heads, topo):
        n = heads[0]
        assert np.array_equal(drain.linear_head[0], W) and np.array_equal(drain.linear_head[1], b)
        recs = rings.rings[0][:n].copy()
        st = O.S2S3(O.layers_from_npz(stub_npz), 16, 20, 4, head=O.Head.linear(W, b))
        p2, p3, _, ref7 = st.run(recs["x"], recs["y"], recs["feat1"], want_head=True)
        assert np.array_equal(drain.timing(0)[:n]["owner"], (p3 == 1).astype(np.uint32))
        pr, ver = drain.preds(0)
        m = p3 == 1
        c3 = (recs["y"].astype(int) >> 1) * 10 + (recs["x"].astype(int) >> 1)
        for cell in range(80):
            k = np.nonzero(m & (c3 == cell))[0]
            assert ver[cell] == k.size, cell
            if k.size:
                assert np.abs(pr[cell] - ref7[k[-1]]).max() <= HEAD_TOL, cell
        seen["writes"] = int(m.sum())

    r = LV.run_live(headless_dir, rate_mev=2.0, duration_s=1.0, n_shards=6, halo=2, seed=seed,
                    gpu_blocks=1, ring_capacity=1 << 18, timing_capacity=1 << 18, group=6,
                    stages=2, inspect=inspect)
    say(f"run_live headless: status {r.status}, {r.ring_records} ring records, "
        f"{seen.get('writes')} prediction writes checked")
    assert r.status == 0 and r.drained == r.ring_records > 0 and seen.get("writes", 0) > 0
