"""Host producer (stages 0 + 1 on CPU shards feeding the drain's rings).

Oracle pins (oracle_s01_run, oracle_preprocess):
- preprocess by its closed form (first event 1, clamp to [0, 1], fp32 of the
  fp64 quotient, zeros off-sensor; ssla_kernels.cpp:288-309);
- the stage composition by the unfused module forward of L0..L3 with
  tdrop_window 1 (every event passes; ssla_ref.py:119-170), including the
  K = 1 first layer;
- the tdrop flags by brute-force arrival ranks per pooled cell.
Product checks (libstage01_to_gpu.so, libstage01_capi.so) against the
pinned oracle: one shard bit-for-bit in flags and within fp32 rounding in
features; several shards against one oracle instance per shard fed the
reference routing (strip ceil(W/N), halo columns, owner min(x//strip, N-1));
the ring protocol (seq_done = slot + 1 in every slot, ring boxes); and the
synthetic source against the reference's xorshift64 stream.
"""
import ctypes
import time

import numpy as np
import pytest

from oracle import oracle as O
from ssla_hip import abi, producer as P
from ssla_hip import stub

H0, W0 = 64, 80
FEAT_TOL = 1e-4


@pytest.fixture(scope="module")
def stub_w1(tmp_path_factory):
    d = tmp_path_factory.mktemp("stub_w1")
    stub.write_stub(str(d), height=H0, width=W0, seed=3, tdrop=1)
    return str(d)


def _events(n, seed, width=W0, height=H0):
    """t = event index (exact in fp32, so records can be matched by t)."""
    rng = np.random.default_rng(seed)
    x = rng.integers(0, width, n)
    y = rng.integers(0, height, n)
    p = np.where(rng.random(n) < 0.5, -1.0, 1.0)
    return P.events_array(np.arange(n), x, y, p)


def _oracle_shard(npz, window, height=H0, width=W0):
    return O.S01(O.layers_from_npz(npz, first=0), height, width, window)


# ---- oracle pins -------------------------------------------------------------------------

def test_preprocess_closed_form():
    last = np.full(4 * 6, -1.0)
    f = lambda t, x, y, p: O.preprocess(last, 4, 6, t, x, y, p)
    assert np.array_equal(f(10.0, 2, 1, -1.0), np.float32([1.0, -1.0]))       # first event
    assert np.array_equal(f(50010.0, 2, 1, 1.0), np.float32([0.5, 1.0]))       # 5e4 / 1e5
    assert np.array_equal(f(50011.0, 2, 1, 1.0), np.float32([np.float32(1e-5), 1.0]))
    assert np.array_equal(f(0.0, 2, 1, 1.0), np.float32([0.0, 1.0]))           # clamp below
    assert np.array_equal(f(3e5, 2, 1, 0.0), np.float32([1.0, 0.0]))           # clamp above
    assert np.array_equal(f(7.0, 6, 1, 1.0), np.float32([0.0, 0.0]))           # off-sensor
    assert np.array_equal(f(7.0, 3, 1, 1.0), np.float32([1.0, 1.0]))           # other pixel
    assert last[1 * 6 + 2] == 3e5 and last[1 * 6 + 3] == 7.0


def _raw_layer(npz, li):
    idx = sorted(int(k.split("/")[1]) for k in npz if k.endswith("/W_in_cat"))
    p = f"layers/{idx[li]}"
    raw = dict(W_in_cat=npz[f"{p}/W_in_cat"], W_out_cat=npz[f"{p}/W_out_cat"],
               qW=npz[f"{p}/q_proj/weight"], vW=npz[f"{p}/v_proj/weight"],
               gW=npz[f"{p}/g_proj/weight"], oW=npz[f"{p}/o_proj/weight"])
    ip = npz.get(f"{p}/input_proj/weight")
    return raw, ip, npz[f"{p}/norm/weight"], npz[f"{p}/norm/bias"]


def _module_layer(raw, ip, gamma, beta, x, H, ex, ey, Hl, Wl):
    """Unfused module forward of one layer in fp64: residual, the patch sum
    (only the centre cell when the layer has one position), LayerNorm."""
    d = lambda a: np.asarray(a, np.float64)
    D = raw["qW"].shape[0]
    A = max(raw["W_in_cat"].shape[1] // D, raw["W_out_cat"].shape[0] // D)
    res = d(ip) @ d(x) if ip is not None else d(x)
    acc = np.zeros(D)
    offs = [(0, 0)] if A == 1 else [(dy, dx) for dy in (-1, 0, 1) for dx in (-1, 0, 1)]
    for dy, dx in offs:
        py, px = ey + dy, ex + dx
        if not (0 <= py < Hl and 0 <= px < Wl):
            continue
        p = 0 if A == 1 else (1 - dy) * 3 + (1 - dx)
        pin = 0 if raw["W_in_cat"].shape[1] == D else p
        pout = 0 if raw["W_out_cat"].shape[0] == D else p
        u = d(x) @ d(raw["W_in_cat"][:, pin * D:(pin + 1) * D])
        q, v, g = u @ d(raw["qW"]).T, u @ d(raw["vW"]).T, u @ d(raw["gW"]).T
        c = py * Wl + px
        hn = 1.0 / (1.0 + np.exp(-g)) * d(H[c]) + v
        H[c] = hn.astype(np.float32)
        acc += ((q * hn) @ d(raw["oW"]).T) @ d(raw["W_out_cat"][pout * D:(pout + 1) * D])
    y = acc + res
    mu = y.mean()
    return ((y - mu) / np.sqrt(((y - mu) ** 2).mean() + 1e-5) * d(gamma) + d(beta)).astype(np.float32)


def test_oracle_stages_match_module_forward(stub_w1):
    npz = O.load_npz(stub_w1)
    ev = _events(300, seed=7, width=12, height=8)         # dense: repeated cells and patches
    sh = _oracle_shard(npz, window=1)
    p0, p1, feat, x2, y2 = sh.run(ev, precision=64)
    assert (p0 == 1).all() and (p1 == 1).all()
    raws = [_raw_layer(npz, li) for li in range(4)]
    Hs = [np.zeros((H0 * W0, 12), np.float32), np.zeros((H0 * W0, 12), np.float32),
          np.zeros((H0 * W0 // 4, 24), np.float32), np.zeros((H0 * W0 // 4, 24), np.float32)]
    last = {}
    for i, (t, x, y, p) in enumerate(ev):
        x, y = int(x), int(y)
        dt = 1.0 if (x, y) not in last else min(1.0, max(0.0, (t - last[(x, y)]) / 1e5))
        last[(x, y)] = t
        a = _module_layer(*raws[0], np.float32([dt, p]), Hs[0], x, y, H0, W0)
        b = _module_layer(*raws[1], a, Hs[1], x, y, H0, W0)
        c = _module_layer(*raws[2], b, Hs[2], x >> 1, y >> 1, H0 // 2, W0 // 2)
        o = _module_layer(*raws[3], c, Hs[3], x >> 1, y >> 1, H0 // 2, W0 // 2)
        assert np.abs(feat[i] - o).max() < 1e-4, i
        assert (x2[i], y2[i]) == (x >> 2, y >> 2)
    for li in range(4):
        assert np.abs(sh.H[li] - Hs[li]).max() < 1e-4, li


def _brute_flags(ev, window, H=H0, W=W0):
    c1, c2 = {}, {}
    p0 = np.zeros(len(ev), np.int8)
    p1 = np.zeros(len(ev), np.int8)
    for i, (_, x, y, _) in enumerate(ev):
        k = (int(x) >> 1, int(y) >> 1)
        r = c1.get(k, 0)
        c1[k] = (r + 1) % 256
        if r % window == 0:
            p0[i] = 1
            k2 = (int(x) >> 2, int(y) >> 2)
            r2 = c2.get(k2, 0)
            c2[k2] = (r2 + 1) % 256
            p1[i] = int(r2 % window == 0)
    return p0, p1


def test_oracle_flags_brute_force(stub_dir, stub_npz):
    ev = _events(4000, seed=2)
    ev[17, 1] = W0 + 3                                  # off-sensor event
    sh = _oracle_shard(stub_npz, window=4)
    p0, p1, feat, _, _ = sh.run(ev, precision=32)
    on = np.ones(len(ev), bool)
    on[17] = False
    assert p0[17] == -2 and p1[17] == -2
    b0, b1 = _brute_flags(ev[on], 4)
    assert np.array_equal(p0[on], b0) and np.array_equal(p1[on], b1)
    assert not feat[p1 != 1].any()


def test_oracle_halo_events_touch_stage0_only(stub_npz):
    ev = _events(500, seed=4)
    own = np.ones(len(ev), np.uint8)
    own[::3] = 0
    a = _oracle_shard(stub_npz, window=4)
    pa0, pa1, _, _, _ = a.run(ev, owner=own)
    assert (pa0[own == 0] == -1).all() and (pa1[own == 0] == -1).all()
    # tdrop counters see only owner events ...
    b = _oracle_shard(stub_npz, window=4)
    b.run(ev[own == 1])
    assert np.array_equal(a.td0, b.td0) and np.array_equal(a.td1, b.td1)
    # ... while stage 0 state sees every event
    c = _oracle_shard(stub_npz, window=4)
    c.run(ev)
    assert np.array_equal(a.H[0], c.H[0]) and np.array_equal(a.H[1], c.H[1])
    assert np.array_equal(a.last_t, c.last_t)


# ---- the product: libstage01_to_gpu.so ------------------------------------------------------

class _Rings:
    """Rings in plain host memory (the producer only stores into them)."""

    def __init__(self, n, cap=1 << 16):
        self.cap = cap
        self.bufs = [np.zeros(cap, abi.INPUT_DTYPE) for _ in range(n)]
        self.heads = np.zeros(n, np.uint64)

    def buf_ptrs(self):
        return [b.ctypes.data for b in self.bufs]

    def head_ptrs(self):
        return [self.heads.ctypes.data + 8 * k for k in range(len(self.bufs))]

    def records(self, k):
        n = int(self.heads[k])
        assert n <= self.cap
        r = self.bufs[k][:n]
        assert np.array_equal(r["seq_done"], np.arange(1, n + 1, dtype=np.uint64))
        return r


def _run_producer(weights, ev, n_shards, halo, rings, boxes, W2, H2):
    api = P.S01gAPI()
    api.init(weights, n_shards, halo, -1, 1 << 14, 1 << 12)
    try:
        lo_x, hi_x, lo_y, hi_y = zip(*boxes)
        api.attach_multi(rings.buf_ptrs(), rings.head_ptrs(), rings.cap - 1, W2, H2,
                         lo_x, hi_x, lo_y, hi_y)
        acc = api.submit(ev)
        owner, halo_to = P.routing(ev[:, 1], W0, n_shards, halo)
        inb = (ev[:, 1] >= 0) & (ev[:, 1] < W0) & (ev[:, 2] >= 0) & (ev[:, 2] < H0)
        assert acc == int(inb.sum())
        st = api.wait_processed(acc, sum(1 for i, _ in halo_to if inb[i]))
    finally:
        api.shutdown()
    return st


def _oracle_sharded(npz, ev, n_shards, halo, window):
    """One oracle shard per producer shard, fed what the routing delivers."""
    owner, halo_to = P.routing(ev[:, 1], W0, n_shards, halo)
    per = [[] for _ in range(n_shards)]
    for i in range(len(ev)):
        per[int(owner[i])].append((i, 1))
    for i, k in halo_to:
        per[k].append((i, 0))
    n = len(ev)
    p0, p1 = np.zeros(n, np.int8), np.zeros(n, np.int8)
    feat = np.zeros((n, 24), np.float32)
    for k in range(n_shards):
        idx = np.array(sorted(per[k]), dtype=np.int64).reshape(-1, 2)
        sh = _oracle_shard(npz, window)
        a0, a1, f, _, _ = sh.run(ev[idx[:, 0]], owner=idx[:, 1].astype(np.uint8), precision=32)
        o = idx[:, 1] == 1
        p0[idx[o, 0]], p1[idx[o, 0]], feat[idx[o, 0]] = a0[o], a1[o], f[o]
    return p0, p1, feat


def _check_records(recs, ev, p1, feat):
    want = np.nonzero(p1 == 1)[0]
    got = recs["t"].astype(np.int64)
    assert np.array_equal(np.sort(got), want)
    order = np.argsort(got)
    r = recs[order]
    assert np.array_equal(r["x"], (ev[want, 1].astype(np.int64) >> 2).astype(np.uint16))
    assert np.array_equal(r["y"], (ev[want, 2].astype(np.int64) >> 2).astype(np.uint16))
    assert np.abs(r["feat1"] - feat[want]).max() < FEAT_TOL
    assert (r["t_push_ns"] >= r["t_emit_ns"]).all() and (r["t_emit_ns"] > 0).all()


def test_one_shard_matches_oracle(stub_dir, stub_npz):
    ev = _events(6000, seed=11)
    rings = _Rings(1)
    st = _run_producer(stub_dir, ev, 1, 2, rings, [(0, W0 // 4, 0, H0 // 4)], W0 // 4, H0 // 4)
    sh = _oracle_shard(stub_npz, window=4)
    p0, p1, feat, _, _ = sh.run(ev, precision=32)
    assert st[0] == len(ev) and st[1] == 0
    assert st[2] == (p0 == 1).sum() and st[13] == (p1 == 1).sum() and st[14] == (p1 == 1).sum()
    _check_records(rings.records(0), ev, p1, feat)
    assert st[12] == len(ev) and 0 < st[6] <= st[8] <= st[10]
    assert st[22 + P.SEGMENTS.index("push")] == (p1 == 1).sum()


@pytest.mark.parametrize("n_shards,halo", [(3, 2), (6, 2), (4, 0)])
def test_sharded_matches_oracle_per_shard(stub_dir, stub_npz, n_shards, halo):
    ev = _events(8000, seed=20 + n_shards)
    ev[5, 1] = -1.0                                      # off-sensor: counted, not routed
    rings = _Rings(1)
    st = _run_producer(stub_dir, ev, n_shards, halo, rings, [(0, W0 // 4, 0, H0 // 4)],
                       W0 // 4, H0 // 4)
    p0, p1, feat = _oracle_sharded(stub_npz, ev[np.arange(len(ev)) != 5], n_shards, halo, 4)
    p0 = np.insert(p0, 5, 0)
    p1 = np.insert(p1, 5, 0)
    feat = np.insert(feat, 5, 0, axis=0)
    assert st[3] == 1
    assert st[2] == (p0 == 1).sum() and st[13] == (p1 == 1).sum()
    _check_records(rings.records(0), ev, p1, feat)


@pytest.mark.parametrize("n_shards,halo", [(1, 2), (3, 2), (6, 2), (8, 4)])
def test_halo_count_matches_routing(n_shards, halo):
    x = np.arange(-3, W0 + 3)
    want = len(P.routing(x, W0, n_shards, halo)[1])
    assert P.halo_count(x, W0, n_shards, halo) == want
    # brute force over shard strips: every shard whose halo-widened strip
    # holds x, other than the owner
    strip = (W0 + n_shards - 1) // n_shards
    brute = 0
    for xi in x:
        own = min(xi // strip, n_shards - 1)
        for k in range(n_shards):
            if k != own and abs(k - xi // strip) <= 1 and k * strip - halo <= xi < (k + 1) * strip + halo:
                brute += 1
    assert want == brute


def test_ring_boxes(stub_dir, stub_npz):
    """Two rings over overlapping s2 x ranges (block_proc_range with halo 2):
    each record goes to every ring whose box holds its s2 cell."""
    W2, H2 = W0 // 4, H0 // 4
    boxes = [(0, W2 // 2 + 2, 0, H2), (W2 // 2 - 2, W2, 0, H2)]
    ev = _events(5000, seed=5)
    rings = _Rings(2)
    st = _run_producer(stub_dir, ev, 2, 2, rings, boxes, W2, H2)
    p0, p1, feat = _oracle_sharded(stub_npz, ev, 2, 2, 4)
    x2 = ev[:, 1].astype(np.int64) >> 2
    for k, (lo, hi, _, _) in enumerate(boxes):
        sel = (p1 == 1) & (x2 >= lo) & (x2 < hi)
        r = rings.records(k)
        assert st[14 + k] == sel.sum() == r.size
        _check_records(r, ev, np.where(sel, p1, 0), feat)


def test_unattached_and_reset(stub_dir):
    api = P.S01gAPI()
    api.init(stub_dir, 2, 2, -1, 4096)
    try:
        ev = _events(1000, seed=8)
        assert api.submit(ev) == 1000
        owner, halo_to = P.routing(ev[:, 1], W0, 2, 2)
        st = api.wait_processed(1000, len(halo_to))
        assert st[14] == 0 and st[22 + P.SEGMENTS.index("push")] == 0 and st[13] > 0
        api.reset()
        st = api.stats()
        assert st[0] == st[1] == st[2] == st[12] == st[13] == 0
        assert api.submit(np.zeros((0, 4), np.float32)) == 0
    finally:
        api.shutdown()


def test_bad_dir_and_null_handle(tmp_path):
    lib = P.load_to_gpu()
    assert not lib.s01g_init(str(tmp_path).encode(), 1, 2, -1, 1024)
    out = (ctypes.c_double * 32)(*([7.0] * 32))
    lib.s01g_snapshot_stats(None, out)
    assert list(out) == [0.0] * 32
    assert lib.s01g_submit_batch(None, None, 5) == 0
    lib.s01g_shutdown(None)


def _xorshift_stream(seed, n, W, H):
    s = seed or 0x9E3779B97F4A7C15
    m = (1 << 64) - 1
    out = []
    for _ in range(n):
        s ^= (s << 13) & m
        s ^= s >> 7
        s ^= (s << 17) & m
        out.append((s % W, (s >> 16) % H, (s >> 32) & 1))
    return np.array(out, np.int64)


def test_synthetic_uniform_is_reference_xorshift(stub_w1):
    """tdrop window 1: every event reaches the ring, so the ring holds the
    source's stream in order (one shard)."""
    api = P.S01gAPI()
    api.init(stub_w1, 1, 2, -1, 4096)
    rings = _Rings(1)
    api.attach_multi(rings.buf_ptrs(), rings.head_ptrs(), rings.cap - 1, W0 // 4, H0 // 4,
                     [0], [W0 // 4], [0], [H0 // 4])
    try:
        api.start_synthetic(0.02, -1, 12345)
        time.sleep(0.15)
        api.stop_synthetic()
        n = api.synthetic_n_pushed()
        st = api.wait_processed(n, 0)
    finally:
        api.shutdown()
    assert 500 < n < 20000 and st[0] == n
    r = rings.records(0)
    assert r.size == n
    ref = _xorshift_stream(12345, n, W0, H0)
    assert np.array_equal(r["x"], (ref[:, 0] >> 2).astype(np.uint16))
    assert np.array_equal(r["y"], (ref[:, 1] >> 2).astype(np.uint16))
    t = np.float32(0)
    ts = np.empty(n, np.float32)
    for k in range(n):
        t = np.float32(t + np.float32(1.0 / 0.02))
        ts[k] = t
    assert np.array_equal(r["t"], ts)


def test_synthetic_blobs_runs(stub_w1):
    api = P.S01gAPI()
    api.init(stub_w1, 2, 2, -1, 4096)
    rings = _Rings(1)
    api.attach_multi(rings.buf_ptrs(), rings.head_ptrs(), rings.cap - 1, W0 // 4, H0 // 4,
                     [0], [W0 // 4], [0], [H0 // 4])
    try:
        api.start_synthetic_blobs(0.05, -1, 1, n_blobs=8, sigma_px=3.0, bg_frac=0.1)
        time.sleep(0.1)
        api.stop_synthetic()
        n = api.synthetic_n_pushed()
        st = api.wait_processed(n, 0)
    finally:
        api.shutdown()
    r = rings.records(0)
    assert n > 1000 and r.size == st[14] > 0
    assert (r["x"] < W0 // 4).all() and (r["y"] < H0 // 4).all()
    # with tdrop window 1 every event is a record; blob events cluster, so the
    # per-cell counts are far more dispersed than uniform (Poisson) counts
    counts = np.bincount(r["y"].astype(np.int64) * (W0 // 4) + r["x"], minlength=(W0 // 4) * (H0 // 4))
    assert counts.std() > 2 * np.sqrt(counts.mean())


# ---- libstage01_capi.so --------------------------------------------------------------------

def test_capi_counts_match_oracle(stub_dir, stub_npz):
    ev = _events(5000, seed=31)
    api = P.S0API()
    api.init(stub_dir, 3, 2, -1, 4096)
    try:
        assert api.submit(ev) == len(ev)
        _, halo_to = P.routing(ev[:, 1], W0, 3, 2)
        st = api.wait_processed(len(ev), len(halo_to))
    finally:
        api.shutdown()
    p0, p1, _ = _oracle_sharded(stub_npz, ev, 3, 2, 4)
    assert st[0] == len(ev) and st[1] == len(halo_to)
    assert st[2] == (p0 == 1).sum() and st[13] == (p1 == 1).sum()
    assert st[14] == st[15] == 0


def test_replay_publishes_every_ring_in_order():
    """s01g_replay_*: each ring receives its records in order with the
    publish protocol; rings of different lengths; unpaced and paced."""
    from ssla_hip import events
    rng = np.random.default_rng(9)
    recs = []
    for n in (700, 0, 1234):
        r = events.Records(np.arange(n, dtype=np.float32), rng.integers(0, 20, n).astype(np.uint16),
                           rng.integers(0, 16, n).astype(np.uint16),
                           rng.normal(0, 0.5, (n, 24)).astype(np.float32))
        recs.append(events.to_records(r))
    for rate in (0.0, 2e6):
        rings = _Rings(3, cap=1 << 11)
        rp = P.Replay(rings.buf_ptrs(), rings.head_ptrs(), rings.cap - 1, recs, rate)
        t_end = time.monotonic() + 30
        while not rp.done() and time.monotonic() < t_end:
            time.sleep(0.001)
        assert rp.done() and rp.published() == 700 + 1234
        rp.stop()
        for k, src in enumerate(recs):
            got = rings.records(k)
            assert got.size == src.size
            for f in ("t", "x", "y", "feat1"):
                assert np.array_equal(got[f], src[f]), (k, f)
            assert np.array_equal(got["t_push_ns"], got["t_emit_ns"])
            assert (got["t_push_ns"] > 0).all() and (np.diff(got["t_push_ns"].astype(np.int64)) >= 0).all()
    with pytest.raises(RuntimeError):
        P.Replay([0], [0], 1023, [recs[0]], 0.0)


def test_back_pressure_never_overwrites_unread_slots(stub_dir, stub_npz):
    """A 64-slot ring drained slowly by a consumer thread: with the tails
    set, publishers wait for their slot, so every record arrives once, in
    slot order, and none is overwritten."""
    import threading
    import time
    ev = _events(6000, seed=31)
    cap = 64
    buf = np.zeros(cap, abi.INPUT_DTYPE)
    words = np.zeros(2, np.uint64)            # head, tail
    got = []
    stop = threading.Event()

    def consumer():
        t = 0
        while not stop.is_set() or int(words[0]) > t:
            if int(buf[t & (cap - 1)]["seq_done"]) == t + 1:
                got.append(buf[t & (cap - 1)].copy())
                t += 1
                words[1] = t
                if t % 16 == 0:
                    time.sleep(0.0005)
            else:
                time.sleep(0)

    api = P.S01gAPI()
    api.init(stub_dir, 2, 2, -1, 1 << 14, 1 << 12)
    th = threading.Thread(target=consumer)
    th.start()
    try:
        api.attach_multi([buf.ctypes.data], [words.ctypes.data], cap - 1, W0 // 4, H0 // 4,
                         [0], [W0 // 4], [0], [H0 // 4])
        api.set_ring_tails([words.ctypes.data + 8], timeout_ms=5000)
        api.submit(ev)
        owner, halo_to = P.routing(ev[:, 1], W0, 2, 2)
        st = api.wait_processed(len(ev), len(halo_to))
    finally:
        api.shutdown()
        stop.set()
        th.join(30)
    n = int(words[0])
    assert len(got) == n == st[14] and st[28] > 0 and st[30] == 0
    recs = np.array(got)
    p0, p1, feat = _oracle_sharded(stub_npz, ev, 2, 2, 4)
    _check_records(recs, ev, p1, feat)


def test_back_pressure_times_out_and_overwrites(stub_dir):
    """A consumer that never advances: publishers give up after the
    timeout, count it, and overwrite (the drain would report the overrun)."""
    ev = _events(3000, seed=32)
    cap = 16
    buf = np.zeros(cap, abi.INPUT_DTYPE)
    words = np.zeros(2, np.uint64)
    api = P.S01gAPI()
    api.init(stub_dir, 1, 2, -1, 1 << 14, 1 << 12)
    try:
        api.attach_multi([buf.ctypes.data], [words.ctypes.data], cap - 1, W0 // 4, H0 // 4,
                         [0], [W0 // 4], [0], [H0 // 4])
        api.set_ring_tails([words.ctypes.data + 8], timeout_ms=0.05)
        api.submit(ev)
        st = api.wait_processed(len(ev), 0)
    finally:
        api.shutdown()
    n = int(words[0])
    assert n == st[14] > cap
    assert st[30] == n - cap and st[28] == n - cap
