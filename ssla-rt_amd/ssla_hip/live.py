"""The live hybrid pipeline: host producer shards -> fine-grained rings ->
persistent drain kernel, with emit -> prediction latency.

Mirrors the reference's live runner (orin/hybrid_runner_multi.py:430-760):
the producer (libstage01_to_gpu.so) runs stages 0 + 1 on CPU shards fed by
its paced synthetic source and publishes records to one ring per block; the
persistent kernel drains them and writes a GpuTimingSlot per record.  GPU
clock stamps are put on the host clock with a two-point calibration
(hybrid_runner_multi.py:525-534, 688-760).  Each point is a clock
handshake with the running kernel (the host writes a ping word, the kernel
answers with its clock), bracketed by two host clock readings; the
sample with the tightest bracket is kept, before the source starts and
after the rings have drained.  (The kernel's own start and exit stamps,
observed by a host thread spinning on them, remain the fallback: the host
can see them late, e.g. when the kernel started before the host began to
spin.)  Latency statistics cover output-producing records (owner, pass2 and
pass3), as the reference reports them.
"""
from __future__ import annotations

import time
from dataclasses import dataclass, field
from typing import Callable, Dict, Optional

import numpy as np

from . import abi, lib
from .hybrid import Drain, HostRings, LiveDrain, build_head_weights
from .producer import S01gAPI
from .topology import grid_topology


def model_info(weights_dir: str) -> "abi.SslaHipModelInfo":
    """Grid sizes of a weight directory (meta.json), without a GPU."""
    meta = (abi.ctypes.c_int * 4)()
    lib.check(lib.load().ssla_hip_meta_read(weights_dir.encode(), meta), "meta_read")
    i = abi.SslaHipModelInfo()
    i.height, i.width, i.num_classes, i.tdrop_window = meta
    i.H2, i.W2 = i.height >> 2, i.width >> 2
    i.H3, i.W3 = i.H2 >> 1, i.W2 >> 1
    return i


def _now_ns() -> int:
    return time.clock_gettime_ns(time.CLOCK_MONOTONIC_RAW)


def _spin_nonzero(read, timeout_s: float) -> int:
    t_end = time.monotonic() + timeout_s
    while True:
        v = read()
        if v:
            return v
        if time.monotonic() > t_end:
            return 0


def clock_pair(drain: Drain, blk: int, tries: int = 32, timeout_s: float = 0.05):
    """(host ns, GPU wall-clock ticks) of one instant from the live kernel's
    clock handshake on block blk (ssla_hip_timing_alloc's ping / pong words),
    and the host bracket in ns; None when the kernel does not answer."""
    words = np.ctypeslib.as_array(
        (np.ctypeslib.ctypes.c_ulonglong * 4).from_address(drain.cfg.kernel_start_clk[blk]))
    best = None
    for _ in range(tries):
        seq = (int(words[2]) + 1) & 0xffffffff or 1
        ta = _now_ns()
        words[2] = seq
        t_end = time.monotonic() + timeout_s
        while (int(words[3]) & 0xff) != (seq & 0xff):
            if time.monotonic() > t_end:
                return best
        tb = _now_ns()
        clk = int(words[3]) >> 8
        if best is None or tb - ta < best[2]:
            best = ((ta + tb) // 2, clk, tb - ta)
    return best


def _calibration(p0, p1, k0: int, t0_cpu: int, k1: int, t1_cpu: int):
    """(host ns at GPU tick k_ref, k_ref, ns per tick): from two handshake
    points when both exist, else from the kernel's start and exit stamps."""
    if p0 is not None and p1 is not None and p1[1] > p0[1]:
        return p0[0], p0[1], (p1[0] - p0[0]) / (p1[1] - p0[1])
    npt = (t1_cpu - t0_cpu) / max(1, (k1 - k0)) if k1 else 10.0
    return t0_cpu, k0, npt


def pct(a: np.ndarray, q: float) -> float:
    """Linear-interpolation percentile (include/lat_stats.h:33-40)."""
    return float(np.percentile(a, q * 100.0)) if a.size else float("nan")


@dataclass
class LiveResult:
    status: int                       # kernel exit: 0 stop flag, 2 overrun, 3 idle
    duration_s: float
    synth_events: int
    ring_records: int                 # records the producer published
    drained: int                      # records the kernel consumed
    output_records: int               # owner & pass2 & pass3 records timed
    lat_us: Dict[str, float] = field(default_factory=dict)
    producer_stats: list = field(default_factory=list)
    phase_us: Optional[np.ndarray] = None
    batch_sizes: Dict[str, float] = field(default_factory=dict)
    gpu_blocks: int = 1

    @property
    def drain_rate_kev_s(self) -> float:
        return self.drained / self.duration_s / 1e3

    @property
    def output_rate_kev_s(self) -> float:
        return self.output_records / self.duration_s / 1e3


def pick_cores(n_shards: int):
    """(synth_core, base_core) inside this process's CPU set: the shards on
    n_shards consecutive cores after the first allowed one, the source on
    the next allowed core after them (else on the first), so that the
    source shares its core with neither the shards nor this process's main
    thread; -1 (unpinned) where the set has no such run."""
    import os
    allowed = sorted(os.sched_getaffinity(0))
    if len(allowed) < n_shards + 1:
        return -1, -1
    first = allowed[0]
    for i in range(1, len(allowed) - n_shards + 1):
        run = allowed[i:i + n_shards]
        if run[-1] - run[0] == n_shards - 1:
            after = allowed[i + n_shards:]
            return (after[0] if after else first), run[0]
    return first, -1


def run_live(weights_dir: str, rate_mev: float = 2.0, duration_s: float = 8.0, n_shards: int = 6,
             halo: int = 2, base_core: Optional[int] = None, synth_core: Optional[int] = None,
             seed: int = 1, gpu_blocks: int = 8,
             n_blobs: int = 8, sigma_px: float = 3.0, bg_frac: float = 0.1,
             ring_capacity: int = 1 << 16, timing_capacity: int = 1 << 22, max_batch: int = 32,
             spin_ns: int = 200, profile: bool = True, drain_timeout_s: float = 30.0,
             back_pressure: bool = False, group: int = 0, stages: int = 1,
             inspect: Optional[Callable] = None) -> LiveResult:
    """One live run on one GPU.  back_pressure makes the producer wait for
    each ring's tail instead of overwriting unread slots.  gpu_blocks (1, 2, 4, 8, 16; the reference's
    default is 8) splits the s2 grid into owned strips with a 2-cell halo
    (topology.grid_topology); each strip has its own ring, hidden state and
    prediction grid and is drained by its own workgroup.  Halo records are
    published to every strip whose processed window holds them; latency
    covers the records that produce a prediction (owner, pass2, pass3).
    inspect(drain, rings, heads, topo), when given, is called once the kernel
    has stopped and before any buffer is freed (heads: records published per
    ring), e.g. to check the rings' contents and the final state.  group
    (3..6) drains each strip with that many workgroups, each owning channel
    slices of every layer (0: one workgroup per strip); stages 2 adds a second
    such group per strip that runs L6, L7 and the head of a batch while the
    first runs L4 and L5 of the next."""
    if base_core is None or synth_core is None:
        sc, bc = pick_cores(n_shards)
        synth_core = sc if synth_core is None else synth_core
        base_core = bc if base_core is None else base_core
    info = model_info(weights_dir)
    topo = grid_topology(gpu_blocks, info.W2, info.H2)
    nb = len(topo)
    # a directory without head keys gets the reference runner's random
    # single-linear head from the run's seed (hybrid_runner_multi.py:395-423)
    drain = Drain.from_weights_dir(weights_dir, n_blocks=nb, strips=[t.owned for t in topo],
                                   linear_head=build_head_weights(np.random.default_rng(seed)))
    rings = HostRings(nb, ring_capacity)
    prod = S01gAPI()
    live = None
    try:
        drain.alloc_timing(timing_capacity)
        c = drain.cfg
        prod.init(weights_dir, n_shards, halo, base_core, 1 << 16, 1 << 16)
        prod.attach_multi([rings.bufs[b].ptr for b in range(nb)], rings.head_ptrs(),
                          ring_capacity - 1, c.W2, c.H2,
                          [t.proc_x_lo for t in topo], [t.proc_x_hi for t in topo],
                          [t.proc_y_lo for t in topo], [t.proc_y_hi for t in topo])
        if back_pressure:
            prod.set_ring_tails(rings.tail_ptrs(), timeout_ms=1000.0 * drain_timeout_s)
        live = LiveDrain(drain, rings, spin_ns=spin_ns, max_batch=max_batch,
                         idle_timeout_ms=int((duration_s + drain_timeout_s + 30) * 1000),
                         profile=profile, group=group, stages=stages)
        clks = [np.ctypeslib.as_array((np.ctypeslib.ctypes.c_ulonglong * 2).from_address(
            c.kernel_start_clk[b])) for b in range(nb)]
        k0 = [_spin_nonzero(lambda a=a: int(a[0]), 30.0) for a in clks]
        t0_cpu = _now_ns()
        if not all(k0):
            raise RuntimeError("the live kernel did not start")
        sync0 = [clock_pair(drain, b) for b in range(nb)]
        prod.reset()
        t_start = time.monotonic()
        prod.start_synthetic_blobs(rate_mev, synth_core, seed, n_blobs, sigma_px, bg_frac)
        time.sleep(duration_s)
        prod.stop_synthetic()
        t_stop = time.monotonic()
        n_synth = prod.synthetic_n_pushed()
        # let the shards finish what was routed, then the kernel catch up
        t_end = time.monotonic() + drain_timeout_s
        while True:
            st = prod.stats()
            if st[0] >= n_synth and st[5] == 0:
                break
            if time.monotonic() > t_end:
                break
            time.sleep(0.001)
        heads = [int(rings.head[b]) for b in range(nb)]
        while any(int(rings.done[b]) < heads[b] for b in range(nb)) and time.monotonic() < t_end:
            time.sleep(0.0005)
        drained = [int(rings.done[b]) for b in range(nb)]
        sync1 = [clock_pair(drain, b) for b in range(nb)]
        rings.stop()
        k1 = [_spin_nonzero(lambda a=a: int(a[1]), 30.0) for a in clks]
        t1_cpu = _now_ns()
        status = live.wait()
        phase = live.phase_us
        live = None
        prod_stats = prod.stats()
        if inspect is not None:
            inspect(drain, rings, heads, topo)
        cols = {k: [] for k in ("e2d", "e2p", "p2d", "kern", "own", "ok")}
        for b in range(nb):
            # per-block two-point calibration of the GPU clock
            h_ref, k_ref, ns_per_tick = _calibration(sync0[b], sync1[b], k0[b], t0_cpu, k1[b], t1_cpu)
            tv = drain.timing(b)
            n_keep = min(drained[b], tv.size)
            tv = tv[(np.arange(drained[b] - n_keep, drained[b]) & (tv.size - 1))] if n_keep else tv[:0]
            ok = (tv["t_done_clk"] != 0) & (tv["t_emit_ns"] != 0) & (tv["t_push_ns"] != 0)
            t_done = h_ref + (tv["t_done_clk"].astype(np.float64) - k_ref) * ns_per_tick
            cols["e2d"].append((t_done - tv["t_emit_ns"].astype(np.float64)) / 1e3)
            cols["e2p"].append((tv["t_push_ns"].astype(np.float64)
                                - tv["t_emit_ns"].astype(np.float64)) / 1e3)
            cols["p2d"].append((t_done - tv["t_push_ns"].astype(np.float64)) / 1e3)
            cols["kern"].append((tv["t_done_clk"].astype(np.float64)
                                 - tv["t_pop_clk"].astype(np.float64)) * ns_per_tick / 1e3)
            cols["own"].append(ok & (tv["owner"] == 1))
            cols["ok"].append(ok)
        cat = {k: np.concatenate(v) if v else np.zeros(0) for k, v in cols.items()}
        own, ok = cat["own"].astype(bool), cat["ok"].astype(bool)
        lat = {}
        for name, key in (("emit_to_done", "e2d"), ("emit_to_push", "e2p"),
                          ("push_to_done", "p2d"), ("kernel", "kern")):
            a = cat[key][own]
            lat[name + "_p50"] = pct(a, 0.50)
            lat[name + "_p99"] = pct(a, 0.99)
            lat[name + "_max"] = float(a.max()) if a.size else float("nan")
        a = cat["e2d"][ok]
        lat["all_emit_to_done_p50"] = pct(a, 0.50)
        lat["all_emit_to_done_p99"] = pct(a, 0.99)
        bs = {}
        if phase is not None and phase[26] > 0:
            bs = {"batches": float(phase[25]), "mean": float(phase[26] / max(1.0, phase[25]))}
        return LiveResult(status=status, duration_s=t_stop - t_start, synth_events=n_synth,
                          ring_records=sum(heads), drained=sum(drained),
                          output_records=int(own.sum()), lat_us=lat, producer_stats=prod_stats,
                          phase_us=phase, batch_sizes=bs, gpu_blocks=nb)
    finally:
        if live is not None:
            rings.stop()
            try:
                live.wait(60000)
            except Exception:
                pass
        prod.shutdown()
        drain.close()
        rings.free()


@dataclass
class ReplayResult:
    status: int
    duration_s: float
    streams: list                      # per stream: dict of counts and latencies (us)
    phase_us: Optional[np.ndarray] = None

    @property
    def drained(self) -> int:
        return sum(s["drained"] for s in self.streams)


def run_replay(weights_dir: str, streams, rate_per_stream: float, ring_capacity: int = 1 << 16,
               timing_capacity: int = 1 << 18, max_batch: int = 32, spin_ns: int = 200,
               pin_core: Optional[int] = None, profile: bool = True, expect_p3=None,
               drain_timeout_s: float = 60.0, strips=None,
               speed: Optional[float] = None, group: int = 0, stages: int = 1,
               inspect: Optional[Callable] = None, seed: int = 1) -> ReplayResult:
    """Several rings live on one GPU: pre-built ring records (one array per
    ring) replayed into one ring each, one persistent workgroup per ring.
    Independent streams: rate_per_stream records/s each, round-robin.  One
    stream split into owned strips (strips = owned s2 boxes, the arrays
    holding each strip's processed-window records): speed paces all rings by
    the records' own times, (t - t_first) / speed us after the start.
    Latency is push -> prediction (records are published at their emit
    time).  expect_p3 (optional, one flag array per ring) gives each ring's
    drop drift: records whose timing-slot owner flag differs from it.
    inspect(drain), when given, is called once the kernel has stopped and
    before the state is freed.  group and stages as in run_live; a weight
    directory without head keys gets a random single-linear head from seed."""
    from .producer import Replay
    nb = len(streams)
    if pin_core is None:
        pin_core, _ = pick_cores(1)
    drain = Drain.from_weights_dir(weights_dir, n_blocks=nb, strips=strips,
                                   linear_head=build_head_weights(np.random.default_rng(seed)))
    rings = HostRings(nb, ring_capacity)
    live = rp = None
    try:
        drain.alloc_timing(timing_capacity)
        c = drain.cfg
        live = LiveDrain(drain, rings, spin_ns=spin_ns, max_batch=max_batch,
                         idle_timeout_ms=int((drain_timeout_s + 60) * 1000), profile=profile,
                         group=group, stages=stages)
        clk = np.ctypeslib.as_array((np.ctypeslib.ctypes.c_ulonglong * 2).from_address(c.kernel_start_clk[0]))
        k0 = _spin_nonzero(lambda: int(clk[0]), 30.0)
        t0_cpu = _now_ns()
        if not k0:
            raise RuntimeError("the live kernel did not start")
        sync0 = clock_pair(drain, 0)
        t_start = time.monotonic()
        rp = Replay([b.ptr for b in rings.bufs], rings.head_ptrs(), ring_capacity - 1, streams,
                    rate_per_stream * nb, pin_core, speed=speed)
        if speed is not None:
            ts = [float(x["t"][-1]) - float(x["t"][0]) for x in streams if x.size]
            span_s = (max(ts) if ts else 0.0) / 1e6 / speed
        else:
            span_s = sum(x.size for x in streams) / max(1.0, rate_per_stream * nb)
        t_end = time.monotonic() + span_s + drain_timeout_s
        while not rp.done() and time.monotonic() < t_end:
            time.sleep(0.001)
        duration = time.monotonic() - t_start
        counts = [int(s.size) for s in streams]
        while any(int(rings.done[b]) < counts[b] for b in range(nb)) and time.monotonic() < t_end:
            time.sleep(0.0005)
        drained = [int(rings.done[b]) for b in range(nb)]
        rp.stop()
        rp = None
        sync1 = clock_pair(drain, 0)
        rings.stop()
        k1 = _spin_nonzero(lambda: int(clk[1]), 30.0)
        t1_cpu = _now_ns()
        status = live.wait()
        phase = live.phase_us
        live = None
        if inspect is not None:
            inspect(drain)
        h_ref, k_ref, ns_per_tick = _calibration(sync0, sync1, k0, t0_cpu, k1, t1_cpu)
        out = []
        for b in range(nb):
            n = min(drained[b], timing_capacity)
            tv = drain.timing(b)[:n]
            own = tv["owner"] == 1
            t_done = h_ref + (tv["t_done_clk"].astype(np.float64) - k_ref) * ns_per_tick
            lat = (t_done - tv["t_push_ns"].astype(np.float64)) / 1e3
            kern = (tv["t_done_clk"].astype(np.float64) - tv["t_pop_clk"].astype(np.float64)) \
                * ns_per_tick / 1e3
            a = lat[own]
            s = {"records": counts[b], "drained": drained[b], "output_records": int(own.sum()),
                 "push_to_done_p50": pct(a, 0.50), "push_to_done_p99": pct(a, 0.99),
                 "push_to_done_max": float(a.max()) if a.size else float("nan"),
                 "kernel_p50": pct(kern[own], 0.50)}
            if expect_p3 is not None:
                e = np.asarray(expect_p3[b])[:n] == 1
                s["drop_drift"] = int((own != e).sum())
            out.append(s)
        return ReplayResult(status=status, duration_s=duration, streams=out, phase_us=phase)
    finally:
        if rp is not None:
            rp.stop()
        if live is not None:
            rings.stop()
            try:
                live.wait(60000)
            except Exception:
                pass
        drain.close()
        rings.free()
