#!/usr/bin/env python3
"""Offline drain throughput of SSLA-S s2 + s3 + YOLOX head on one MI355X.

Workload: 200,000 pre-filled ring records at 80x64 (s2 grid 20x16) drawn
from 8 moving Gaussian blobs (sigma 3 px, 0.5-2 px/ms, reflecting) plus 10%
uniform background, feat1 ~ N(0, 0.5^2), stub weights (schema of
tools/make_ssla_stub.py, seed 1, tdrop window 4).  Records are resident in
HBM before timing starts.  One step = reset the instance state, then drain
all 200k records (L4, L5, tdrop_s2, L6, L7, tdrop_s3, head) through the C
ABI.  Every step does identical work, so the output-producing count of a
step is the count of the first warmup step (re-checked after timing).

value = output-producing records (owner & pass2 & pass3) per second, in
kev/s, over exactly --steps timed steps.  Alongside: ring-record kev/s (the
unit of the reference's 247 kev/s Orin figure), the roofline of the
dominant kernel from HIP events on the drain's stream, and the CPU baseline
on bounded samples (the oracle's fp32 s2 + s3 + head on one core; s0 + s1 on
6 shard threads; the 50,000-event CPU reference case end to end on one core).

The metric's latency half comes from the live pipeline, run after the timed
region: the host producer (6 shards, halo 2) fed by its paced synthetic
source at 2.0 Mev/s with the same blob distribution, fine-grained rings, the
persistent drain kernel over 8 GPU blocks (the reference's default 2 x 4
strip topology with a 2-cell halo), for 8 s; emit -> prediction p50 / p99 / max of the
output-producing records, GPU clocks put on the host clock by the kernel's
start / exit stamps.
"""
import argparse
import ctypes
import json
import re
import os
import sys
import tempfile
import time
from pathlib import Path

import numpy as np

ROOT = Path(__file__).resolve().parent
for _p in (str(ROOT), str(ROOT / "ssla-rt_amd")):
    if _p not in sys.path:
        sys.path.insert(0, _p)

METRIC = ("drain kev/s (output-producing) at 80×64 on 1 GPU; "
          "p50/p99 emit→prediction µs")
PEAK_FP32_TFLOPS = 157.3
PEAK_HBM_GBS = 8000.0
C1, C2, C3 = 24, 48, 96


def inbounds(x, y, H, W):
    n = np.zeros(x.shape, np.int64)
    for dy in (-1, 0, 1):
        for dx in (-1, 0, 1):
            n += ((x + dx >= 0) & (x + dx < W) & (y + dy >= 0) & (y + dy < H))
    return n


def algorithmic_work(x, y, p2, p3, owner, H2=16, W2=20):
    """Algorithmic work of each launch of the whole-ring drain: the minimal
    MACs of the reference's skipping semantics (L5 output and L6/L7 only for
    pass2, L7 output and head for pass3), the algorithmic bytes of the
    measurement's per-record accounting (each layer's input rows, the
    hidden-state read and write per pair, the output slots; weights excluded,
    they stay in cache) and the bytes each launch moves at its interface,
    which also counts this design's intermediates (the projections' [v | g]
    pair rows, the recurrence's h rows).  Returns ({phase: flops},
    {phase: algorithmic bytes}, {phase: interface bytes}, total MACs)."""
    x = x.astype(np.int64)
    y = y.astype(np.int64)
    ok = (x >= 0) & (x < W2) & (y >= 0) & (y < H2)     # off-grid records are skipped
    n2 = np.where(ok, inbounds(x, y, H2, W2), 0)
    m2, m3 = ok & (p2 == 1), ok & (p3 == 1)
    n3 = inbounds(x >> 1, y >> 1, H2 >> 1, W2 >> 1)
    S2, S2p, S3p, S3pp = n2.sum(), n2[m2].sum(), n3[m2].sum(), n3[m3].sum()
    N, N2, N3 = int(ok.sum()), int(m2.sum()), int(m3.sum())
    F = 4.0
    # projections compute v, g for every pair entering the layer; the
    # contraction computes q for the pairs of its output records, then
    # q*h through goW, and the residual (input_proj where IN != OUT)
    mac = {
        "L4.proj": S2 * C1 * 2 * C2,
        "L4.out": S2 * C1 * C2 + S2 * C2 * C2 + N * C1 * C2,
        "L5.proj": S2 * C2 * 2 * C2,
        "L5.out": S2p * C2 * C2 + S2p * C2 * C2,
        "L6.proj": S3p * C2 * 2 * C3,
        "L6.out": S3p * C2 * C3 + S3p * C3 * C3 + N2 * C2 * C3,
        "L7.proj": S3p * C3 * 2 * C3,
        "L7.out": S3pp * C3 * C3 + S3pp * C3 * C3,
        "head": int((m3 & (owner == 1)).sum()) * (2 * C3 * C3 + 7 * C3),
    }
    flops = {k: 2.0 * v for k, v in mac.items()}
    iface = {
        "L4.proj": F * (N * C1 + S2 * 2 * C2),
        "L4.out": F * (S2 * C2 + N * C1 + N * C2),
        "L5.proj": F * (N * C2 + S2 * 2 * C2),
        "L5.out": F * (S2p * C2 + 2 * N2 * C2),
        "L6.proj": F * (N2 * C2 + S3p * 2 * C3),
        "L6.out": F * (S3p * C3 + N2 * C2 + N2 * C3),
        "L7.proj": F * (N2 * C3 + S3p * 2 * C3),
        "L7.out": F * (S3pp * C3 + 2 * N3 * C3),
    }
    # algorithmic: a projection reads its layer's input rows, a contraction
    # those and writes its output rows
    byts = {
        "L4.proj": F * N * C1,
        "L4.out": F * (N * C1 + N * C2),
        "L5.proj": F * N * C2,
        "L5.out": F * 2 * N2 * C2,
        "L6.proj": F * N2 * C2,
        "L6.out": F * (N2 * C2 + N2 * C3),
        "L7.proj": F * N2 * C3,
        "L7.out": F * 2 * N3 * C3,
    }
    # the recurrence h = sigmoid(g) h + v over every pair entering the layer
    # (sigmoid ~ 4 FLOP, the map composition and the replay 2 FMA):
    # algorithmically the pair's hidden state is read and written; one launch
    # (k_scan, in the apply slot) reads each pair's v, g rows once and writes
    # h where the output is consumed
    for L, pairs, need, out in (("L4", S2, S2, C2), ("L5", S2, S2p, C2),
                                ("L6", S3p, S3p, C3), ("L7", S3p, S3pp, C3)):
        byts[f"{L}.apply"] = F * pairs * out * 2
        iface[f"{L}.apply"] = F * (pairs * 2 * out + need * out)
        flops[f"{L}.apply"] = 6.0 * pairs * out
    byts["emit"] = iface["emit"] = float(x.size * 392)     # every ring record's slot
    total_mac = sum(mac.values())
    return flops, byts, iface, total_mac


def _cpu_model() -> str:
    try:
        with open("/proc/cpuinfo") as f:
            for line in f:
                if line.startswith("model name"):
                    return line.split(":", 1)[1].strip()
    except OSError:
        pass
    return "unknown"


def _pin(cores) -> bool:
    try:
        os.sched_setaffinity(0, set(cores))
        return True
    except (AttributeError, OSError):
        return False


SEGMENTS = ("preprocess", "s0", "tdrop0", "s1", "tdrop1", "push")


def _stage01(stub_dir, ev, n_shards, base_core, submit_cores, spawn_cores, W2, H2, ring=False):
    """s0 + s1 of `ev` (raw [t, x, y, p] events) on n_shards shard threads
    (halo 2; pinned to base_core, base_core + 1, ... or, when base_core < 0,
    left on `spawn_cores`), submitted from this thread pinned to
    `submit_cores`.
    With `ring`, one host ring covering the whole s2 grid receives the
    records.  Returns (seconds from submit to the last shard done, stats
    slots, records or None)."""
    from ssla_hip import producer as P
    from ssla_hip.abi import INPUT_DTYPE
    api = P.S01gAPI()
    _pin(spawn_cores)                  # shard threads start with this mask
    api.init(stub_dir, n_shards, 2, base_core, 1 << 14)
    buf = head = None
    try:
        if ring:
            cap = 1 << max(1, int(np.ceil(np.log2(len(ev)))))   # no wrap
            buf = np.zeros(cap, INPUT_DTYPE)
            head = np.zeros(1, np.uint64)
            api.attach_multi([buf.ctypes.data], [head.ctypes.data], cap - 1, W2, H2,
                             [0], [W2], [0], [H2])
        n_halo = P.halo_count(ev[:, 1], 4 * W2, n_shards, 2)
        _pin(submit_cores)
        api.reset()
        t0 = time.perf_counter()
        acc = api.submit(ev)
        st = api.wait_processed(acc, n_halo, timeout_s=120.0)
        dt = time.perf_counter() - t0
    finally:
        api.shutdown()
    return dt, st, (buf[:int(head[0])] if ring else None)


def _segments(st, n_events):
    """Per-segment mean time: us per item the segment handled and us per
    submitted event (stats slots 16..27)."""
    out = {}
    for k, name in enumerate(SEGMENTS):
        ns, cnt = st[16 + k], st[22 + k]
        if cnt > 0:
            out[name] = {"us_per_item": round(ns / cnt / 1e3, 4),
                         "us_per_event": round(ns / n_events / 1e3, 4), "items": int(cnt)}
    return out


def _compare(gpu_out, n, p2, p3, feat, head7):
    """The drain's first-step outputs against the oracle's fp32 path over the
    first n records: decisions bit for bit, s3_feat and raw head outputs of
    records both mark pass-3 (and the drain owns)."""
    out, head = gpu_out
    g2, g3 = out["pass2"][:n] == 1, out["pass3"][:n] == 1
    m = g3 & (p3 == 1)
    res = {"records_checked": int(n), "pass2_differ": int((g2 != (p2 == 1)).sum()),
           "pass3_differ": int((g3 != (p3 == 1)).sum()), "pass3_records": int(m.sum())}
    if m.any():
        d = np.abs(out["s3_feat"][:n][m] - feat[m])
        res["s3_feat_max_abs_diff"] = float(d.max())
        res["s3_feat_max_rel_diff"] = float(d.max() / max(np.abs(feat[m]).max(), 1e-30))
        if head is not None:
            res["head_max_abs_diff"] = float(np.abs(head[:n][m] - head7[m]).max())
    return res


def cpu_baseline(stub_dir, rec, budget_s=15.0, H2=16, W2=20, gpu_out=None):
    """The CPU path timed on this host:
      value       the oracle's fp32 s2 + s3 + head (the generic C++
                  reference path restated), one pinned thread, on the first
                  records of the GPU workload -- output-producing kev/s,
                  the unit of the GPU value;
      stage01     s0 + s1 of raw uniform events at 80x64 / 2 Mev/s on 6
                  shard threads (cores 1-6, submission from core 0, when
                  this process may use them);
      end_to_end  the 50,000-event CPU reference case on one core: s0 + s1
                  on one shard, then the records through the fp32 oracle.
    gpu_out = (output slots, head rows) of the drain's first step over `rec`
    (from reset state), compared with the oracle over the same records.
    About budget_s seconds of CPU work in all."""
    from oracle import oracle as O
    from ssla_hip import events as E
    all_cores = sorted(os.sched_getaffinity(0)) if hasattr(os, "sched_getaffinity") else [0]
    core0 = all_cores[0]
    w = O.load_npz(stub_dir)
    layers = O.layers_from_npz(w)
    head = O.head_from_npz(w)

    # s2 + s3 + head, one thread
    _pin([core0])
    st = O.S2S3(layers, H2, W2, 4, head=head)
    k = 4000
    t0 = time.perf_counter()
    st.run(rec.x[:k], rec.y[:k], rec.feat1[:k], precision=32, want_feat=False, want_head=True)
    rate = k / (time.perf_counter() - t0)
    n = int(min(rec.x.size, max(k, rate * 0.55 * budget_s)))
    st = O.S2S3(layers, H2, W2, 4, head=head)
    t0 = time.perf_counter()
    p2, p3, feat, head7 = st.run(rec.x[:n], rec.y[:n], rec.feat1[:n], precision=32,
                                 want_feat=True, want_head=True)
    dt = time.perf_counter() - t0
    n_out = int((p3 == 1).sum())
    res = {"value": round(n_out / dt / 1e3, 4), "unit": "kev/s", "cores": 1, "kind": "port",
           "sample": f"first {n} of the {rec.x.size} records (fp32 oracle path, "
                     f"-O3 -ffast-math -march=x86-64-v3, one pinned thread); "
                     f"{n_out} output-producing in {dt:.2f} s",
           "ring_record_kev_s": round(n / dt / 1e3, 3),
           "parity_vs_oracle": None if gpu_out is None else _compare(gpu_out, n, p2, p3,
                                                                          feat, head7),
           "_oracle": (n, p2, p3, feat),
           "s2s3_head_us_per_record": round(dt / n * 1e6, 3),
           "host": {"cpu_model": _cpu_model(), "nproc": os.cpu_count(),
                    "usable_cores": len(all_cores)},
           "compiler_flags": {
               "oracle_fp32": "gcc -O3 -ffast-math -march=x86-64-v3",
               "stage01": "g++ -O3 -march=x86-64-v3 -funroll-loops -ffast-math "
                          "-fno-finite-math-only"}}

    # s0 + s1 on 6 shards
    want = list(range(core0, core0 + 7))
    pinned = all(c in all_cores for c in want)
    base, sub = (core0 + 1, [core0]) if pinned else (-1, all_cores)
    ev = E.raw_uniform(200_000, seed=2)
    dt, _, _ = _stage01(stub_dir, ev, 6, base, sub, all_cores, W2, H2)
    n_ev = int(min(16_000_000, max(200_000, 200_000 / dt * 0.3 * budget_s)))
    ev = E.raw_uniform(n_ev, seed=3)
    dt, s, _ = _stage01(stub_dir, ev, 6, base, sub, all_cores, W2, H2)
    res["stage01"] = {
        "events_per_s": round(n_ev / dt, 1), "events": n_ev, "seconds": round(dt, 3),
        "shards": 6, "halo": 2,
        "cores": (f"shards on {base}-{base + 5}, submit on {core0}" if pinned
                  else f"unpinned over {len(all_cores)} usable cores"),
        "pass_s0": int(s[2]), "pass_s1": int(s[13]),
        "segments": _segments(s, n_ev),
        "sample": f"{n_ev} raw uniform events, 80x64, 2 Mev/s timestamps, seed 3"}

    # the 50k-event CPU reference case, end to end on one core
    ev = E.raw_uniform(50_000, seed=1)
    t01, s, recs = _stage01(stub_dir, ev, 1, core0, [core0], all_cores, W2, H2, ring=True)
    _pin([core0])
    st = O.S2S3(layers, H2, W2, 4, head=head)
    t0 = time.perf_counter()
    p2, p3, _, _ = st.run(recs["x"], recs["y"], recs["feat1"], precision=32,
                          want_feat=False, want_head=True)
    t23 = time.perf_counter() - t0
    n_out = int((p3 == 1).sum())
    res["end_to_end"] = {
        "events_per_s": round(len(ev) / (t01 + t23), 1), "events": len(ev),
        "records": int(len(recs)), "output_producing": n_out,
        "output_kev_s": round(n_out / (t01 + t23) / 1e3, 4),
        "stage01_s": round(t01, 4), "s2s3_head_s": round(t23, 4), "cores": 1,
        "us_per_event": {"stage01": round(t01 / len(ev) * 1e6, 4),
                         "s2s3_head": round(t23 / len(ev) * 1e6, 4)},
        "segments": _segments(s, len(ev)),
        "sample": "50,000 raw uniform events at 80x64, 2 Mev/s, seed 1; one shard "
                  f"thread and the oracle on core {core0}"}
    _pin(all_cores)
    return res


# kernel of each timed launch of the whole-ring drain (ssla-rt_amd/csrc/drain_scan.hip)
PHASE_KERNEL = {"order": "ordering kernels", "head": "k_head + k_pred_*", "emit": "k_emit"}
for _L, (_i, _o) in zip(("L4", "L5", "L6", "L7"), ((C1, C2), (C2, C2), (C2, C3), (C3, C3))):
    PHASE_KERNEL[f"{_L}.proj"] = f"k_qvg<{_i}, {_o}>"
    # the recurrence is one launch (k_scan, in the apply slot); the sum slot
    # holds L4's wait for the s2 ticket order (L6's for the s3 one comes
    # before its projection), carry nothing
    PHASE_KERNEL[f"{_L}.sum"] = "(wait for k_group_order)" if _L == "L4" else "(none)"
    PHASE_KERNEL[f"{_L}.carry"] = "(none)"
    PHASE_KERNEL[f"{_L}.apply"] = f"k_scan<{_o}, {_o if _o == C2 else 2 * _o}>"
    PHASE_KERNEL[f"{_L}.out"] = f"k_outt<{_i}, {_o}>"
RIDGE = PEAK_FP32_TFLOPS * 1e12 / (PEAK_HBM_GBS * 1e9)     # FLOP/B


def _profile(name: str):
    f = ROOT / "profiles" / name
    if not f.exists():
        return None
    try:
        return json.loads(f.read_text())
    except ValueError:
        return None


def hbm_traffic(phase: str = None):
    """HBM bytes of the launch `phase` (None: of the whole call) from the
    committed rocprofv3 PMC summary (FETCH_SIZE x fetch scale + WRITE_SIZE x
    write scale, scales from a plain copy of known size), or None."""
    p = _profile("drain_80x64_200k_hbm_traffic.json")
    if p is None:
        return None
    if phase is None:
        return int(sum(v["hbm_bytes"] for v in p["launches"].values()))
    return p["launches"].get(phase, {}).get("hbm_bytes")


def trace_ms(phase: str):
    """Average duration (ms) of the launch `phase` in the committed
    rocprofv3 --kernel-trace summary of the same workload, or None."""
    p = _profile("drain_80x64_200k_kernel_trace.json")
    if p is None:
        return None
    v = p["launches"].get(phase)
    return None if v is None else v["avg_ms"]


def compulsory_bytes(x, y, p2, H2=16, W2=20):
    """HBM bytes a drain of these records cannot avoid, in the per-record
    accounting of the reference's kernel (state kept in HBM, read and
    written per patch): the 128 B record, the s2 hidden read-modify-write of
    L4 and L5 (n2 patches x 48 floats x 2 layers x read + write), that of L6
    and L7 for pass-2 records (n3 patches x 96 floats), the 392 B output
    slot and the two uint8 counters."""
    x = x.astype(np.int64)
    y = y.astype(np.int64)
    ok = (x < W2) & (y < H2)
    n2 = np.where(ok, inbounds(x, y, H2, W2), 0)
    n3 = np.where(ok & (p2 == 1), inbounds(x >> 1, y >> 1, H2 >> 1, W2 >> 1), 0)
    return float(x.size * (128 + 392 + 2) + n2.sum() * 48 * 4 * 2 * 2 + n3.sum() * 96 * 4 * 2 * 2)


def _per_batch(phase_us):
    """In-kernel wall-clock profile of the live kernel, per batch (µs)."""
    from ssla_hip import abi
    if phase_us is None or phase_us[25] <= 0:
        return None
    nb = float(phase_us[25])
    return {k: round(float(phase_us[i]) / nb, 2) for i, k in enumerate(abi.BATCH_PHASES)
            if k not in ("batches", "records") and (i < 25 or phase_us[i] > 0)}


def live_latency(stub_dir, rate_mev=2.0, duration_s=8.0, gpu_blocks=8, group=0, stages=1):
    from ssla_hip import live
    r = live.run_live(stub_dir, rate_mev=rate_mev, duration_s=duration_s, n_shards=6, halo=2,
                      gpu_blocks=gpu_blocks, group=group, stages=stages)
    lat = r.lat_us
    return {
        "p50": round(lat["emit_to_done_p50"], 2), "p99": round(lat["emit_to_done_p99"], 2),
        "max": round(lat["emit_to_done_max"], 2),
        "push_to_done_p50": round(lat["push_to_done_p50"], 2),
        "push_to_done_p99": round(lat["push_to_done_p99"], 2),
        "emit_to_push_p50": round(lat["emit_to_push_p50"], 2),
        "emit_to_push_p99": round(lat["emit_to_push_p99"], 2),
        "kernel_batch_p50": round(lat["kernel_p50"], 2),
        "mean_batch": round(r.batch_sizes.get("mean", 0.0), 2),
        "sustained_drain_kev_s": round(r.drain_rate_kev_s, 2),
        "output_kev_s": round(r.output_rate_kev_s, 3),
        "records": r.ring_records, "drained": r.drained, "kernel_status": r.status,
        "kernel_phase_us_per_batch": _per_batch(r.phase_us),
        "config": f"live: paced blob source {rate_mev} Mev/s -> 6 host shards (halo 2) -> "
                  + (f"{r.gpu_blocks} GPU blocks (owned s2 strips, halo 2), one fine-grained ring "
                     f"each" if r.gpu_blocks > 1 else "one ownership domain (the whole grid, no "
                     "halo), one fine-grained ring")
                  + (f", each drained by a group of {group} workgroups (16-channel slices, "
                     f"partial sums exchanged per layer)" if group > 1
                     else ", one persistent workgroup each")
                  + (" in two pipelined stages (L4-L5 of a batch beside L6-head of the "
                     "previous one, 2 groups per ring)" if stages == 2 else "")
                  + f", {r.duration_s:.1f} s; {r.synth_events} events emitted",
        "gpu_blocks": r.gpu_blocks, "group": group, "stages": stages,
    }


def halo_divergence(stub_dir, rec, n, p2o, p3o, feat_o, H2, W2, blocks=8):
    """The reference's multi-block live topology (owned s2 strips with a
    2-cell halo, orin/orin/multi_block.py:90-125) over the first n records,
    offline: each strip drains the records of its processed window in ring
    order with private state (whole-ring drain, `blocks` blocks in one call).
    Owned records see every record of their s2 and s3 cells in ring order,
    so their pass flags equal the single domain's; their s3_feat differs
    from the single-domain oracle's where a patch reaches cells beyond the
    halo -- the divergence the reference's max|d| <= 5.0 budget absorbs
    (orin/bench_s2_s3_head_celled.py:116)."""
    from ssla_hip import events as E
    from ssla_hip import hybrid as HY
    from ssla_hip.topology import grid_topology
    topo = grid_topology(blocks, W2, H2)
    x, y = rec.x[:n].astype(int), rec.y[:n].astype(int)
    full = E.to_records(rec)[:n]
    sels = [np.nonzero((x >= t.proc_x_lo) & (x < t.proc_x_hi) & (y >= t.proc_y_lo)
                       & (y < t.proc_y_hi))[0] for t in topo]
    with HY.Drain.from_weights_dir(stub_dir, n_blocks=len(topo),
                                   strips=[t.owned for t in topo]) as d:
        outs, _ = d.drain([full[s] for s in sels])
    flag_diff, worst, worst_rel, n_cmp, n_halo = 0, 0.0, 0.0, 0, 0
    for o, sel in zip(outs, sels):
        own = o["pass2"] != -1
        n_halo += int((~own).sum())
        g = sel[own]
        flag_diff += int((o["pass2"][own] != p2o[g]).sum() + (o["pass3"][own] != p3o[g]).sum())
        m = own & (o["pass3"] == 1)
        if m.any():
            ref = feat_o[sel[m]]
            dd = np.abs(o["s3_feat"][m] - ref)
            worst = max(worst, float(dd.max()))
            worst_rel = max(worst_rel, float(dd.max() / max(1e-12, np.abs(ref).max())))
            n_cmp += int(m.sum())
    return {"blocks": len(topo), "halo": 2, "records": int(n), "halo_copies": n_halo,
            "owned_flags_differ": flag_diff, "owned_pass3_compared": n_cmp,
            "s3_feat_max_abs_diff": round(worst, 4), "s3_feat_max_rel_diff": round(worst_rel, 4),
            "note": "owned records of the strip topology (the live leg's layout) against the "
                    "single-domain oracle over the same records; the reference reports 4.4 "
                    "for its 2-strip P1 split (budget 5.0)"}


def _roofline_phase(per):
    """The phase of the longest single-kernel launch (the ordering phase is
    several kernels, the head two)."""
    single = {k: v for k, v in per.items() if k not in ("order", "head")}
    return max(single, key=single.get)


def _roofline(per, flops, byts, iface, dom):
    kname = PHASE_KERNEL.get(dom, dom)
    traffic = hbm_traffic(dom)
    fl, by, ib = flops.get(dom, 0.0), byts.get(dom, 0.0), iface.get(dom, 0.0)
    base = {"kernel": f"{kname} ({dom})", "traffic": traffic, "avg_launch_ms": round(per[dom], 5),
            "algorithmic_bytes_per_launch": int(by), "algorithmic_flops_per_launch": int(fl),
            "interface_bytes_per_launch": int(ib),
            "interface_gbs": round(ib / (per[dom] * 1e-3) / 1e9, 1)}
    tr = trace_ms(dom)
    if by > 0 and fl / by < RIDGE:
        ach = by / (per[dom] * 1e-3) / 1e9
        r = dict(base, bound="hbm", achieved=round(ach, 2), peak=PEAK_HBM_GBS, unit="GB/s",
                 frac=round(ach / PEAK_HBM_GBS, 5))
        if tr:
            r["frac_kernel_trace"] = round(by / (tr * 1e-3) / 1e9 / PEAK_HBM_GBS, 5)
    else:
        ach = fl / (per[dom] * 1e-3) / 1e12
        r = dict(base, bound="mfma", achieved=round(ach, 4), peak=PEAK_FP32_TFLOPS,
                 unit="TFLOP/s", frac=round(ach / PEAK_FP32_TFLOPS, 5))
        if tr:
            r["frac_kernel_trace"] = round(fl / (tr * 1e-3) / 1e12 / PEAK_FP32_TFLOPS, 5)
    if tr:
        r["avg_launch_ms_kernel_trace"] = tr
    r["frac_note"] = ("frac: avg_launch_ms from HIP events around this launch on the drain's "
                      "stream over the timed steps; frac_kernel_trace: the launch's average "
                      "duration in the committed rocprofv3 --kernel-trace summary "
                      "(profiles/drain_80x64_200k_kernel_trace.json) of the same workload")
    return r


WORKLOADS = {
    "80x64": dict(height=64, width=80, streams=1, n=200_000, steps=20, warmup=3),
    "640x480": dict(height=480, width=640, streams=1, n=1_250_000, steps=5, warmup=1),
    "16streams": dict(height=64, width=80, streams=16, n=200_000, steps=5, warmup=1),
}


def replay_latency(stub_dir, recs, offline_p3, rate_per_stream=125_000.0, group=0, stages=1):
    """Live multi-stream run: each stream's ring records replayed at the
    2 Mev/s stream's record rate into its own ring of one persistent kernel
    (each ring drained by one workgroup, or by a group of `group`);
    push -> prediction latency per stream and drop drift against the same
    records' offline decisions."""
    from ssla_hip import events, live
    r = live.run_replay(stub_dir, [events.to_records(x) for x in recs], rate_per_stream,
                        timing_capacity=1 << 18, expect_p3=offline_p3, group=group,
                        stages=stages)
    st = r.streams
    p50 = [s["push_to_done_p50"] for s in st]
    p99 = [s["push_to_done_p99"] for s in st]
    return {
        "p50": round(float(np.median(p50)), 2), "p99": round(float(max(p99)), 2),
        "per_stream_p50": [round(v, 2) for v in p50], "per_stream_p99": [round(v, 2) for v in p99],
        "drop_drift_per_stream": [s["drop_drift"] for s in st],
        "aggregate_drain_kev_s": round(r.drained / r.duration_s / 1e3, 2),
        "kernel_status": r.status, "kernel_phase_us_per_batch": _per_batch(r.phase_us),
        "config": f"live: {len(recs)} rings replayed at {rate_per_stream:.0f} records/s each "
                  "(post-stage-1 records, published at emit) -> one persistent kernel, "
                  + (f"a group of {group} workgroups per stream" if group else
                     "one workgroup per stream")
                  + (" in two pipelined stages" if stages == 2 else "")
                  + "; latency push -> prediction",
        "group": group, "stages": stages,
    }


def split_replay_latency(stub_dir, rec, H2, W2, n_blocks=16, speed=1.0, group=0, stages=1):
    """Live run of one full-resolution stream split over owned strips (the
    reference's multi-block layout, 4 x 4 here): every strip's ring gets the
    records of its processed window (halo copies included), all rings
    replayed by the records' own times at `speed`; push -> prediction per
    strip and drop drift against each strip's own decision schedule (the
    whole-ring drain of the same strip rings)."""
    from ssla_hip import events, hybrid, live
    from ssla_hip.topology import grid_topology
    topo = grid_topology(n_blocks, W2, H2)
    full = events.to_records(rec)
    x, y = rec.x.astype(np.int64), rec.y.astype(np.int64)
    rings = []
    for t in topo:
        m = (x >= t.proc_x_lo) & (x < t.proc_x_hi) & (y >= t.proc_y_lo) & (y < t.proc_y_hi)
        rings.append(full[m])
    with hybrid.Drain.from_weights_dir(stub_dir, n_blocks=len(topo),
                                       strips=[t.owned for t in topo]) as d:
        d.drain(rings)
        outs, _ = d.results()
    expect = [(o["pass3"] == 1).astype(np.int8) for o in outs]
    cap = 1 << max(16, int(np.ceil(np.log2(max(r.size for r in rings) + 1))))
    r = live.run_replay(stub_dir, rings, 0.0, strips=[t.owned for t in topo], speed=speed,
                        timing_capacity=cap, expect_p3=expect, group=group, stages=stages)
    st = r.streams
    p50 = [s["push_to_done_p50"] for s in st]
    p99 = [s["push_to_done_p99"] for s in st]
    return {
        "p50": round(float(np.median(p50)), 2), "p99": round(float(max(p99)), 2),
        "per_strip_p50": [round(v, 2) for v in p50], "per_strip_p99": [round(v, 2) for v in p99],
        "drop_drift_per_strip": [s["drop_drift"] for s in st],
        "records_per_strip": [s["records"] for s in st],
        "aggregate_drain_kev_s": round(r.drained / r.duration_s / 1e3, 2),
        "kernel_status": r.status, "kernel_phase_us_per_batch": _per_batch(r.phase_us),
        "config": f"live: the full-resolution stream split into {n_blocks} owned strips "
                  f"({len(set(t.owned_x_lo for t in topo))} x {len(set(t.owned_y_lo for t in topo))}, "
                  "halo 2), each strip's records (halo copies included) replayed into its own "
                  f"ring by record time at {speed:g}x real time -> one persistent kernel, "
                  + (f"a group of {group} workgroups per strip" if group else
                     "one workgroup per strip")
                  + (" in two pipelined stages" if stages == 2 else "")
                  + "; latency push -> prediction",
        "group": group, "stages": stages,
    }


def batch_bench(a, d, recs, n, S, steps, warmup, desc, tmp) -> int:
    """Offline drain through the live kernel's batch loop (the persistent
    kernel's code path, fed from pre-filled rings)."""
    from ssla_hip import lib
    for _ in range(warmup):
        d.reset(sync=False)
        d.run(sync=True, batch=a.batch, group=a.batch_group)
    lib.check(lib.load().ssla_hip_device_synchronize())
    t0 = time.perf_counter()
    for _ in range(steps):
        d.reset(sync=False)
        d.run(sync=True, batch=a.batch, group=a.batch_group)
    lib.check(lib.load().ssla_hip_device_synchronize())
    dt = time.perf_counter() - t0
    outs, _ = d.results()
    n_out = sum(int((o["pass3"] == 1).sum()) for o in outs)
    d.close()
    tmp.cleanup()
    print(json.dumps({
        "metric": METRIC, "value": round(n_out * max(steps, 1) / dt / 1e3, 3) if steps else None,
        "unit": "kev/s", "n_gpus": 1, "steps": steps, "warmup": warmup,
        "ms_per_step": round(dt * 1e3 / steps, 4) if steps else None,
        "higher_is_better": True, "scaling": "weak", "vs_baseline": None, "dtype": "f32",
        "data": "synthetic",
        "config": {"workload": desc, "records": n * S, "instances": S,
                   "mode": f"in-kernel batches of {a.batch} (live kernel), "
                           + (f"a group of {a.batch_group} workgroups" if a.batch_group > 1
                              else "one workgroup") + " per instance",
                   "output_producing_per_step": n_out},
        "ring_record_kev_s": round(n * S * steps / dt / 1e3, 2) if steps else None}))
    return 0


# ---- rocprofv3 summaries (the files under profiles/ are made by these) ------
# whole-ring drain launches per call, in launch order, by kernel name; names
# launched twice per call belong to the two layers in turn; the ordering
# kernels are summed into "order"
TRAFFIC_PHASES = {
    "k_qvg<24, 48>": ["L4.proj"], "k_qvg<48, 48>": ["L5.proj"], "k_qvg<48, 96>": ["L6.proj"],
    "k_qvg<96, 96>": ["L7.proj"],
    "k_scan<48, 48>": ["L4.apply", "L5.apply"], "k_scan<96, 192>": ["L6.apply", "L7.apply"],
    "k_outt<24, 48, 2, 1>": ["L4.out"], "k_outt<48, 48, 1, 3>": ["L5.out"],
    "k_outt<48, 96, 1, 3>": ["L6.out"], "k_outt<96, 96, 1, 3>": ["L7.out"],
    "k_head": ["head"], "k_head_linear": ["head"], "k_pred_write": ["head"], "k_emit": ["emit"],
}
ORDER_KERNELS = ("k_decode", "k_rs_hist", "k_exscan", "k_rs_scatter", "k_runs", "k_keys2",
                 "k_keyscan", "k_s2_tables", "k_pair_rank", "k_chunks", "k_keys3a", "k_place3",
                 "k_tdrop3", "k_keys3b", "k_group_order")


def _traffic_key(k: str):
    """The TRAFFIC_PHASES key of kernel name k: the key itself, or a key
    whose template arguments are the first arguments of k's (the launch
    parameters that follow them -- tile sizes, waves per SIMD, row strides --
    do not change the phase)."""
    for key in TRAFFIC_PHASES:
        base = key[:-1]
        if k == key or (key.endswith(">") and k.startswith(base) and k[len(base)] in ",>"):
            return key
    return None


def _kname(n: str) -> str:
    m = n.replace("ssla::(anonymous namespace)::", "").replace("ssla::", "").replace("void ", "")
    m = re.sub(r"\(.*", "", m).strip()
    return m or n.strip() or "(unnamed)"


def pmc_summary(fetch_dir, write_dir, cfetch_dir, cwrite_dir, copy_bytes, command):
    """Per-launch HBM bytes of the whole-ring drain from rocprofv3 --pmc
    FETCH_SIZE / WRITE_SIZE runs of bench.py (counters in KiB per dispatch),
    each scaled by what the same counter reads for a plain device copy of
    copy_bytes bytes (cfetch / cwrite runs)."""
    import collections
    import csv
    import glob

    def rows(d):
        f = glob.glob(f"{d}/**/*counter_collection.csv", recursive=True)[0]
        return sorted(csv.DictReader(open(f)), key=lambda r: int(r["Dispatch_Id"]))

    def per_phase(rs):
        seen, out = collections.Counter(), collections.defaultdict(float)
        calls = sum(1 for r in rs if _kname(r["Kernel_Name"]) == "k_decode")
        for r in rs:
            k = _kname(r["Kernel_Name"])
            v = float(r["Counter_Value"]) * 1024.0
            key = _traffic_key(k)
            if k.split("<")[0] in ORDER_KERNELS:
                out["order"] += v / max(1, calls)
            elif key is not None:
                ph = TRAFFIC_PHASES[key]
                out[ph[seen[key] % len(ph)]] += v / max(1, calls)
                seen[key] += 1
        return out

    cf = max(float(r["Counter_Value"]) for r in rows(cfetch_dir)) * 1024.0
    cw = max(float(r["Counter_Value"]) for r in rows(cwrite_dir)) * 1024.0
    fs, ws = copy_bytes / cf, copy_bytes / cw
    fetch, write = per_phase(rows(fetch_dir)), per_phase(rows(write_dir))
    res = {"copy_bytes": copy_bytes, "fetch_scale": round(fs, 4), "write_scale": round(ws, 4),
           "command": command,
           "workload": "bench.py defaults: 200,000 ring records at 80x64, stub weights seed 1",
           "launches": {}}
    for ph in sorted(set(fetch) | set(write)):
        f, w = fetch.get(ph, 0.0) * fs, write.get(ph, 0.0) * ws
        res["launches"][ph] = {"fetch_bytes": int(f), "write_bytes": int(w),
                               "hbm_bytes": int(f + w)}
    return res


def trace_summary(trace_dir, command):
    """Per-launch average durations of the whole-ring drain from a rocprofv3
    --kernel-trace run of bench.py (kernel_trace.csv), with the kernel ->
    launch mapping of the PMC summary (a kernel launched twice per call
    belongs to its two layers in turn)."""
    import collections
    import csv
    import glob
    f = glob.glob(f"{trace_dir}/**/*kernel_trace.csv", recursive=True)[0]
    rs = sorted(csv.DictReader(open(f)), key=lambda r: int(r["Dispatch_Id"]))
    seen, tot, cnt = collections.Counter(), collections.defaultdict(float), collections.Counter()
    for r in rs:
        k = _kname(r["Kernel_Name"])
        key = _traffic_key(k)
        if key is None or k.split("<")[0] in ORDER_KERNELS:
            continue
        ph = TRAFFIC_PHASES[key]
        lab = ph[seen[key] % len(ph)]
        if lab == "head":                         # two kernels: kept apart
            lab += ":" + k.split("<")[0]
        seen[key] += 1
        tot[lab] += (int(r["End_Timestamp"]) - int(r["Start_Timestamp"])) * 1e-6
        cnt[lab] += 1
    return {"command": command,
            "workload": "bench.py defaults: 200,000 ring records at 80x64, stub weights seed 1",
            "launches": {k: {"launches": cnt[k], "avg_ms": round(tot[k] / cnt[k], 5)}
                         for k in sorted(tot)}}


def stats_summary(csv_path, title, workload, command, calls_note, top=30):
    """Markdown table of a rocprofv3 --kernel-trace --stats kernel_stats.csv."""
    import csv
    rs = list(csv.DictReader(open(csv_path)))
    tot = sum(float(r["TotalDurationNs"]) for r in rs)
    out = [f"# {title}", "", f"Workload: {workload}", "",
           "Command (repo root on the MI355X box; `cd /tmp && export TMPDIR=/tmp` first):", "",
           "```", command, "```", "",
           f"## Kernel stats ({calls_note}; top {top} by total time)", "",
           "| kernel | calls | avg µs | % of GPU time |", "|---|---:|---:|---:|"]
    for r in sorted(rs, key=lambda r: -float(r["TotalDurationNs"]))[:top]:
        out.append(f"| {_kname(r['Name'])} | {r['Calls']} | {float(r['AverageNs']) / 1e3:.1f} | "
                   f"{float(r['Percentage']):.2f} |")
    out += ["", f"Total kernel time: {tot / 1e6:.2f} ms over "
                f"{sum(int(r['Calls']) for r in rs)} launches."]
    return "\n".join(out)


def sq_summary(dir_a, dir_b, xcc=8, cus=256, slots=32, ghz=2.4):
    """Per-kernel SQ metrics (markdown) from the two rocprofv3 --pmc passes
    listed in profiles/drain_80x64_200k_sq_counters.md, summed over each
    kernel's launches, with rocprofv3's metric formulas.  GRBM_GUI_ACTIVE is
    summed over the XCDs, so it is divided by their number."""
    import collections
    import csv
    import glob

    def load(d):
        f = glob.glob(f"{d}/**/*counter_collection.csv", recursive=True)[0]
        out = collections.OrderedDict()
        for r in csv.DictReader(open(f)):
            e = out.setdefault(int(r["Dispatch_Id"]), {
                "name": _kname(r["Kernel_Name"]), "lds": int(r["LDS_Block_Size"]),
                "vgpr": int(r["VGPR_Count"]), "agpr": int(r["Accum_VGPR_Count"])})
            e[r["Counter_Name"]] = float(r["Counter_Value"])
        return out

    A, B = load(dir_a), load(dir_b)
    agg = collections.OrderedDict()
    for k, e in A.items():
        g = agg.setdefault(e["name"], collections.Counter())
        g["n"] += 1
        for c, v in e.items():
            if isinstance(v, float):
                g["A_" + c] += v
        for c, v in B.get(k, {}).items():
            if isinstance(v, float):
                g["B_" + c] += v
        g["vgpr"], g["agpr"], g["lds"] = e["vgpr"], e["agpr"], e["lds"]
    simds = 4 * cus
    rows = ["| kernel | launches | µs/launch | occupancy % | VALU busy % | MFMA busy % | "
            "LDS busy % | LDS bank conflicts / access | wave time waiting % | "
            "VALU / MFMA / LDS / VMEM-rd / VMEM-wr instr per wave | VGPR + AGPR | LDS B |",
            "|---|---:|---:|---:|---:|---:|---:|---:|---:|---|---:|---:|"]
    for nm, g in sorted(agg.items(), key=lambda kv: -kv[1]["A_GRBM_GUI_ACTIVE"]):
        grbm = g["A_GRBM_GUI_ACTIVE"] / xcc
        if grbm <= 0:
            continue
        occ = 400 * g["A_SQ_WAVE_CYCLES"] / grbm / cus / slots   # WAVE_CYCLES: units of 4
        valu = 100 * g["A_SQ_ACTIVE_INST_VALU"] / cus / grbm
        mfma = 100 * g["A_SQ_VALU_MFMA_BUSY_CYCLES"] / (grbm * simds)
        lds = 100 * g["A_SQ_LDS_IDX_ACTIVE"] / (grbm * cus)
        conf = g["A_SQ_LDS_BANK_CONFLICT"] / max(1.0, g["A_SQ_LDS_IDX_ACTIVE"]
                                                  - g["A_SQ_LDS_BANK_CONFLICT"])
        wait = 100 * g["B_SQ_WAIT_ANY"] / max(1.0, g["B_SQ_WAVE_CYCLES"] or g["A_SQ_WAVE_CYCLES"])
        w = max(1.0, g["B_SQ_WAVES"] or g["A_SQ_WAVES"])
        ins = "/".join(str(int(g["B_SQ_INSTS_" + x] / w))
                       for x in ("VALU", "MFMA", "LDS", "VMEM_RD", "VMEM_WR"))
        rows.append(f"| `{nm}` | {g['n']} | {grbm / g['n'] / (ghz * 1e3):.1f} | {occ:.1f} | "
                    f"{valu:.1f} | {mfma:.1f} | {lds:.1f} | {conf:.3f} | {wait:.1f} | {ins} | "
                    f"{g['vgpr']} + {g['agpr']} | {g['lds']} |")
    return "\n".join(rows)


def main() -> int:
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=None)
    ap.add_argument("--warmup", type=int, default=None)
    ap.add_argument("--n", type=int, default=None, help="ring records per stream")
    ap.add_argument("--workload", choices=sorted(WORKLOADS), default="80x64",
                    help="80x64: the offline-drain configuration (+ live latency); 640x480: "
                         "one second of the 20 Mev/s full-resolution stream; 16streams: 16 "
                         "independent 80x64 instances in one call")
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--cpu-seconds", type=float, default=15.0)
    ap.add_argument("--no-live", action="store_true", help="skip the live latency run")
    ap.add_argument("--live-seconds", type=float, default=8.0)
    ap.add_argument("--live-rate", type=float, default=2.0,
                    help="raw event rate of the live run's synthetic source, Mev/s")
    ap.add_argument("--live-blocks", type=int, default=1, choices=[1, 2, 4, 8, 16],
                    help="GPU blocks (owned strips) of the live run; 1 = one ownership domain")
    ap.add_argument("--live-group", type=int, default=6, choices=[0, 3, 4, 5, 6],
                    help="workgroups per block of the live run (0 = one)")
    ap.add_argument("--live-stages", type=int, default=None, choices=[1, 2],
                    help="2: two groups per block in a pipeline (L4-L5 of a batch beside "
                         "L6-head of the previous one); default 2 for the 80x64 live legs, "
                         "1 for the 16-ring ones (16 streams, 640x480 strips), as measured "
                         "fastest")
    ap.add_argument("--no-live-strips", action="store_true",
                    help="skip the second live run on the reference's 8-strip topology "
                         "(2 x 4 owned strips, halo 2, each drained by --live-group workgroups)")
    ap.add_argument("--batch", type=int, default=0,
                    help="1..32: drain through the live kernel's in-kernel batches of this "
                         "many records (one workgroup per instance) instead of the whole-ring "
                         "drain; reports throughput only")
    ap.add_argument("--batch-group", type=int, default=0, choices=[0, 3, 4, 5, 6],
                    help="with --batch: drain each instance with a group of this many "
                         "workgroups (channel slices; 0 = one workgroup)")
    ap.add_argument("--pmc-summary", nargs=4, metavar=("FETCH", "WRITE", "CFETCH", "CWRITE"),
                    help="print the per-launch HBM traffic JSON from rocprofv3 --pmc output "
                         "directories (drain FETCH_SIZE, WRITE_SIZE, copy FETCH_SIZE, WRITE_SIZE)")
    ap.add_argument("--copy-bytes", type=int, default=256 << 20)
    ap.add_argument("--stats-summary", nargs=5,
                    metavar=("CSV", "TITLE", "WORKLOAD", "COMMAND", "CALLS"),
                    help="print a markdown table of a rocprofv3 kernel_stats.csv")
    ap.add_argument("--trace-summary", metavar="TRACE_DIR",
                    help="print per-launch average durations (JSON) from a rocprofv3 "
                         "--kernel-trace output directory of bench.py")
    ap.add_argument("--sq-summary", nargs=2, metavar=("PASS_A", "PASS_B"),
                    help="print per-kernel SQ metrics from the two rocprofv3 --pmc passes")
    a = ap.parse_args()
    if a.trace_summary:
        print(json.dumps(trace_summary(a.trace_summary,
                                       "rocprofv3 --kernel-trace --stats -f csv -d <dir> -- python3 "
                                       "bench.py --steps 5 --warmup 1 --no-live --no-cpu-baseline"),
                         indent=1))
        return 0
    if a.sq_summary:
        print(sq_summary(*a.sq_summary))
        return 0
    if a.pmc_summary:
        print(json.dumps(pmc_summary(*a.pmc_summary, a.copy_bytes,
                                     "rocprofv3 --pmc FETCH_SIZE (then WRITE_SIZE) -f csv -d <dir> "
                                     "-- python3 bench.py --steps 2 --warmup 1 --no-live "
                                     "--no-cpu-baseline"), indent=1))
        return 0
    if a.stats_summary:
        print(stats_summary(*a.stats_summary))
        return 0
    if not 0 <= a.batch <= 32:
        print("bench.py: --batch must be 0..32", file=sys.stderr)
        return 2
    if a.gpus != 1 or int(os.environ.get("WORLD_SIZE", "1")) > 1:
        print("bench.py: this build measures one GPU only (one drain instance set per "
              "device, no collectives); run with --gpus 1", file=sys.stderr)
        return 2
    wl = WORKLOADS[a.workload]
    n = a.n or wl["n"]
    steps = a.steps if a.steps is not None else wl["steps"]
    warmup = a.warmup if a.warmup is not None else wl["warmup"]
    H0, W0, S = wl["height"], wl["width"], wl["streams"]
    H2, W2 = H0 // 4, W0 // 4

    from ssla_hip import abi, events, hybrid, lib, stub
    lib.load()
    lib.check_layout()
    tmp = tempfile.TemporaryDirectory()
    stub.write_stub(tmp.name, height=H0, width=W0, seed=1, tdrop=4)
    if a.workload == "640x480":
        recs = [events.edge_blob_records(n, seed=1)]
        desc = (f"offline drain of {n} ring records at 640x480 (s2 160x120): 64 moving edge "
                "blobs + 5% hot pixels (1% of pixels), one second of the 20 Mev/s stream")
    else:
        recs = [events.blob_records(n, seed=1 + s, height=H0, width=W0) for s in range(S)]
        desc = (f"offline drain of {n} ring records at 80x64 (s2 20x16): 8 moving "
                "Gaussian blobs + 10% background")
        if S > 1:
            desc = f"{S} independent instances (stream seeds 1..{S}), each an " + desc
    desc += ", stub weights seed 1, tdrop 4"

    d = hybrid.Drain.from_weights_dir(tmp.name, n_blocks=S)
    d.load_rings([events.to_records(r) for r in recs], want_head=True)
    if a.batch:
        return batch_bench(a, d, recs, n, S, steps, warmup, desc, tmp)
    nph = len(abi.DRAIN_PHASES)
    for _ in range(warmup):
        d.reset(sync=False)
        d.run(sync=True)
    outs, heads = d.results()
    n_out = sum(int((o["pass3"] == 1).sum()) for o in outs)

    # Per-phase split: the same steps with HIP events at every phase boundary
    # (each event adds a few us of queue time, so this loop is not the timed
    # one); it also names the phase of the longest single launch.
    phase = np.zeros(nph, np.float32)
    for _ in range(steps):
        d.reset(sync=False)
        d.run(sync=True, phase_ms=phase)
    per = {k: float(v) / steps for k, v in zip(abi.DRAIN_PHASES, phase)}
    roof_phase = _roofline_phase(per)
    # Timed steps: events only around the roofline kernel's launch.
    rphase = np.zeros(nph, np.float32)
    mask = 1 << abi.DRAIN_PHASES.index(roof_phase)
    # The steps are queued back to back (the host prepares step k + 1 while
    # the GPU runs step k); the last call waits, and its return adds the
    # queued calls' event times to rphase.
    lib.check(lib.load().ssla_hip_device_synchronize())
    t0 = time.perf_counter()
    for i in range(steps):
        d.reset(sync=False)
        d.run(sync=i == steps - 1, phase_ms=rphase, phase_mask=mask)
    lib.check(lib.load().ssla_hip_device_synchronize())
    dt = time.perf_counter() - t0
    outs2, _ = d.results()
    assert sum(int((o["pass3"] == 1).sum()) for o in outs2) == n_out, \
        "steps did not repeat identical work"
    per_timed = dict(per)
    per_timed[roof_phase] = float(rphase[abi.DRAIN_PHASES.index(roof_phase)]) / steps

    ms_step = dt * 1e3 / steps
    value = n_out * steps / dt / 1e3
    ring_rate = n * S * steps / dt / 1e3
    flops, byts, ibyts, total_mac = {}, {}, {}, 0
    for r, o in zip(recs, outs):
        f_, b_, i_, m_ = algorithmic_work(r.x, r.y, o["pass2"], o["pass3"], np.ones(n, np.int32),
                                          H2, W2)
        for src, dst in ((f_, flops), (b_, byts), (i_, ibyts)):
            for k, v in src.items():
                dst[k] = dst.get(k, 0.0) + v
        total_mac += m_
    roof = _roofline(per_timed, flops, byts, ibyts, roof_phase)
    if a.workload != "80x64":
        roof["traffic"] = None           # the committed PMC summary is of the 80x64 workload
    if roof.get("unit") == "GB/s":
        # what this device reaches on write-dominated traffic (the published
        # 8 TB/s counts read and write capacity together)
        ceil = (ctypes.c_double * 3)()
        probe = ctypes.CDLL(str(ROOT / "ssla-rt_amd" / "libssla_probe.so"))
        probe.ssla_probe_hbm_ceiling.argtypes = [ctypes.POINTER(ctypes.c_double), ctypes.c_int]
        probe.ssla_probe_last_error.restype = ctypes.c_char_p
        if probe.ssla_probe_hbm_ceiling(ceil, 3) != 0:
            raise RuntimeError("hbm probe: " + probe.ssla_probe_last_error().decode())
        roof["measured_ceiling_gbs"] = {"write_stream": round(ceil[0], 1),
                                        "copy_read_write": round(ceil[1], 1),
                                        "rows_576B_permuted": round(ceil[2], 1)}
        # the launch's interface traffic (rows included) against those ceilings
        roof["interface_frac_of_write_ceiling"] = round(roof["interface_gbs"] / ceil[0], 4)
    roof["bytes_note"] = ("achieved / frac: the algorithmic bytes or FLOPs of the launch (for a "
                          "recurrence, each pair's hidden-state read and write); interface_*: "
                          "the bytes it moves at its interface, which include this design's "
                          "own pair rows and h rows; traffic: the committed PMC measurement")
    whole = 2.0 * total_mac / (ms_step * 1e-3) / 1e12
    iface = sum(ibyts.values())
    comp = sum(compulsory_bytes(r.x, r.y, o["pass2"], H2, W2) for r, o in zip(recs, outs))
    measured = hbm_traffic() if a.workload == "80x64" else None
    res = {
        "metric": METRIC, "value": round(value, 3), "unit": "kev/s", "n_gpus": 1,
        "steps": steps, "warmup": warmup, "ms_per_step": round(ms_step, 4),
        "higher_is_better": True, "scaling": "weak", "vs_baseline": None, "dtype": "f32",
        "data": "synthetic",
        "config": {"workload": desc, "records": n * S, "instances": S,
                   "output_producing_per_step": n_out},
        "ring_record_kev_s": round(ring_rate, 2),
        "latency_us": None,
        "whole_drain_tflops": round(whole, 4),
        # HBM bytes per call: the compulsory ones (records, hidden-state RMW
        # per patch, output slots, counters) against what rocprofv3 measured
        # for this build (committed PMC summary; 80x64 workload only)
        "compulsory_hbm_bytes": int(comp),
        "measured_hbm_bytes": measured,
        "measured_over_compulsory": round(measured / comp, 3) if measured else None,
        "whole_drain_compulsory_hbm_gbs": round(comp / (ms_step * 1e-3) / 1e9, 1),
        # the bytes every launch moves at its interface, including the design's
        # own intermediates (pair rows, h rows, chunk maps): not compulsory
        "whole_drain_launch_interface_gbs": round(iface / (ms_step * 1e-3) / 1e9, 1),
        "phase_ms": {k: round(v, 5) for k, v in per.items()},
        "phase_ms_note": "HIP-event time per phase from an extra loop of the same steps with "
                         "events at every phase boundary (each adds a few us of queue time); "
                         "the timed loop records events around the roofline kernel only",
        "roofline": roof,
        # every single-kernel phase against its own bound, from the per-phase
        # loop's event times (these include a few us of queue time each)
        "roofline_by_phase_note": "per launch against its bound, on its algorithmic bytes or "
                                  "FLOPs; interface_gbs: the rate on the bytes it moves at its "
                                  "interface, which include the design's own intermediates "
                                  "(pair rows, h rows)",
        "roofline_by_phase": {
            k: {x: r[x] for x in ("bound", "achieved", "unit", "frac", "interface_gbs")}
            for k, r in ((k, _roofline(per, flops, byts, ibyts, k)) for k in per
                         if k not in ("order", "head") and per[k] > 0
                         and (flops.get(k, 0.0) > 0 or byts.get(k, 0.0) > 0))},
    }
    d.close()
    # The latency and CPU legs run after the timed drain; a failure in one is
    # reported in its field and in the exit status, after the line is printed.
    failed = []

    def leg(name, fn):
        try:
            return fn()
        except Exception as e:            # noqa: BLE001 - reported, not hidden
            failed.append(name)
            print(f"bench.py: {name} failed: {e!r}", file=sys.stderr)
            return {"error": f"{type(e).__name__}: {e}"}

    if a.live_stages is None:
        a.live_stages = 2 if a.workload == "80x64" and a.live_group > 1 else 1
    if a.workload == "80x64" and not a.no_live:
        res["latency_us"] = leg("live", lambda: live_latency(tmp.name, a.live_rate,
                                                             a.live_seconds, a.live_blocks,
                                                             a.live_group, a.live_stages))
        if not a.no_live_strips:
            res["latency_us_8_strips"] = leg("live 8 strips", lambda: live_latency(
                tmp.name, a.live_rate, a.live_seconds, 8, a.live_group, a.live_stages))
    if a.workload == "16streams" and not a.no_live:
        res["latency_us"] = leg("replay", lambda: replay_latency(
            tmp.name, recs, [o["pass3"] for o in outs], group=a.live_group,
            stages=a.live_stages))
    if a.workload == "640x480" and not a.no_live:
        res["latency_us"] = leg("split replay", lambda: split_replay_latency(
            tmp.name, recs[0], H2, W2, group=a.live_group, stages=a.live_stages))
    if not a.no_cpu_baseline:
        res["cpu_baseline"] = leg("cpu baseline", lambda: cpu_baseline(
            tmp.name, recs[0], a.cpu_seconds, H2, W2, (outs[0], heads[0])))
        orc = res["cpu_baseline"].pop("_oracle", None)
        if orc is not None and a.workload == "80x64":
            res["halo_topology_vs_single_domain"] = leg("halo topology", lambda: halo_divergence(
                tmp.name, recs[0], orc[0], orc[1], orc[2], orc[3], H2, W2))
    tmp.cleanup()
    print(json.dumps(res))
    return 1 if failed else 0


if __name__ == "__main__":
    sys.exit(main())
