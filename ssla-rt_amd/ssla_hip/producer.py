"""ctypes bindings of the host producer libraries.

`S01gAPI` binds libstage01_to_gpu.so with the method names and argument
meaning of the reference driver's wrapper (orin/orin/hybrid_common.py:468-605),
so a driver written against it runs unchanged; `S0API` binds
libstage01_capi.so (the stage 0 + 1 shards without rings,
orin/legacy/live_stage01_bench.py:66-90).

Both libraries are plain host code; they are built in-tree next to
libssla_hip.so and loading fails loudly when they are missing.
"""
from __future__ import annotations

import ctypes
import os
import time
from pathlib import Path
from typing import Optional, Sequence

import numpy as np

PKG_ROOT = Path(__file__).resolve().parent.parent
TO_GPU_PATH = PKG_ROOT / "libstage01_to_gpu.so"
CAPI_PATH = PKG_ROOT / "libstage01_capi.so"

N_STATS = 32
SEGMENTS = ("preprocess", "s0", "tdrop0", "s1", "tdrop1", "push")

_vp, _i, _d, _u64 = ctypes.c_void_p, ctypes.c_int, ctypes.c_double, ctypes.c_uint64
_fptr = ctypes.POINTER(ctypes.c_float)
_dptr = ctypes.POINTER(ctypes.c_double)
_vpp = ctypes.POINTER(ctypes.c_void_p)
_ip = ctypes.POINTER(ctypes.c_int)

_TO_GPU_SIGNATURES = {
    "s01g_init": (_vp, [ctypes.c_char_p, _i, _i, _i, _i]),
    "s01g_init_full": (_vp, [ctypes.c_char_p, _i, _i, _i, _i, ctypes.c_uint]),
    "s01g_attach_gpu_rings": (None, [_vp, _vp, _vp, _vp, _vp, _u64, _i, _i, _i, _i, _i, _i]),
    "s01g_attach_gpu_rings_multi": (None, [_vp, _i, _vpp, _vpp, _u64, _i, _i, _ip, _ip, _ip, _ip]),
    "s01g_set_ring_tails": (None, [_vp, _i, _vpp, _u64]),
    "s01g_submit_batch": (_i, [_vp, _fptr, _i]),
    "s01g_snapshot_stats": (None, [_vp, _dptr]),
    "s01g_reset_stats": (None, [_vp]),
    "s01g_shutdown": (None, [_vp]),
    "s01g_start_synthetic": (None, [_vp, _d, _i, _u64]),
    "s01g_stop_synthetic": (None, [_vp]),
    "s01g_synthetic_n_pushed": (_u64, [_vp]),
    "s01g_start_synthetic_blobs": (None, [_vp, _d, _i, _u64, _i, _d, _d]),
    "s01g_replay_start": (_vp, [_i, _vpp, _vpp, _u64, _vpp, _ip, _d, _i]),
    "s01g_replay_start_timed": (_vp, [_i, _vpp, _vpp, _u64, _vpp, _ip, _d, _i]),
    "s01g_replay_done": (_i, [_vp]),
    "s01g_replay_published": (_u64, [_vp]),
    "s01g_replay_stop": (None, [_vp]),
}

_CAPI_SIGNATURES = {
    "s0_init": (_vp, [ctypes.c_char_p, _i, _i, _i, _i]),
    "s0_submit_batch": (_i, [_vp, _fptr, _i]),
    "s0_snapshot_stats": (None, [_vp, _dptr]),
    "s0_reset_stats": (None, [_vp]),
    "s0_shutdown": (None, [_vp]),
}

EXPORTED_TO_GPU = tuple(_TO_GPU_SIGNATURES)
EXPORTED_CAPI = tuple(_CAPI_SIGNATURES)

_libs: dict = {}


def _load(path: Path, sigs: dict) -> ctypes.CDLL:
    key = str(path)
    if key in _libs:
        return _libs[key]
    if not path.exists():
        raise RuntimeError(f"{path.name} is not built; run `make -C {PKG_ROOT}`")
    lib = ctypes.CDLL(key)
    for name, (res, args) in sigs.items():
        f = getattr(lib, name)
        f.restype, f.argtypes = res, args
    _libs[key] = lib
    return lib


def load_to_gpu(path: Optional[os.PathLike] = None) -> ctypes.CDLL:
    return _load(Path(path) if path else TO_GPU_PATH, _TO_GPU_SIGNATURES)


def load_capi(path: Optional[os.PathLike] = None) -> ctypes.CDLL:
    return _load(Path(path) if path else CAPI_PATH, _CAPI_SIGNATURES)


def events_array(t, x, y, p) -> np.ndarray:
    """Packed (n, 4) float32 [t_us, x, y, p] as s01g_submit_batch takes it."""
    ev = np.empty((len(t), 4), np.float32)
    ev[:, 0], ev[:, 1], ev[:, 2], ev[:, 3] = t, x, y, p
    return ev


def routing(x, W: int, n_shards: int, halo: int):
    """Owner shard and halo deliveries of each in-sensor event.

    Strips are ceil(W / N) wide; the owner is min(x // strip, N - 1); a shard
    k also receives the event when x lies in [k*strip - halo, (k+1)*strip +
    halo) (lib_stage01_to_gpu.cpp:504-538).  Returns (owner (n,), halo_to
    list of (event index, shard))."""
    x = np.asarray(x, np.int64)
    strip = (W + n_shards - 1) // n_shards
    home = x // strip
    owner = np.minimum(home, n_shards - 1)
    halo_to = []
    for dk in (-1, 0, 1):
        k = home + dk
        ok = (k >= 0) & (k < n_shards) & (k != owner)
        ok &= (x >= k * strip - halo) & (x < (k + 1) * strip + halo)
        for i in np.nonzero(ok)[0]:
            halo_to.append((int(i), int(k[i])))
    return owner, halo_to


def halo_count(x, W: int, n_shards: int, halo: int) -> int:
    """len(routing(x, W, n_shards, halo)[1]), without building the list."""
    x = np.asarray(x, np.int64)
    strip = (W + n_shards - 1) // n_shards
    home = x // strip
    owner = np.minimum(home, n_shards - 1)
    n = 0
    for dk in (-1, 0, 1):
        k = home + dk
        ok = (k >= 0) & (k < n_shards) & (k != owner)
        ok &= (x >= k * strip - halo) & (x < (k + 1) * strip + halo)
        n += int(ok.sum())
    return n


class S01gAPI:
    """One libstage01_to_gpu.so handle (hybrid_common.py:468-605)."""

    def __init__(self, lib_path: Optional[os.PathLike] = None):
        self.lib = load_to_gpu(lib_path)
        self.handle = None
        self._attach_keepalive = None

    def init(self, weights_dir: str, n_shards: int, halo: int, base_core: int,
             sample_cap: int, shard_ring_cap: int = 1 << 16):
        self.handle = self.lib.s01g_init_full(str(weights_dir).encode(), n_shards, halo,
                                              base_core, sample_cap, shard_ring_cap)
        if not self.handle:
            raise RuntimeError("s01g_init returned NULL (check weights_dir / meta.json)")

    def attach(self, ring_buf_0, ring_head_0, ring_buf_1, ring_head_1, ring_mask, W2, H2,
               proc_lo_0, proc_hi_0, proc_lo_1, proc_hi_1):
        self.lib.s01g_attach_gpu_rings(self.handle, int(ring_buf_0), int(ring_head_0),
                                       int(ring_buf_1), int(ring_head_1), ring_mask, W2, H2,
                                       proc_lo_0, proc_hi_0, proc_lo_1, proc_hi_1)

    def attach_multi(self, ring_bufs: Sequence[int], ring_heads: Sequence[int], ring_mask: int,
                     W2: int, H2: int, proc_x_los, proc_x_his, proc_y_los, proc_y_his):
        n = len(ring_bufs)
        if not all(len(a) == n for a in (ring_heads, proc_x_los, proc_x_his, proc_y_los, proc_y_his)):
            raise ValueError("attach_multi: per-ring argument lengths differ")
        bufs = (ctypes.c_void_p * n)(*[int(p) for p in ring_bufs])
        heads = (ctypes.c_void_p * n)(*[int(p) for p in ring_heads])
        arrs = [(ctypes.c_int * n)(*[int(v) for v in a])
                for a in (proc_x_los, proc_x_his, proc_y_los, proc_y_his)]
        self._attach_keepalive = (bufs, heads, arrs)
        self.lib.s01g_attach_gpu_rings_multi(self.handle, n, bufs, heads, ring_mask, W2, H2, *arrs)

    def set_ring_tails(self, tail_ptrs: Sequence[int], timeout_ms: float = 1000.0) -> None:
        """Back-pressure: publishers wait (up to timeout_ms) for each ring's
        consumer tail (addresses of u64 words) to free a claimed slot.  An
        empty sequence turns it off."""
        n = len(tail_ptrs)
        arr = (ctypes.c_void_p * max(1, n))(*[int(p) for p in tail_ptrs])
        self._tails_keepalive = arr
        self.lib.s01g_set_ring_tails(self.handle, n, arr if n else None,
                                     int(timeout_ms * 1e6))

    def submit(self, events: np.ndarray) -> int:
        ev = np.ascontiguousarray(events, np.float32)
        if ev.shape[0] == 0:
            return 0
        return self.lib.s01g_submit_batch(self.handle, ev.ctypes.data_as(_fptr), ev.shape[0])

    def stats(self) -> list:
        out = (ctypes.c_double * N_STATS)()
        self.lib.s01g_snapshot_stats(self.handle, out)
        return list(out)

    def reset(self) -> None:
        self.lib.s01g_reset_stats(self.handle)

    def start_synthetic(self, rate_mev: float, pin_core: int, seed: int) -> None:
        self.lib.s01g_start_synthetic(self.handle, rate_mev, pin_core, seed)

    def start_synthetic_blobs(self, rate_mev: float, pin_core: int, seed: int, n_blobs: int = 4,
                              sigma_px: float = 3.0, bg_frac: float = 0.1) -> None:
        self.lib.s01g_start_synthetic_blobs(self.handle, rate_mev, pin_core, seed, n_blobs,
                                            sigma_px, bg_frac)

    def stop_synthetic(self) -> None:
        self.lib.s01g_stop_synthetic(self.handle)

    def synthetic_n_pushed(self) -> int:
        return int(self.lib.s01g_synthetic_n_pushed(self.handle))

    def wait_processed(self, n_owner: int, n_halo: int, timeout_s: float = 60.0) -> list:
        """Poll the stats until the shards have finished n_owner owner and
        n_halo halo events; returns the final stats."""
        t_end = time.monotonic() + timeout_s
        while True:
            s = self.stats()
            if s[0] >= n_owner and s[1] >= n_halo:
                return s
            if time.monotonic() > t_end:
                raise TimeoutError(f"producer processed {s[0]:.0f}/{n_owner} owner and "
                                   f"{s[1]:.0f}/{n_halo} halo events")
            time.sleep(0.001)

    def shutdown(self) -> None:
        if self.handle is not None:
            self.lib.s01g_shutdown(self.handle)
            self.handle = None


class Replay:
    """Paced replay of ring-record arrays into rings (s01g_replay_*)."""

    def __init__(self, ring_bufs, ring_heads, ring_mask: int, records, rate_rec_s: float,
                 pin_core: int = -1, lib_path: Optional[os.PathLike] = None,
                 speed: Optional[float] = None):
        """rate_rec_s: aggregate rate, rings round-robin.  speed (instead):
        publish in merged record-time order, (t - t_first) / speed us after
        the start."""
        self.lib = load_to_gpu(lib_path)
        n = len(ring_bufs)
        self._recs = [np.ascontiguousarray(r) for r in records]   # kept alive until stop
        bufs = (ctypes.c_void_p * n)(*[int(p) for p in ring_bufs])
        heads = (ctypes.c_void_p * n)(*[int(p) for p in ring_heads])
        recp = (ctypes.c_void_p * n)(*[r.ctypes.data for r in self._recs])
        counts = (ctypes.c_int * n)(*[int(r.size) for r in self._recs])
        if speed is not None:
            self.h = self.lib.s01g_replay_start_timed(n, bufs, heads, ring_mask, recp, counts,
                                                      float(speed), pin_core)
        else:
            self.h = self.lib.s01g_replay_start(n, bufs, heads, ring_mask, recp, counts,
                                                rate_rec_s, pin_core)
        if not self.h:
            raise RuntimeError("s01g_replay_start rejected its arguments")

    def done(self) -> bool:
        return bool(self.lib.s01g_replay_done(self.h))

    def published(self) -> int:
        return int(self.lib.s01g_replay_published(self.h))

    def stop(self) -> None:
        if self.h:
            self.lib.s01g_replay_stop(self.h)
            self.h = None


class S0API:
    """One libstage01_capi.so handle: shards without rings."""

    def __init__(self, lib_path: Optional[os.PathLike] = None):
        self.lib = load_capi(lib_path)
        self.handle = None

    def init(self, weights_dir: str, n_shards: int, halo: int, base_core: int, sample_cap: int):
        self.handle = self.lib.s0_init(str(weights_dir).encode(), n_shards, halo, base_core,
                                       sample_cap)
        if not self.handle:
            raise RuntimeError("s0_init returned NULL (check weights_dir / meta.json)")

    def submit(self, events: np.ndarray) -> int:
        ev = np.ascontiguousarray(events, np.float32)
        if ev.shape[0] == 0:
            return 0
        return self.lib.s0_submit_batch(self.handle, ev.ctypes.data_as(_fptr), ev.shape[0])

    def stats(self) -> list:
        out = (ctypes.c_double * 16)()
        self.lib.s0_snapshot_stats(self.handle, out)
        return list(out)

    def reset(self) -> None:
        self.lib.s0_reset_stats(self.handle)

    def wait_processed(self, n_owner: int, n_halo: int, timeout_s: float = 60.0) -> list:
        t_end = time.monotonic() + timeout_s
        while True:
            s = self.stats()
            if s[0] >= n_owner and s[1] >= n_halo:
                return s
            if time.monotonic() > t_end:
                raise TimeoutError("stage 0/1 shards did not finish in time")
            time.sleep(0.001)

    def shutdown(self) -> None:
        if self.handle is not None:
            self.lib.s0_shutdown(self.handle)
            self.handle = None
