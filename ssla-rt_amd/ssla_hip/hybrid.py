"""Host-side driver of libssla_hip.so: device buffers, weight packing,
configuration and the drain calls.

Mirrors the reference's host helpers (orin/orin/hybrid_common.py:138-271,
orin/orin/multi_block.py:128-340): random or weight-directory layers are
packed into the device layouts of include/ssla_abi.h, a HybridS2S3Config is
filled with device pointers, and the drain entry of the C ABI runs the
rings.  All compute happens in the library; this module only moves bytes.
"""
from __future__ import annotations

import ctypes
from dataclasses import dataclass
from typing import List, Optional, Sequence

import numpy as np

from . import abi, grid, lib
from .events import GPU_LAYER_IO, RawLayer


class DeviceBuffer:
    """A device-visible allocation (HBM, or fine-grained host memory)."""

    def __init__(self, nbytes: int, host: bool = False):
        self.nbytes = int(nbytes)
        self.host = host
        p = ctypes.c_void_p()
        L = lib.load()
        rc = (L.ssla_hip_malloc_host if host else L.ssla_hip_malloc_device)(self.nbytes, ctypes.byref(p))
        lib.check(rc, "malloc")
        self.ptr = int(p.value)

    @classmethod
    def from_array(cls, arr: np.ndarray, host: bool = False) -> "DeviceBuffer":
        arr = np.ascontiguousarray(arr)
        b = cls(arr.nbytes, host=host)
        b.upload(arr)
        return b

    def upload(self, arr: np.ndarray, offset: int = 0) -> None:
        arr = np.ascontiguousarray(arr)
        if offset + arr.nbytes > self.nbytes:
            raise ValueError("upload past the end of the buffer")
        lib.check(lib.load().ssla_hip_memcpy(self.ptr + offset, arr.ctypes.data, arr.nbytes), "memcpy")

    def download(self, dtype, count: int, offset: int = 0) -> np.ndarray:
        out = np.empty(count, dtype=dtype)
        if offset + out.nbytes > self.nbytes:
            raise ValueError("download past the end of the buffer")
        lib.check(lib.load().ssla_hip_memcpy(out.ctypes.data, self.ptr + offset, out.nbytes), "memcpy")
        return out

    def zero(self) -> None:
        lib.check(lib.load().ssla_hip_memset(self.ptr, 0, self.nbytes), "memset")

    def free(self) -> None:
        if self.ptr:
            L = lib.load()
            (L.ssla_hip_free_host if self.host else L.ssla_hip_free_device)(self.ptr)
            self.ptr = 0


def download_ptr(ptr: int, dtype, count: int) -> np.ndarray:
    out = np.empty(count, dtype=dtype)
    if count:
        lib.check(lib.load().ssla_hip_memcpy(out.ctypes.data, ptr, out.nbytes), "memcpy")
    return out


def upload_ptr(ptr: int, arr: np.ndarray) -> None:
    arr = np.ascontiguousarray(arr)
    lib.check(lib.load().ssla_hip_memcpy(ptr, arr.ctypes.data, arr.nbytes), "memcpy")


# ---- packing (orin/orin/weights_ssla.py:24-88) ----------------------------

@dataclass
class PackedLayer:
    """Fused weights in the reference (oracle) layout."""
    qvgIn: np.ndarray               # (9, 3*out, in)
    goW: np.ndarray                 # (9, out, out)
    input_proj: Optional[np.ndarray]  # (out, in) or None
    ln_gamma: np.ndarray
    ln_beta: np.ndarray


def pack_raw_layer(raw: RawLayer) -> PackedLayer:
    """qvgIn[p] = [qW; vW; gW] @ scatter_p, goW[p] = gather_p @ oW (fp32)."""
    i = raw.W_in_cat.shape[0]
    D = raw.qW.shape[0]
    n_in = raw.W_in_cat.shape[1] // D
    n_out = raw.W_out_cat.shape[0] // D
    A = max(n_in, n_out)
    qvg = np.empty((A, 3 * D, i), np.float32)
    go = np.empty((A, D, D), np.float32)
    for p in range(A):
        pin = 0 if n_in == 1 else p
        pout = 0 if n_out == 1 else p
        scatter = np.ascontiguousarray(raw.W_in_cat[:, pin * D:(pin + 1) * D].T)
        gather = np.ascontiguousarray(raw.W_out_cat[pout * D:(pout + 1) * D, :].T)
        qvg[p] = np.concatenate([raw.qW @ scatter, raw.vW @ scatter, raw.gW @ scatter])
        go[p] = gather @ raw.oW
    return PackedLayer(qvg, go, raw.input_proj, raw.ln_gamma, raw.ln_beta)


def device_layouts(p: PackedLayer):
    """(qvgIn (9, in, 3*out), goW (9, out_in, out_out), input_proj (in, out))."""
    qvg = np.ascontiguousarray(p.qvgIn.transpose(0, 2, 1))
    go = np.ascontiguousarray(p.goW.transpose(0, 2, 1))
    ip = None if p.input_proj is None else np.ascontiguousarray(p.input_proj.T)
    return qvg, go, ip


# ---- single-linear head (orin/orin/hybrid_common.py:313-325) ---------------------

def build_head_weights(rng: np.random.Generator, head_out_dim: int = abi.HEAD_OUT):
    """Random single-linear head in the draw order of the reference's
    build_head_weights: head_W (96, head_out_dim) ~ N(0, 0.1), in the
    device's (IN, OUT) layout (the kernel reads head_W[i*7 + o]), then
    head_b (head_out_dim,) ~ N(0, 0.1).  The reference's live runner uses it
    for weight directories without head keys (orin/hybrid_runner_multi.py:
    395-423), its legacy runner always (orin/hybrid_runner.py:294-304)."""
    W = rng.normal(scale=0.1, size=(96, head_out_dim)).astype(np.float32)
    b = rng.normal(scale=0.1, size=(head_out_dim,)).astype(np.float32)
    return W, b


# ---- the drain ---------------------------------------------------------------

class Drain:
    """Owns one HybridS2S3Config and its device state; runs drain calls."""

    def __init__(self):
        self.cfg = abi.HybridS2S3Config()
        self._owned: List[DeviceBuffer] = []
        self._model = ctypes.c_void_p()
        self._state_blocks: List[int] = []
        self._pred_blocks: List[int] = []
        self._rings: List[Optional[DeviceBuffer]] = []
        self._outs: List[Optional[DeviceBuffer]] = []
        self._heads: List[Optional[DeviceBuffer]] = []
        self._linear_head: Optional[tuple] = None

    # -- construction ---------------------------------------------------------
    @classmethod
    def from_weights_dir(cls, weights_dir: str, n_blocks: int = 1,
                         with_preds: bool = True,
                         strips: Optional[Sequence[tuple]] = None,
                         linear_head: Optional[tuple] = None) -> "Drain":
        """strips: per block (x_lo, x_hi, y_lo, y_hi) owned s2 box (e.g.
        topology.grid_topology(...)[b].owned); default the whole grid.
        linear_head: (head_W (96, 7), head_b (7,)) bound when the directory has
        no head keys, as the reference's live runner falls back to a
        single-linear head (orin/hybrid_runner_multi.py:395-423); e.g.
        build_head_weights(np.random.default_rng(seed))."""
        d = cls()
        L = lib.load()
        lib.check(L.ssla_hip_model_load(weights_dir.encode(), ctypes.byref(d._model)), "model_load")
        lib.check(L.ssla_hip_config_bind(d._model, n_blocks, ctypes.byref(d.cfg)), "config_bind")
        if strips is not None:
            if len(strips) != n_blocks:
                raise ValueError("from_weights_dir: one strip per block")
            for b, (x_lo, x_hi, y_lo, y_hi) in enumerate(strips):
                s = d.cfg.strip[b]
                s.owned_lo, s.owned_hi, s.owned_y_lo, s.owned_y_hi = x_lo, x_hi, y_lo, y_hi
                s.s3_owned_lo, s.s3_owned_hi = x_lo >> 1, x_hi >> 1
                s.s3_owned_y_lo, s.s3_owned_y_hi = y_lo >> 1, y_hi >> 1
        for b in range(n_blocks):
            lib.check(L.ssla_hip_state_alloc(ctypes.byref(d.cfg), b), "state_alloc")
            d._state_blocks.append(b)
        if linear_head is not None and not d.cfg.head_cls_conv_W:
            d.bind_linear_head(*linear_head, with_preds=with_preds)
        elif with_preds and d.cfg.head_cls_conv_W:
            d.alloc_preds()
        return d

    def alloc_preds(self) -> None:
        """Prediction grids (preds, version) of every block that has none."""
        L = lib.load()
        for b in range(self.cfg.n_blocks):
            if b not in self._pred_blocks:
                lib.check(L.ssla_hip_preds_alloc(ctypes.byref(self.cfg), b), "preds_alloc")
                self._pred_blocks.append(b)

    def bind_linear_head(self, W: np.ndarray, b: np.ndarray, with_preds: bool = True) -> None:
        """Binds the single-linear head (cfg.head_W (96, 7), cfg.head_b (7,),
        orin/kernels/ssla_s2_s3_head_celled.cuh:1476-1481) in place of any
        two-branch head, and allocates the prediction grids."""
        W = np.ascontiguousarray(W, np.float32)
        b = np.ascontiguousarray(b, np.float32)
        if W.shape != (96, abi.HEAD_OUT) or b.shape != (abi.HEAD_OUT,):
            raise ValueError("bind_linear_head: head_W must be (96, 7) and head_b (7,)")
        bw, bb = DeviceBuffer.from_array(W), DeviceBuffer.from_array(b)
        self._owned += [bw, bb]
        c = self.cfg
        for f in abi.HEAD_FIELDS:
            setattr(c, f, None)
        c.head_W, c.head_b = bw.ptr, bb.ptr
        self._linear_head = (W.copy(), b.copy())
        if with_preds:
            self.alloc_preds()

    @property
    def linear_head(self) -> Optional[tuple]:
        """(head_W, head_b) host copies of a bound single-linear head."""
        return self._linear_head

    @classmethod
    def from_packed(cls, layers: Sequence[PackedLayer], H2: int, W2: int, window: int,
                    n_blocks: int = 1, h_init: Optional[Sequence[np.ndarray]] = None,
                    strips: Optional[Sequence[tuple]] = None) -> "Drain":
        """Random / array layers (hybrid_common.build_random_layers +
        build_config).  strips: per block (x_lo, x_hi, y_lo, y_hi) owned s2
        box; default the whole grid."""
        d = cls()
        c = d.cfg
        c.H2, c.W2, c.H3, c.W3 = H2, W2, H2 >> 1, W2 >> 1
        c.tdrop_window = window
        c.head_out_dim = abi.HEAD_OUT
        c.n_blocks = n_blocks
        ptrs = []
        for li, p in enumerate(layers):
            qvg, go, ip = device_layouts(p)
            bufs = [DeviceBuffer.from_array(a) if a is not None else None
                    for a in (qvg, go, ip, p.ln_gamma, p.ln_beta)]
            d._owned += [b for b in bufs if b is not None]
            ptrs.append([b.ptr if b is not None else None for b in bufs])
        for b in range(n_blocks):
            x_lo, x_hi, y_lo, y_hi = strips[b] if strips else (0, W2, 0, H2)
            s = c.strip[b]
            s.owned_lo, s.owned_hi, s.owned_y_lo, s.owned_y_hi = x_lo, x_hi, y_lo, y_hi
            s.s3_owned_lo, s.s3_owned_hi = x_lo >> 1, x_hi >> 1
            s.s3_owned_y_lo, s.s3_owned_y_hi = y_lo >> 1, y_hi >> 1
            for li in range(4):
                lw = c.layers[b][li]
                lw.qvgIn, lw.goW, lw.input_proj, lw.ln_gamma, lw.ln_beta = ptrs[li]
            lib.check(lib.load().ssla_hip_state_alloc(ctypes.byref(c), b), "state_alloc")
            d._state_blocks.append(b)
            if h_init is not None:
                for li in range(4):
                    upload_ptr(c.hidden[b][li], h_init[li])
        return d

    # -- state access ---------------------------------------------------------
    def cells(self, li: int) -> int:
        c = self.cfg
        return c.H2 * c.W2 if li < 2 else c.H3 * c.W3

    def hidden(self, blk: int, li: int) -> np.ndarray:
        out = GPU_LAYER_IO[li][1]
        return download_ptr(self.cfg.hidden[blk][li], np.float32, self.cells(li) * out).reshape(-1, out)

    def set_hidden(self, blk: int, li: int, arr: np.ndarray) -> None:
        upload_ptr(self.cfg.hidden[blk][li], arr.astype(np.float32))

    def counters(self, blk: int):
        c = self.cfg
        return (download_ptr(c.tdrop_s2[blk], np.uint8, c.H2 * c.W2),
                download_ptr(c.tdrop_s3[blk], np.uint8, c.H3 * c.W3))

    def set_counters(self, blk: int, td2: np.ndarray, td3: np.ndarray) -> None:
        upload_ptr(self.cfg.tdrop_s2[blk], td2.astype(np.uint8))
        upload_ptr(self.cfg.tdrop_s3[blk], td3.astype(np.uint8))

    def preds(self, blk: int, max_tries: int = 2000):
        """Torn-free copy of block blk's prediction cells: (preds (n, 7),
        version (n,)).  Raises if a cell stays busy for max_tries reads
        (about 1 us apart)."""
        s = self.cfg.strip[blk]
        n = (s.s3_owned_hi - s.s3_owned_lo) * (s.s3_owned_y_hi - s.s3_owned_y_lo)
        if not self.cfg.preds[blk]:
            return None, None
        p, v, torn = grid.snapshot_ptr(self.cfg.preds[blk], self.cfg.version[blk], n,
                                       abi.HEAD_OUT, max_tries)
        if torn:
            raise lib.SslaHipError(f"preds: {torn} cells of block {blk} kept changing")
        return p, v

    def zero_row(self) -> np.ndarray:
        """The head's raw output for an all-zero feature (the value of a cell
        no record has reached yet in the CPU pipeline)."""
        if self._linear_head is not None:
            return self._linear_head[1].copy()
        if not self._model:
            raise lib.SslaHipError("zero_row: no model loaded (random layers have no head)")
        x = np.zeros(96, np.float32)
        out = np.zeros(abi.HEAD_OUT, np.float32)
        fp = ctypes.POINTER(ctypes.c_float)
        lib.check(lib.load().ssla_hip_model_head_row(self._model, x.ctypes.data_as(fp),
                                                     out.ctypes.data_as(fp)), "model_head_row")
        return out

    def head_grid(self, stride: int = 8, max_tries: int = 2000) -> np.ndarray:
        """Decoded (H3*W3, 7) grid, row gy*W3 + gx, as the CPU pipeline's
        detection output holds it."""
        out, torn = grid.grid_decode(self.cfg, self.zero_row(), stride, stride, max_tries)
        if torn:
            raise lib.SslaHipError(f"head_grid: {torn} cells kept changing")
        return out

    def reset(self, stream: int = 0, sync: bool = True) -> None:
        L = lib.load()
        for b in self._state_blocks:
            if sync:
                lib.check(L.ssla_hip_state_reset(ctypes.byref(self.cfg), b), "state_reset")
            else:
                lib.check(L.ssla_hip_state_reset_async(ctypes.byref(self.cfg), b, stream or None),
                          "state_reset_async")

    # -- rings ------------------------------------------------------------------
    def load_rings(self, records: Sequence[np.ndarray], want_head: bool = False) -> None:
        """Copy each block's records into HBM (resident before any timing)."""
        for bufs in (self._rings, self._outs, self._heads):
            for b in bufs:
                if b is not None:
                    b.free()
        self._rings, self._outs, self._heads = [], [], []
        self._ns = [int(r.size) for r in records]
        for r in records:
            r = np.ascontiguousarray(r, dtype=abi.INPUT_DTYPE)
            n = max(1, r.size)
            rb = DeviceBuffer(n * abi.INPUT_DTYPE.itemsize)
            if r.size:
                rb.upload(r)
            self._rings.append(rb)
            self._outs.append(DeviceBuffer(n * abi.OUTPUT_DTYPE.itemsize))
            self._heads.append(DeviceBuffer(n * 7 * 4) if want_head else None)

    def run(self, stream: int = 0, sync: bool = True, phase_ms: Optional[np.ndarray] = None,
            batch: int = 0, batch_phase_us: Optional[np.ndarray] = None, group: int = 0,
            phase_mask: int = 0) -> None:
        """One drain call over the loaded rings.  phase_ms (float32 array of
        len(abi.DRAIN_PHASES)) accumulates per-phase GPU time of the phases
        in phase_mask (bit k = phase k; 0 = all); a call without sync adds
        its times when a later call with sync returns.  group (batch mode):
        workgroups per block, 3..6 (0 = one)."""
        nb = self.cfg.n_blocks
        if len(self._rings) != nb:
            raise ValueError(f"load_rings needs {nb} rings")
        rings = (ctypes.c_void_p * nb)(*[b.ptr for b in self._rings])
        ns = (ctypes.c_int * nb)(*self._ns)
        outs = (ctypes.c_void_p * nb)(*[b.ptr for b in self._outs])
        opts = abi.SslaHipDrainOpts()
        opts.stream = stream or None
        opts.sync = 1 if sync else 0
        opts.batch = batch
        opts.group = group
        opts.phase_mask = phase_mask
        heads = None
        if self._heads and self._heads[0] is not None:
            heads = (ctypes.c_void_p * nb)(*[b.ptr for b in self._heads])
            opts.head_outs = ctypes.cast(heads, ctypes.POINTER(ctypes.c_void_p))
        if phase_ms is not None:
            assert phase_ms.dtype == np.float32 and phase_ms.size >= len(abi.DRAIN_PHASES)
            opts.phase_ms = phase_ms.ctypes.data_as(ctypes.POINTER(ctypes.c_float))
        if batch_phase_us is not None:
            assert batch_phase_us.dtype == np.float64 and batch_phase_us.size >= abi.N_BATCH_PHASES
            opts.batch_phase_us = batch_phase_us.ctypes.data_as(ctypes.POINTER(ctypes.c_double))
        lib.check(lib.load().ssla_hip_drain_n_ex(ctypes.byref(self.cfg), rings, ns, outs,
                                                 ctypes.byref(opts)), "drain_n_ex")

    def run_two_rings(self) -> None:
        """ssla_hip_drain_n2 over the two loaded rings (the reference's P1
        two-ring entry, orin/bench_s2_s3_head_celled.py:234-244)."""
        if self.cfg.n_blocks != 2 or len(self._rings) != 2:
            raise ValueError("run_two_rings needs two blocks and two loaded rings")
        lib.check(lib.load().ssla_hip_drain_n2(
            ctypes.byref(self.cfg), self._rings[0].ptr, self._rings[1].ptr, self._ns[0],
            self._ns[1], self._outs[0].ptr, self._outs[1].ptr), "drain_n2")

    def results(self):
        outs, heads = [], []
        for b in range(self.cfg.n_blocks):
            n = self._ns[b]
            outs.append(self._outs[b].download(abi.OUTPUT_DTYPE, n))
            h = self._heads[b]
            heads.append(h.download(np.float32, n * 7).reshape(n, 7) if h is not None else None)
        return outs, heads

    def drain(self, records: Sequence[np.ndarray], want_head: bool = False, batch: int = 0,
              group: int = 0):
        """Drain pre-filled rings; batch 0 = whole-ring drain, 1..32 = in-kernel
        batches of that many records (group: workgroups per block, 3..6)."""
        self.load_rings(records, want_head=want_head)
        self.run(batch=batch, group=group)
        return self.results()

    def drain_recorded(self, records: Sequence[np.ndarray], recorder: "grid.OracleRecorder",
                       stride: int = 8, batch: int = 0) -> None:
        """Drain the rings with the head grid recorded after ring position i
        for every i the recorder wants (i % every == 0), as the reference's
        equivalence harness records after each step (include/oracle.h:42-53,
        src/legacy/schemes/s1_reference.cpp:170-180).  Every ring is cut at
        the same positions; records past the last checkpoint are drained too."""
        n = max((len(r) for r in records), default=0)
        cuts = [i + 1 for i in range(n) if recorder.wants(i)]
        if not cuts or cuts[-1] != n:
            cuts.append(n)
        lo = 0
        for hi in cuts:
            if hi > lo:
                self.drain([r[lo:hi] for r in records], batch=batch)
            if hi >= 1 and recorder.wants(hi - 1):
                recorder.record(hi - 1, self.head_grid(stride))
            lo = hi

    def drain_with_clocks(self, records: Sequence[np.ndarray]):
        """ssla_hip_drain_n with batch_clks: in-kernel batches of 8 records and
        a (t_pop, t_done) wall-clock pair per batch."""
        self.load_rings(records)
        nb = self.cfg.n_blocks
        clk = [DeviceBuffer(max(1, (n + 7) // 8) * 16) for n in self._ns]
        try:
            rings = (ctypes.c_void_p * nb)(*[b.ptr for b in self._rings])
            ns = (ctypes.c_int * nb)(*self._ns)
            outs = (ctypes.c_void_p * nb)(*[b.ptr for b in self._outs])
            clks = (ctypes.c_void_p * nb)(*[b.ptr for b in clk])
            lib.check(lib.load().ssla_hip_drain_n(ctypes.byref(self.cfg), rings, ns, outs, clks),
                      "drain_n")
            outs_h, _ = self.results()
            clocks = [c.download(np.uint64, 2 * ((n + 7) // 8)).reshape(-1, 2)
                      for c, n in zip(clk, self._ns)]
        finally:
            for c in clk:
                c.free()
        return outs_h, clocks

    # -- live (persistent) drain ---------------------------------------------------
    def alloc_timing(self, capacity: int = 1 << 16) -> None:
        L = lib.load()
        for b in range(self.cfg.n_blocks):
            lib.check(L.ssla_hip_timing_alloc(ctypes.byref(self.cfg), b, capacity), "timing_alloc")
        self._timing = True

    def timing(self, blk: int) -> np.ndarray:
        n = self.cfg.timing_mask + 1
        return download_ptr(self.cfg.timing[blk], abi.TIMING_DTYPE, n)

    def kernel_clocks(self, blk: int):
        v = np.ctypeslib.as_array((ctypes.c_ulonglong * 2).from_address(self.cfg.kernel_start_clk[blk]))
        return int(v[0]), int(v[1])

    def close(self) -> None:
        L = lib.load()
        if getattr(self, "_timing", False):
            for b in range(self.cfg.n_blocks):
                L.ssla_hip_timing_free(ctypes.byref(self.cfg), b)
            self._timing = False
        for bufs in (self._rings, self._outs, self._heads):
            for b in bufs:
                if b is not None:
                    b.free()
        for b in self._pred_blocks:
            L.ssla_hip_preds_free(ctypes.byref(self.cfg), b)
        for b in self._state_blocks:
            L.ssla_hip_state_free(ctypes.byref(self.cfg), b)
        self._pred_blocks, self._state_blocks = [], []
        for b in self._owned:
            b.free()
        self._owned = []
        if self._model:
            L.ssla_hip_model_free(self._model)
            self._model = ctypes.c_void_p()

    def __enter__(self):
        return self

    def __exit__(self, *exc):
        self.close()


class HostRings:
    """Per-block rings in fine-grained host memory with the producer-side
    head counters and the consumer-side tail / events_done words, plus the
    stop flag (orin/hybrid_runner_multi.py:446-462)."""

    def __init__(self, n_blocks: int, capacity: int = 1 << 16):
        if capacity & (capacity - 1):
            raise ValueError("ring capacity must be a power of two")
        self.n_blocks, self.capacity = n_blocks, capacity
        self.bufs = [DeviceBuffer(capacity * abi.INPUT_DTYPE.itemsize, host=True) for _ in range(n_blocks)]
        self.words = DeviceBuffer(8 * (3 * n_blocks + 1), host=True)
        for b in self.bufs:
            ctypes.memset(b.ptr, 0, b.nbytes)
        ctypes.memset(self.words.ptr, 0, self.words.nbytes)
        self.rings = [np.ctypeslib.as_array((ctypes.c_ubyte * b.nbytes).from_address(b.ptr))
                      .view(abi.INPUT_DTYPE) for b in self.bufs]
        w = np.ctypeslib.as_array((ctypes.c_ulonglong * (3 * n_blocks + 1)).from_address(self.words.ptr))
        self.head, self.tail, self.done = w[:n_blocks], w[n_blocks:2 * n_blocks], w[2 * n_blocks:3 * n_blocks]
        self.stop_ptr = self.words.ptr + 8 * 3 * n_blocks
        self._stop = np.ctypeslib.as_array((ctypes.c_int * 1).from_address(self.stop_ptr))

    def ptrs(self):
        nb = self.n_blocks
        base = self.words.ptr
        return ((ctypes.c_void_p * nb)(*[b.ptr for b in self.bufs]),
                (ctypes.c_void_p * nb)(*[base + 8 * (nb + b) for b in range(nb)]),
                (ctypes.c_void_p * nb)(*[base + 8 * (2 * nb + b) for b in range(nb)]))

    def head_ptrs(self):
        """Addresses of the producer-side head words (one per block)."""
        return [self.words.ptr + 8 * b for b in range(self.n_blocks)]

    def tail_ptrs(self):
        """Addresses of the consumer-side tail words (for back-pressure)."""
        return [self.words.ptr + 8 * (self.n_blocks + b) for b in range(self.n_blocks)]

    def push(self, blk: int, recs: np.ndarray) -> None:
        """Single-producer publish: write each record, then its seq_done tag."""
        ring = self.rings[blk]
        h = int(self.head[blk])
        for k in range(recs.size):
            slot = (h + k) & (self.capacity - 1)
            r = recs[k].copy()
            r["seq_done"] = 0
            ring[slot] = r
            ring["seq_done"][slot] = h + k + 1
        self.head[blk] = h + recs.size

    def stop(self) -> None:
        self._stop[0] = 1

    def free(self) -> None:
        for b in self.bufs:
            b.free()
        self.words.free()


class LiveDrain:
    """A running persistent drain over HostRings (ssla_hip_persistent_start;
    with two_ring=True the legacy two-ring entry ssla_hip_persistent_start2,
    orin/hybrid_runner.py:334-393, which fixes batches of 8 and one
    workgroup per block)."""

    def __init__(self, drain: Drain, rings: HostRings, spin_ns: int = 200, max_batch: int = 32,
                 idle_timeout_ms: int = 30000, profile: bool = False, group: int = 0,
                 stages: int = 1, two_ring: bool = False):
        self.rings = rings
        self.h = ctypes.c_void_p()
        bufs, tails, dones = rings.ptrs()
        self.phase_us = None
        if two_ring:
            lib.check(lib.load().ssla_hip_persistent_start2(
                ctypes.byref(drain.cfg), bufs[0], bufs[1], rings.capacity - 1, tails[0],
                tails[1], rings.stop_ptr, dones[0], dones[1], spin_ns, ctypes.byref(self.h)),
                "persistent_start2")
            return
        # in-kernel phase profile, filled by wait() (abi.BATCH_PHASES order)
        self.phase_us = np.zeros(abi.N_BATCH_PHASES, np.float64) if profile else None
        opts = abi.SslaHipLiveOpts(max_batch, idle_timeout_ms)
        opts.group = group
        opts.stages = stages
        if profile:
            opts.phase_us = self.phase_us.ctypes.data_as(ctypes.POINTER(ctypes.c_double))
        lib.check(lib.load().ssla_hip_persistent_start(
            ctypes.byref(drain.cfg), bufs, rings.capacity - 1, tails, rings.stop_ptr, dones,
            spin_ns, ctypes.byref(opts), ctypes.byref(self.h)), "persistent_start")

    def wait(self, timeout_ms: int = 60000) -> int:
        st = ctypes.c_int(-1)
        lib.check(lib.load().ssla_hip_persistent_wait(self.h, timeout_ms, ctypes.byref(st)),
                  "persistent_wait")
        self.h = ctypes.c_void_p()
        return st.value

    def stop(self, timeout_ms: int = 60000) -> int:
        self.rings.stop()
        return self.wait(timeout_ms)
