"""Host-side consumer of the prediction grid, over libssla_hip's C ABI.

Mirrors what the reference does on the CPU with the head's output:

* ``snapshot``        torn-free copy of cells the device may be writing
                      (the reference reads its pinned views directly,
                      orin/hybrid_runner_multi.py:648-656);
* ``decode_cells``    decode_yolox_cell's grid/exp/stride transform
                      (vendor/openeva/heads/async_yolox.h:189-196);
* ``collect_bboxes``  the live demo's box collection
                      (orin/hybrid_runner_multi.py:163-207);
* ``OracleRecorder`` / ``diff_dumps``  the OEVA head-grid dump and its diff
                      (include/oracle.h:35-150), same names and behaviour.

Every computation runs in libssla_hip.so (host code, no GPU needed); this
module only shapes arrays.
"""
from __future__ import annotations

import ctypes
from dataclasses import dataclass
from typing import List, Optional, Sequence, Tuple

import numpy as np

from . import abi, lib

HEAD_OUT = abi.HEAD_OUT
PRED_BUSY = abi.PRED_BUSY


def _fp(a: np.ndarray):
    return a.ctypes.data_as(ctypes.POINTER(ctypes.c_float))


def _up(a: np.ndarray):
    return a.ctypes.data_as(ctypes.POINTER(ctypes.c_uint))


def _f32c(a) -> np.ndarray:
    return np.ascontiguousarray(a, dtype=np.float32)


# ---- prediction grid --------------------------------------------------------

def snapshot_ptr(preds_ptr: int, version_ptr: int, n_cells: int, cols: int = HEAD_OUT,
                 max_tries: int = 64) -> Tuple[np.ndarray, np.ndarray, int]:
    """Torn-free copy of n_cells cells at host-visible addresses (the drain's
    fine-grained preds / version buffers).  Returns (preds, version, torn)."""
    preds = np.zeros((n_cells, cols), np.float32)
    version = np.zeros(n_cells, np.uint32)
    torn = lib.check(lib.load().ssla_hip_preds_snapshot(
        ctypes.cast(ctypes.c_void_p(preds_ptr), ctypes.POINTER(ctypes.c_float)),
        ctypes.cast(ctypes.c_void_p(version_ptr), ctypes.POINTER(ctypes.c_uint)),
        n_cells, cols, _fp(preds), _up(version), max_tries), "preds_snapshot")
    return preds, version, torn


def snapshot(preds: np.ndarray, version: np.ndarray,
             max_tries: int = 64) -> Tuple[np.ndarray, np.ndarray, int]:
    """Same for numpy views (e.g. of pinned memory): preds (n, cols) float32,
    version (n,) uint32, both C-contiguous views of the shared memory."""
    if preds.dtype != np.float32 or version.dtype != np.uint32 or preds.ndim != 2 \
            or not preds.flags.c_contiguous or not version.flags.c_contiguous \
            or preds.shape[0] != version.shape[0]:
        raise ValueError("snapshot: need C-contiguous float32 (n, cols) and uint32 (n,)")
    return snapshot_ptr(preds.ctypes.data, version.ctypes.data, preds.shape[0], preds.shape[1],
                        max_tries)


def decode_cells(raw: np.ndarray, grid_w: int, gx0: int = 0, gy0: int = 0,
                 stride_w: int = 8, stride_h: int = 8) -> np.ndarray:
    """Raw rows [tx, ty, log_w, log_h, obj, cls...] of cells laid row-major
    over a grid_w-wide box at (gx0, gy0) -> pixel-space rows
    [cx, cy, w, h, obj, cls...]."""
    raw = _f32c(raw)
    if raw.ndim != 2 or raw.shape[1] < 5:
        raise ValueError("decode_cells: raw must be (n, >=5)")
    out = np.empty_like(raw)
    lib.check(lib.load().ssla_hip_decode_cells(_fp(raw), raw.shape[0], raw.shape[1], grid_w, gx0,
                                               gy0, stride_w, stride_h, _fp(out)), "decode_cells")
    return out


def grid_decode(cfg: abi.HybridS2S3Config, zero_row: np.ndarray, stride_w: int = 8,
                stride_h: int = 8, max_tries: int = 64) -> Tuple[np.ndarray, int]:
    """The whole s3 grid, decoded, as the CPU pipeline's detection output
    holds it: (H3*W3, 7), row gy*W3 + gx; never-written cells hold the
    decoded zero_row.  Returns (grid, torn)."""
    zero_row = _f32c(zero_row).reshape(HEAD_OUT)
    out = np.zeros((cfg.H3 * cfg.W3, HEAD_OUT), np.float32)
    torn = lib.check(lib.load().ssla_hip_grid_decode(ctypes.byref(cfg), _fp(zero_row), stride_w,
                                                     stride_h, max_tries, _fp(out)), "grid_decode")
    return out, torn


def head_row(weights_dir: str, feat: Optional[np.ndarray] = None) -> np.ndarray:
    """Raw head row of one 96-channel feature (all zeros by default) from a
    weight directory's head."""
    x = np.zeros(96, np.float32) if feat is None else _f32c(feat).reshape(96)
    out = np.zeros(HEAD_OUT, np.float32)
    lib.check(lib.load().ssla_hip_head_row(str(weights_dir).encode(), _fp(x), _fp(out)),
              "head_row")
    return out


def collect_bboxes(preds_view: Sequence[np.ndarray], topo: Sequence, frame_w: int, frame_h: int,
                   scale: float, obj_thresh: float, W_full: int, H_full: int):
    """orin/hybrid_runner_multi.py:163-207, same arguments and results:
    (boxes_xywh, scores, max_score_seen).  topo[b] is an s3 box: a
    HybridStrip, or any object with owned_x_lo/owned_x_hi/owned_y_lo/
    owned_y_hi in s2 cells (the reference's BlockTopo).  frame_w/frame_h are
    accepted and unused, as in the reference."""
    del frame_w, frame_h
    L = lib.load()
    boxes: List[List[float]] = []
    scores: List[float] = []
    max_seen = ctypes.c_float(0.0)
    for b, t in enumerate(topo):
        if hasattr(t, "s3_owned_lo"):
            x_lo, x_hi, y_lo, y_hi = t.s3_owned_lo, t.s3_owned_hi, t.s3_owned_y_lo, t.s3_owned_y_hi
        else:
            x_lo, x_hi = t.owned_x_lo >> 1, t.owned_x_hi >> 1
            y_lo, y_hi = t.owned_y_lo >> 1, t.owned_y_hi >> 1
        s3w, s3h = x_hi - x_lo, y_hi - y_lo
        if s3w == 0 or s3h == 0:
            continue
        raw = _f32c(preds_view[b]).reshape(-1, HEAD_OUT)
        if raw.shape[0] < s3w * s3h:
            raise ValueError(f"collect_bboxes: block {b} has {raw.shape[0]} cells, box needs "
                             f"{s3w * s3h}")
        cap = s3w * s3h
        bx = np.zeros((cap, 4), np.float32)
        sc = np.zeros(cap, np.float32)
        n = lib.check(L.ssla_hip_collect_boxes(_fp(raw), s3w, s3h, x_lo, y_lo, scale, obj_thresh,
                                               W_full, H_full, _fp(bx), _fp(sc), cap,
                                               ctypes.byref(max_seen)), "collect_boxes")
        boxes += [[float(v) for v in row] for row in bx[:n]]
        scores += [float(v) for v in sc[:n]]
    return boxes, scores, float(max_seen.value)


# ---- OEVA dumps ---------------------------------------------------------------

class OracleRecorder:
    """include/oracle.h:35-89: keeps (event_idx, predictions) at every
    ``every_n_events``-th event (and event 0) and writes them with save().
    predictions whose size is not num_anchors*cols are skipped, as the
    reference skips a head that is not ready yet."""

    def __init__(self, num_anchors: int, cols: int, every_n_events: int, path: str):
        if num_anchors <= 0 or cols <= 0:
            raise ValueError("OracleRecorder: invalid shape")
        self.num_anchors, self.cols = int(num_anchors), int(cols)
        self.every, self.path = int(every_n_events), str(path)
        self._idx: List[int] = []
        self._preds: List[np.ndarray] = []

    def wants(self, event_idx: int) -> bool:
        return self.every != 0 and (event_idx % self.every == 0 or event_idx == 0)

    def record(self, event_idx: int, predictions: Optional[np.ndarray]) -> None:
        if not self.wants(event_idx) or predictions is None:
            return
        p = _f32c(predictions).reshape(-1)
        if p.size != self.num_anchors * self.cols:
            return
        self._idx.append(int(event_idx))
        self._preds.append(p.copy())

    def num_checkpoints(self) -> int:
        return len(self._idx)

    def save(self) -> None:
        write_dump(self.path, self.num_anchors, self.cols, self._idx, self._preds)


def write_dump(path: str, num_anchors: int, cols: int, event_idx: Sequence[int],
               preds: Sequence[np.ndarray]) -> None:
    n = len(event_idx)
    idx = (ctypes.c_ulonglong * max(n, 1))(*[int(e) for e in event_idx])
    body = np.concatenate([_f32c(p).reshape(-1) for p in preds]) if n else np.zeros(1, np.float32)
    if body.size != n * num_anchors * cols and n:
        raise ValueError("write_dump: predictions do not match num_anchors*cols")
    lib.check(lib.load().ssla_hip_oeva_write(str(path).encode(), num_anchors, cols, n, idx,
                                             _fp(body)), "oeva_write")


def read_dump(path: str) -> Tuple[np.ndarray, np.ndarray]:
    """(event_idx (n,), predictions (n, num_anchors, cols))."""
    L = lib.load()
    hdr = (ctypes.c_uint * 3)()
    lib.check(L.ssla_hip_oeva_header(str(path).encode(), hdr), "oeva_header")
    na, cols, n = hdr
    idx = (ctypes.c_ulonglong * max(n, 1))()
    preds = np.zeros((max(n, 1), na, cols), np.float32)
    lib.check(L.ssla_hip_oeva_read(str(path).encode(), idx, _fp(preds), n), "oeva_read")
    return np.array(idx[:n], np.uint64), preds[:n]


@dataclass
class DiffReport:
    ok: bool
    n_cp: int
    max_abs_delta: float
    n_mismatched_cp: int


def diff_dumps(path_a: str, path_b: str, tol_abs: float = 1e-4) -> DiffReport:
    """deploy::diff_dumps (include/oracle.h:90-150)."""
    r = abi.SslaHipOevaDiff()
    lib.check(lib.load().ssla_hip_oeva_diff(str(path_a).encode(), str(path_b).encode(), tol_abs,
                                            ctypes.byref(r)), "oeva_diff")
    return DiffReport(bool(r.ok), int(r.n_cp), float(r.max_abs_delta), int(r.n_mismatched_cp))
