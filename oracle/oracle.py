"""ctypes binding of the CPU oracle (oracle/libssla_oracle.so).

TEST INFRASTRUCTURE ONLY: imported by tests/, __graft_entry__.smoke() and
the cpu_baseline leg of bench.py, as the checker or the timed CPU baseline.
The product (libssla_hip.so and its Python host side) never imports it.

The C sources (ssla_oracle.c, ssla_oracle_f32.c) list the reference file:line
each function restates.
"""
from __future__ import annotations

import ctypes
import subprocess
import threading
from dataclasses import dataclass
from pathlib import Path
from typing import Dict, List, Optional, Sequence

import numpy as np

HERE = Path(__file__).resolve().parent
LIB_PATH = HERE / "libssla_oracle.so"
REF_LIB_PATH = HERE / "_ref" / "libssla_ref.so"

C1, C2, C3 = 24, 48, 96
GPU_LAYER_IO = ((C1, C2), (C2, C2), (C2, C3), (C3, C3))

_FP = ctypes.POINTER(ctypes.c_float)


class OracleLayer(ctypes.Structure):
    _fields_ = [("qvgIn", _FP), ("goW", _FP), ("input_proj", _FP),
                ("ln_gamma", _FP), ("ln_beta", _FP),
                ("in_dim", ctypes.c_int), ("out_dim", ctypes.c_int), ("K", ctypes.c_int),
                ("qvgInT", _FP), ("goWT", _FP)]


class OracleHead(ctypes.Structure):
    _fields_ = [(n, _FP) for n in ("cls_conv_W", "cls_conv_b", "cls_pred_W", "cls_pred_b",
                                   "reg_conv_W", "reg_conv_b", "reg_pred_W", "reg_pred_b",
                                   "obj_pred_W", "obj_pred_b")] + [("C", ctypes.c_int),
                                                                   ("lin_W", _FP), ("lin_b", _FP)]


class OracleS2S3(ctypes.Structure):
    _fields_ = [("L", OracleLayer * 4), ("H", _FP * 4),
                ("td2", ctypes.POINTER(ctypes.c_uint8)), ("td3", ctypes.POINTER(ctypes.c_uint8)),
                ("H2", ctypes.c_int), ("W2", ctypes.c_int), ("H3", ctypes.c_int), ("W3", ctypes.c_int),
                ("window", ctypes.c_int), ("head", ctypes.POINTER(OracleHead))]


_lib = None


class OracleS01(ctypes.Structure):
    _fields_ = [("L", OracleLayer * 4), ("H", ctypes.POINTER(ctypes.c_float) * 4),
                ("td0", ctypes.POINTER(ctypes.c_uint8)), ("td1", ctypes.POINTER(ctypes.c_uint8)),
                ("last_t", ctypes.POINTER(ctypes.c_double)),
                ("height", ctypes.c_int), ("width", ctypes.c_int), ("window", ctypes.c_int)]


def build() -> None:
    subprocess.run(["make", "-s", "-C", str(HERE), "all"], check=True)


def load() -> ctypes.CDLL:
    global _lib
    if _lib is None:
        if not LIB_PATH.exists():
            build()
        L = ctypes.CDLL(str(LIB_PATH))
        L.oracle_reshape_layer.restype = ctypes.c_int
        L.oracle_reshape_layer.argtypes = [_FP, ctypes.c_int, _FP, ctypes.c_int, _FP, _FP, _FP, _FP,
                                           ctypes.c_int, ctypes.c_int, _FP, _FP]
        for nm in ("oracle_layer_step_f64", "oracle_layer_step_f32"):
            f = getattr(L, nm)
            f.restype = None
            f.argtypes = [ctypes.POINTER(OracleLayer), _FP, _FP, ctypes.c_int, ctypes.c_int,
                          ctypes.c_int, ctypes.c_int, _FP]
        L.oracle_tdrop.restype = ctypes.c_int
        L.oracle_tdrop.argtypes = [ctypes.POINTER(ctypes.c_uint8), ctypes.c_int, ctypes.c_int]
        L.oracle_s2s3_run.restype = ctypes.c_int
        L.oracle_s2s3_run.argtypes = [ctypes.POINTER(OracleS2S3), ctypes.c_void_p, ctypes.c_void_p,
                                      ctypes.c_void_p, ctypes.c_void_p, ctypes.c_int, ctypes.c_int,
                                      ctypes.c_void_p, ctypes.c_void_p, ctypes.c_void_p,
                                      ctypes.c_void_p]
        L.oracle_s2s3_decisions.restype = ctypes.c_int
        L.oracle_s2s3_decisions.argtypes = [ctypes.c_void_p, ctypes.c_void_p, ctypes.c_int,
                                            ctypes.c_int, ctypes.c_int, ctypes.c_void_p,
                                            ctypes.c_void_p, ctypes.c_int, ctypes.c_void_p,
                                            ctypes.c_void_p]
        for nm in ("oracle_head_raw_f64", "oracle_head_raw_f32"):
            f = getattr(L, nm)
            f.restype = None
            f.argtypes = [ctypes.POINTER(OracleHead), _FP, _FP]
        L.oracle_preprocess.restype = None
        L.oracle_preprocess.argtypes = [ctypes.c_void_p, ctypes.c_int, ctypes.c_int, ctypes.c_float,
                                        ctypes.c_int, ctypes.c_int, ctypes.c_float, _FP]
        L.oracle_s01_run.restype = ctypes.c_int
        L.oracle_s01_run.argtypes = [ctypes.POINTER(OracleS01), ctypes.c_void_p, ctypes.c_void_p,
                                     ctypes.c_int, ctypes.c_int, ctypes.c_void_p, ctypes.c_void_p,
                                     ctypes.c_void_p, ctypes.c_void_p, ctypes.c_void_p]
        L.oracle_fuse_conv_bn.restype = None
        L.oracle_fuse_conv_bn.argtypes = [_FP, _FP, _FP, _FP, _FP, _FP, ctypes.c_int, ctypes.c_int,
                                          ctypes.c_float, _FP, _FP]
        _lib = L
    return _lib


def _fp(a: Optional[np.ndarray]):
    if a is None:
        return None
    assert a.dtype == np.float32 and a.flags.c_contiguous
    return a.ctypes.data_as(_FP)


def _f32(a) -> np.ndarray:
    return np.ascontiguousarray(a, dtype=np.float32)


# ---- layers -------------------------------------------------------------------

_T_LOCK = threading.Lock()


@dataclass
class Layer:
    """Fused weights in the oracle layout (qvgIn (A, 3D, in), goW (A, D, D))."""
    qvgIn: np.ndarray
    goW: np.ndarray
    input_proj: Optional[np.ndarray]
    ln_gamma: np.ndarray
    ln_beta: np.ndarray
    K: int = 3

    def c(self) -> OracleLayer:
        A, three_d, i = self.qvgIn.shape
        for a in (self.qvgIn, self.goW, self.input_proj, self.ln_gamma, self.ln_beta):
            if a is not None:
                assert a.dtype == np.float32 and a.flags.c_contiguous
        qT, gT = self._input_major()
        return OracleLayer(_fp(self.qvgIn), _fp(self.goW), _fp(self.input_proj),
                           _fp(self.ln_gamma), _fp(self.ln_beta), i, three_d // 3, self.K,
                           _fp(qT), _fp(gT))

    def _input_major(self):
        """Input-major copies of qvgIn and goW for the fp64 step's dot
        products (same sums, same order).  Rebuilt when the weights change;
        every copy handed out lives as long as the layer, so structs built
        earlier never point at freed memory."""
        with _T_LOCK:                   # layers are shared by oracle threads
            t = self.__dict__.get("_t")
            if t is None or not (np.array_equal(t[0], self.qvgIn)
                                 and np.array_equal(t[1], self.goW)):
                self.__dict__.setdefault("_t_old", []).append(t)
                t = (self.qvgIn.copy(), self.goW.copy(),
                     np.ascontiguousarray(self.qvgIn.transpose(0, 2, 1)),
                     np.ascontiguousarray(self.goW.transpose(0, 2, 1)))
                self.__dict__["_t"] = t
            return t[2], t[3]


def reshape(W_in_cat, W_out_cat, qW, vW, gW, oW):
    """oracle_reshape_layer: returns (qvgIn (A, 3D, in), goW (A, D, D))."""
    Win, Wout = _f32(W_in_cat), _f32(W_out_cat)
    q, v, g, o = (_f32(a) for a in (qW, vW, gW, oW))
    in_dim, D = Win.shape[0], q.shape[0]
    A = max(Win.shape[1] // D, Wout.shape[0] // D)
    qvg = np.zeros((A, 3 * D, in_dim), np.float32)
    go = np.zeros((A, D, D), np.float32)
    rc = load().oracle_reshape_layer(_fp(Win), Win.shape[1], _fp(Wout), Wout.shape[0],
                                     _fp(q), _fp(v), _fp(g), _fp(o), in_dim, D, _fp(qvg), _fp(go))
    if rc < 0:
        raise ValueError("oracle_reshape_layer rejected the shapes")
    return qvg, go


def layer_from_raw(raw) -> Layer:
    qvg, go = reshape(raw.W_in_cat, raw.W_out_cat, raw.qW, raw.vW, raw.gW, raw.oW)
    K = 3 if qvg.shape[0] == 9 else 1
    ip = None if raw.input_proj is None else _f32(raw.input_proj)
    return Layer(qvg, go, ip, _f32(raw.ln_gamma), _f32(raw.ln_beta), K)


def layer_step(layer: Layer, x: np.ndarray, H: np.ndarray, ev_x: int, ev_y: int,
               Hl: int, Wl: int, precision: int = 64) -> np.ndarray:
    out = np.zeros(layer.goW.shape[1], np.float32)
    x = _f32(x)
    assert H.dtype == np.float32 and H.flags.c_contiguous
    L = layer.c()
    f = load().oracle_layer_step_f64 if precision == 64 else load().oracle_layer_step_f32
    f(ctypes.byref(L), _fp(x), _fp(H), ev_x, ev_y, Hl, Wl, _fp(out))
    return out


# ---- head -------------------------------------------------------------------

def fuse_conv_bn(W, b_conv, bn_w, bn_b, bn_mu, bn_var, eps: float = 1e-5):
    W = _f32(W).reshape(W.shape[0], -1)
    co, ci = W.shape
    Wo = np.zeros_like(W)
    bo = np.zeros(co, np.float32)
    load().oracle_fuse_conv_bn(_fp(W), _fp(None if b_conv is None else _f32(b_conv)), _fp(_f32(bn_w)),
                               _fp(_f32(bn_b)), _fp(_f32(bn_mu)), _fp(_f32(bn_var)), co, ci, eps,
                               _fp(Wo), _fp(bo))
    return Wo, bo


@dataclass
class Head:
    """Either head kind: the two-branch YOLOX head (BN folded, keys
    cls_conv_W ... obj_pred_b) or the single-linear head (keys lin_W (96, 7)
    in the device's (IN, OUT) layout and lin_b (7,))."""
    arrays: Dict[str, np.ndarray]

    @classmethod
    def linear(cls, W, b) -> "Head":
        W, b = _f32(W), _f32(b)
        if W.shape != (C3, 7) or b.shape != (7,):
            raise ValueError("single-linear head needs W (96, 7) and b (7,)")
        return cls({"lin_W": W, "lin_b": b})

    @property
    def is_linear(self) -> bool:
        return "cls_conv_W" not in self.arrays

    def c(self) -> OracleHead:
        a = self.arrays
        if self.is_linear:
            h = OracleHead()
            h.C = C3
            h.lin_W, h.lin_b = _fp(a["lin_W"]), _fp(a["lin_b"])
            return h
        return OracleHead(*[_fp(a[k]) for k in ("cls_conv_W", "cls_conv_b", "cls_pred_W",
                                                 "cls_pred_b", "reg_conv_W", "reg_conv_b",
                                                 "reg_pred_W", "reg_pred_b", "obj_pred_W",
                                                 "obj_pred_b")], 96)


def head_from_npz(w) -> Head:
    """BN-fold level 0 of a weights.npz mapping (hybrid_common.py:352-409)."""
    a = {}
    for br, tag in (("cls_convs", "cls"), ("reg_convs", "reg")):
        base = f"head/{br}/0"
        bias_key = f"{base}/0/bias"
        b = w[bias_key] if bias_key in w else None
        a[f"{tag}_conv_W"], a[f"{tag}_conv_b"] = fuse_conv_bn(
            w[f"{base}/0/weight"], b, w[f"{base}/1/weight"], w[f"{base}/1/bias"],
            w[f"{base}/1/running_mean"], w[f"{base}/1/running_var"])
    for tag in ("cls", "reg", "obj"):
        a[f"{tag}_pred_W"] = _f32(w[f"head/{tag}_preds/0/weight"]).reshape(-1, 96).copy()
        a[f"{tag}_pred_b"] = _f32(w[f"head/{tag}_preds/0/bias"]).copy()
    return Head(a)


def head_raw(head: Head, x: np.ndarray, precision: int = 64) -> np.ndarray:
    out = np.zeros(7, np.float32)
    h = head.c()
    f = load().oracle_head_raw_f64 if precision == 64 else load().oracle_head_raw_f32
    f(ctypes.byref(h), _fp(_f32(x)), _fp(out))
    return out


# ---- weight directory -------------------------------------------------------------

def load_npz(weights_dir: str) -> Dict[str, np.ndarray]:
    with np.load(str(Path(weights_dir) / "weights.npz"), allow_pickle=False) as z:
        return {k: np.array(z[k]) for k in z.files}


def layers_from_npz(w, first: int = 4) -> List[Layer]:
    """Four layers from position `first` of the sorted SSLA layer indices
    (ssla_kernels.cpp:178-198): 4 gives L4..L7, 0 gives L0..L3."""
    idx = sorted(int(k.split("/")[1]) for k in w if k.startswith("layers/") and k.endswith("/W_in_cat"))
    out = []
    for li in range(4):
        p = f"layers/{idx[first + li]}"
        qvg, go = reshape(w[f"{p}/W_in_cat"], w[f"{p}/W_out_cat"], w[f"{p}/q_proj/weight"],
                          w[f"{p}/v_proj/weight"], w[f"{p}/g_proj/weight"], w[f"{p}/o_proj/weight"])
        ipk = f"{p}/input_proj/weight"
        out.append(Layer(qvg, go, _f32(w[ipk]) if ipk in w else None,
                         _f32(w[f"{p}/norm/weight"]), _f32(w[f"{p}/norm/bias"]),
                         3 if qvg.shape[0] == 9 else 1))
    return out


# ---- the drain schedule ---------------------------------------------------------------

class S2S3:
    """One drain instance: layers L4..L7, hidden state, tdrop counters."""

    def __init__(self, layers: Sequence[Layer], H2: int, W2: int, window: int,
                 h_init: Optional[Sequence[np.ndarray]] = None, head: Optional[Head] = None):
        self.layers = list(layers)
        self.H2, self.W2, self.H3, self.W3 = H2, W2, H2 >> 1, W2 >> 1
        self.window = window
        cells = (H2 * W2, H2 * W2, self.H3 * self.W3, self.H3 * self.W3)
        self.H = [np.zeros((cells[li], GPU_LAYER_IO[li][1]), np.float32) for li in range(4)]
        if h_init is not None:
            for li in range(4):
                self.H[li][...] = h_init[li]
        self.td2 = np.zeros(H2 * W2, np.uint8)
        self.td3 = np.zeros(self.H3 * self.W3, np.uint8)
        self.head = head

    def run(self, x, y, feat1, owner=None, precision: int = 64, want_feat: bool = True,
            want_head: bool = False):
        n = len(x)
        x = np.ascontiguousarray(x, np.uint16)
        y = np.ascontiguousarray(y, np.uint16)
        f = _f32(feat1).reshape(n, C1)
        own = None if owner is None else np.ascontiguousarray(owner, np.uint8)
        p2 = np.zeros(n, np.int8)
        p3 = np.zeros(n, np.int8)
        feat = np.zeros((n, C3), np.float32) if want_feat else None
        head7 = np.zeros((n, 7), np.float32) if want_head else None
        st = OracleS2S3()
        for li in range(4):
            st.L[li] = self.layers[li].c()
            st.H[li] = _fp(self.H[li])
        st.td2 = self.td2.ctypes.data_as(ctypes.POINTER(ctypes.c_uint8))
        st.td3 = self.td3.ctypes.data_as(ctypes.POINTER(ctypes.c_uint8))
        st.H2, st.W2, st.H3, st.W3 = self.H2, self.W2, self.H3, self.W3
        st.window = self.window
        hc = None
        if want_head:
            if self.head is None:
                raise ValueError("no head weights")
            hc = self.head.c()
            st.head = ctypes.pointer(hc)
        rc = load().oracle_s2s3_run(ctypes.byref(st), x.ctypes.data, y.ctypes.data, f.ctypes.data,
                                    None if own is None else own.ctypes.data, n, precision,
                                    p2.ctypes.data, p3.ctypes.data,
                                    None if feat is None else feat.ctypes.data,
                                    None if head7 is None else head7.ctypes.data)
        if rc < 0:
            raise ValueError("oracle_s2s3_run rejected its arguments")
        return p2, p3, feat, head7


class S01:
    """One producer shard over stages 0 + 1 (oracle_s01_run): layers L0..L3,
    hidden state, tdrop counters and per-pixel last event times."""

    def __init__(self, layers: Sequence[Layer], height: int, width: int, window: int):
        self.layers = list(layers)
        self.height, self.width, self.window = height, width, window
        c0, c1 = height * width, (height // 2) * (width // 2)
        dims = [L.goW.shape[1] for L in self.layers]
        self.H = [np.zeros((c, d), np.float32) for c, d in zip((c0, c0, c1, c1), dims)]
        self.td0 = np.zeros(c1, np.uint8)
        self.td1 = np.zeros((height // 4) * (width // 4), np.uint8)
        self.last_t = np.full(c0, -1.0, np.float64)

    def run(self, events: np.ndarray, owner=None, precision: int = 64):
        """events (n, 4) [t_us, x, y, p] -> (pass0, pass1, feat1 (n, 24), x2, y2)."""
        ev = _f32(events).reshape(-1, 4)
        n = ev.shape[0]
        own = None if owner is None else np.ascontiguousarray(owner, np.uint8)
        p0 = np.zeros(n, np.int8)
        p1 = np.zeros(n, np.int8)
        feat = np.zeros((n, C1), np.float32)
        x2 = np.zeros(n, np.uint16)
        y2 = np.zeros(n, np.uint16)
        st = OracleS01()
        for li in range(4):
            st.L[li] = self.layers[li].c()
            st.H[li] = _fp(self.H[li])
        st.td0 = self.td0.ctypes.data_as(ctypes.POINTER(ctypes.c_uint8))
        st.td1 = self.td1.ctypes.data_as(ctypes.POINTER(ctypes.c_uint8))
        st.last_t = self.last_t.ctypes.data_as(ctypes.POINTER(ctypes.c_double))
        st.height, st.width, st.window = self.height, self.width, self.window
        rc = load().oracle_s01_run(ctypes.byref(st), ev.ctypes.data,
                                   None if own is None else own.ctypes.data, n, precision,
                                   p0.ctypes.data, p1.ctypes.data, feat.ctypes.data,
                                   x2.ctypes.data, y2.ctypes.data)
        if rc < 0:
            raise ValueError("oracle_s01_run rejected its arguments")
        return p0, p1, feat, x2, y2


def preprocess(last_t: np.ndarray, height: int, width: int, t_us: float, x: int, y: int,
               p: float) -> np.ndarray:
    """oracle_preprocess on a (height*width,) float64 last-time array."""
    assert last_t.dtype == np.float64 and last_t.flags.c_contiguous
    out = np.zeros(2, np.float32)
    load().oracle_preprocess(last_t.ctypes.data, height, width, t_us, x, y, p, _fp(out))
    return out


def decisions(x, y, H2: int, W2: int, window: int, td2=None, td3=None):
    """Pass flags only (the same tdrop schedule), for full-size checks."""
    n = len(x)
    x = np.ascontiguousarray(x, np.uint16)
    y = np.ascontiguousarray(y, np.uint16)
    td2 = np.zeros(H2 * W2, np.uint8) if td2 is None else td2
    td3 = np.zeros((H2 >> 1) * (W2 >> 1), np.uint8) if td3 is None else td3
    p2 = np.zeros(n, np.int8)
    p3 = np.zeros(n, np.int8)
    load().oracle_s2s3_decisions(td2.ctypes.data, td3.ctypes.data, H2, W2, window,
                                 x.ctypes.data, y.ctypes.data, n, p2.ctypes.data, p3.ctypes.data)
    return p2, p3, td2, td3


# ---- the reference checker (oracle/_ref) ------------------------------------------

def load_ref() -> Optional[ctypes.CDLL]:
    """libssla_ref.so built from the reference's own CPU sources, or None."""
    if not REF_LIB_PATH.exists():
        return None
    L = ctypes.CDLL(str(REF_LIB_PATH))
    L.ref_meta.restype = ctypes.c_int
    L.ref_meta.argtypes = [ctypes.c_char_p, ctypes.POINTER(ctypes.c_int)]
    L.ref_tensor.restype = ctypes.c_int
    L.ref_tensor.argtypes = [ctypes.c_char_p, ctypes.c_char_p, _FP, ctypes.c_int]
    L.ref_head_decode.restype = ctypes.c_int
    L.ref_head_decode.argtypes = [ctypes.c_char_p, ctypes.c_int, ctypes.c_int, _FP, _FP]
    L.ref_layernorm.restype = ctypes.c_int
    L.ref_layernorm.argtypes = [_FP, ctypes.c_int, _FP, _FP]
    L.ref_lru_step.restype = ctypes.c_int
    L.ref_lru_step.argtypes = [_FP, _FP, _FP, _FP, _FP, ctypes.c_int]
    L.ref_mm.restype = ctypes.c_int
    L.ref_mm.argtypes = [_FP, ctypes.c_int, ctypes.c_int, _FP, ctypes.c_int, _FP]
    if hasattr(L, "ref_matvec96x7"):
        L.ref_matvec96x7.restype = ctypes.c_int
        L.ref_matvec96x7.argtypes = [_FP, _FP, _FP, _FP]
    if hasattr(L, "ref_oeva_record"):
        L.ref_oeva_record.restype = ctypes.c_int
        L.ref_oeva_record.argtypes = [ctypes.c_char_p, ctypes.c_int, ctypes.c_int,
                                      ctypes.c_ulonglong, ctypes.c_int,
                                      ctypes.POINTER(ctypes.c_ulonglong), _FP,
                                      ctypes.POINTER(ctypes.c_int)]
        L.ref_oeva_diff.restype = ctypes.c_int
        L.ref_oeva_diff.argtypes = [ctypes.c_char_p, ctypes.c_char_p, ctypes.c_double,
                                    ctypes.POINTER(ctypes.c_double)]
    return L
