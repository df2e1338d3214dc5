"""The weight-directory schema (tools/make_ssla_stub.py:29-149) and the
product's host reader (libssla_hip.so: ssla_hip_npz_read / meta_read),
checked against numpy's reader and the reference's C++ loader
(vendor/src/weights_loader.cpp, compiled into oracle/_ref).  CPU only: no
call here touches a GPU."""
import ctypes
import json
import os
import zipfile

import numpy as np
import pytest

from oracle import oracle as O
from ssla_hip import lib, stub

EXPECTED_LAYERS = ((2, 12, 1), (12, 12, 3), (12, 24, 3), (24, 24, 3),
                   (24, 48, 3), (48, 48, 3), (48, 96, 3), (96, 96, 3))


def test_stub_schema(stub_dir, stub_npz):
    w = stub_npz
    for li, (i, o, k) in enumerate(EXPECTED_LAYERS):
        p = f"layers/{li}"
        assert w[f"{p}/W_in_cat"].shape == (i, k * k * o)
        assert w[f"{p}/W_out_cat"].shape == (k * k * o, o)
        for proj in "qvgo":
            assert w[f"{p}/{proj}_proj/weight"].shape == (o, o)
        assert (f"{p}/input_proj/weight" in w) == (i != o)
        if i != o:
            assert w[f"{p}/input_proj/weight"].shape == (o, i)
        assert w[f"{p}/norm/weight"].shape == (o,) and w[f"{p}/norm/bias"].shape == (o,)
    for br in ("cls_convs", "reg_convs"):
        assert w[f"head/{br}/0/0/weight"].shape == (96, 96)
        assert np.all(w[f"head/{br}/0/1/running_var"] == 1)
        assert np.all(w[f"head/{br}/0/1/running_mean"] == 0)
    assert w["head/cls_preds/0/weight"].shape == (2, 96)
    assert w["head/reg_preds/0/weight"].shape == (4, 96)
    assert w["head/obj_preds/0/weight"].shape == (1, 96)
    assert all(a.dtype == np.float32 for a in w.values())
    meta = json.load(open(os.path.join(stub_dir, "meta.json")))
    assert meta["schema_version"] == 1 and meta["model"] == "ssla_s_yolox_det"
    assert (meta["height"], meta["width"], meta["ssla_tdrop_window"]) == (64, 80, 4)
    assert meta["total_params"] == sum(a.size for a in w.values())
    with zipfile.ZipFile(os.path.join(stub_dir, "weights.npz")) as z:
        assert all(info.compress_type == zipfile.ZIP_STORED for info in z.infolist())


def test_stub_is_deterministic(tmp_path):
    a = stub.make_weights(seed=1)
    b = stub.make_weights(seed=1)
    c = stub.make_weights(seed=2)
    assert a.keys() == b.keys()
    assert all(np.array_equal(a[k], b[k]) for k in a)
    assert not np.array_equal(a["layers/4/W_in_cat"], c["layers/4/W_in_cat"])


def _lib_read(d, key):
    L = lib.load()
    shape = (ctypes.c_longlong * 4)()
    nd = ctypes.c_int()
    n = L.ssla_hip_npz_read(d.encode(), key.encode(), None, 0, shape, ctypes.byref(nd))
    lib.check(n, key)
    out = np.zeros(n, np.float32)
    lib.check(L.ssla_hip_npz_read(d.encode(), key.encode(),
                                  out.ctypes.data_as(ctypes.POINTER(ctypes.c_float)), n, None, None))
    return out.reshape(tuple(shape[:nd.value]))


def test_library_reader_matches_numpy(stub_dir, stub_npz):
    for k in ("layers/4/W_in_cat", "layers/7/o_proj/weight", "layers/6/input_proj/weight",
              "head/cls_convs/0/1/running_var", "head/obj_preds/0/bias"):
        got = _lib_read(stub_dir, k)
        assert got.shape == stub_npz[k].shape and np.array_equal(got, stub_npz[k])
    meta = (ctypes.c_int * 4)()
    lib.check(lib.load().ssla_hip_meta_read(stub_dir.encode(), meta))
    assert list(meta) == [64, 80, 2, 4]


def test_library_reader_matches_reference_loader(stub_dir):
    R = O.load_ref()
    if R is None:
        pytest.skip("oracle/_ref not built (reference checkout absent)")
    meta = (ctypes.c_int * 4)()
    assert R.ref_meta(stub_dir.encode(), meta) == 0
    assert list(meta) == [64, 80, 2, 4]
    buf = np.zeros(96 * 96 * 9, np.float32)
    for k in ("layers/5/W_out_cat", "head/reg_convs/0/0/weight", "layers/0/W_in_cat"):
        n = R.ref_tensor(stub_dir.encode(), k.encode(),
                         buf.ctypes.data_as(ctypes.POINTER(ctypes.c_float)), buf.size)
        assert n > 0
        assert np.array_equal(buf[:n], _lib_read(stub_dir, k).ravel())


def test_reader_zip64_members(tmp_path):
    # force_zip64 members carry 0xFFFFFFFF sizes plus a ZIP64 extra field
    d = tmp_path / "z64"
    d.mkdir()
    a = np.arange(12, dtype=np.float32).reshape(3, 4)
    with zipfile.ZipFile(d / "weights.npz", "w", zipfile.ZIP_STORED) as z:
        with z.open("t.npy", "w", force_zip64=True) as f:
            np.lib.format.write_array(f, a)
    assert np.array_equal(_lib_read(str(d), "t"), a)


@pytest.mark.parametrize("case", ["compressed", "float64", "missing", "schema"])
def test_reader_rejects_bad_directories(tmp_path, case):
    d = tmp_path / case
    d.mkdir()
    a = np.ones((2, 3), np.float32)
    if case == "compressed":
        np.savez_compressed(d / "weights.npz", t=a)
    elif case == "float64":
        np.savez(d / "weights.npz", t=a.astype(np.float64))
    else:
        np.savez(d / "weights.npz", t=a)
    json.dump({"schema_version": 2 if case == "schema" else 1, "model": "ssla_s_yolox_det",
               "height": 64, "width": 80}, open(d / "meta.json", "w"))
    L = lib.load()
    key = b"nope" if case == "missing" else b"t"
    rc = L.ssla_hip_npz_read(str(d).encode(), key, None, 0, None, None)
    if case == "schema":
        assert rc >= 0
        assert L.ssla_hip_meta_read(str(d).encode(), (ctypes.c_int * 4)()) < 0
    else:
        assert rc < 0
        assert L.ssla_hip_last_error()
