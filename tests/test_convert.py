"""Trained-checkpoint conversion (tools/convert_dsec_ckpt.py) and the
weight-directory readers on a converted directory.

Pins: the slot remap {0,1,4,5,8,9,12,13} -> 0..7 and dropped keys against a
synthetic checkpoint whose tensors are known; the converted directory read
back by the reference's own C++ loader (oracle/_ref, weights_loader.cpp);
the head with real BatchNorm statistics and conv biases against the
reference's load_yolox_level + decode_yolox_cell_ct.
"""
import ctypes
import json

import numpy as np
import pytest

from conftest import make_trained_checkpoint
from oracle import oracle as O
from ssla_hip import convert, grid, lib


def fp(a):
    return a.ctypes.data_as(ctypes.POINTER(ctypes.c_float))


def test_convert_remaps_slots_and_keeps_head(tmp_path):
    ck, ema, live = make_trained_checkpoint(tmp_path / "m.ckpt")
    rep, meta = convert.convert(str(tmp_path / "m.ckpt"), str(tmp_path / "out"), h=64, w=80)
    assert rep.source == "ema_state_dict" and rep.tdrop_window == 6 and rep.num_classes == 2
    got = dict(np.load(tmp_path / "out" / "weights.npz"))
    assert sorted(got) == sorted(ema)
    for k, v in ema.items():
        assert got[k].dtype == np.float32 and np.array_equal(got[k], v), k
    assert got["head/cls_convs/0/0/weight"].shape == (96, 96, 1, 1)
    assert rep.n_skipped == 4 + 2 + 1            # 4 LUTs, 2 BN counters, 1 unknown key
    assert len(rep.warnings) == 2                # layer slot 2, criterion.weight
    m = json.loads((tmp_path / "out" / "meta.json").read_text())
    assert m == meta
    assert (m["height"], m["width"], m["ssla_tdrop_window"], m["num_classes"]) == (64, 80, 6, 2)
    assert (m["ckpt_epoch"], m["ckpt_global_step"]) == (7, 1234)
    assert (m["ckpt_native_h"], m["ckpt_native_w"]) == (430, 640)
    assert m["model"] == "ssla_s_yolox_det" and m["source_state_dict"] == "ema_state_dict"
    assert m["total_params"] == sum(int(np.prod(v.shape)) for v in ema.values())


def test_convert_live_state_dict(tmp_path):
    make_trained_checkpoint(tmp_path / "m.ckpt")
    rep, _ = convert.convert(str(tmp_path / "m.ckpt"), str(tmp_path / "a"), use_ema=False)
    _, _, live = make_trained_checkpoint(tmp_path / "m2.ckpt", with_ema=False)
    rep2, meta2 = convert.convert(str(tmp_path / "m2.ckpt"), str(tmp_path / "b"))
    assert rep.source == rep2.source == "state_dict"
    a, b = dict(np.load(tmp_path / "a" / "weights.npz")), dict(np.load(tmp_path / "b" / "weights.npz"))
    for k, v in live.items():
        assert np.array_equal(a[k], v) and np.array_equal(b[k], v), k
    assert (meta2["height"], meta2["width"]) == (120, 160)   # defaults


def test_convert_cli_and_defaults(tmp_path, capsys):
    import torch
    torch.save({"state_dict": {"layers.0.norm.weight": torch.ones(12)}}, str(tmp_path / "s.ckpt"))
    assert convert.main([str(tmp_path / "s.ckpt"), str(tmp_path / "o"), "--h", "32",
                         "--w", "48"]) == 0
    m = json.loads((tmp_path / "o" / "meta.json").read_text())
    assert (m["ssla_tdrop_window"], m["num_classes"], m["ckpt_epoch"]) == (4, 2, -1)
    assert "kept 1 layer + 0 head" in capsys.readouterr().out


class _NotATensor:
    pass


def test_convert_refuses_code_in_checkpoint(tmp_path):
    import torch
    torch.save({"state_dict": {}, "hyper_parameters": {"x": _NotATensor()}},
               str(tmp_path / "bad.ckpt"))
    with pytest.raises(ValueError, match="weights-only"):
        convert.convert(str(tmp_path / "bad.ckpt"), str(tmp_path / "o"))


def test_converted_dir_reads_back_through_reference_loader(trained_dir):
    R = O.load_ref()
    if R is None:
        pytest.skip("oracle/_ref not built (reference checkout absent)")
    meta = (ctypes.c_int * 4)()
    assert R.ref_meta(trained_dir.encode(), meta) == 0
    assert list(meta) == [64, 80, 2, 6]
    L = lib.load()
    ours = (ctypes.c_int * 4)()
    lib.check(L.ssla_hip_meta_read(trained_dir.encode(), ours))
    assert list(ours) == list(meta)
    w = dict(np.load(f"{trained_dir}/weights.npz"))
    for k in ("layers/7/W_in_cat", "head/cls_convs/0/0/weight", "head/reg_convs/0/1/running_var",
              "head/cls_convs/0/0/bias"):
        buf = np.zeros(w[k].size, np.float32)
        assert R.ref_tensor(trained_dir.encode(), k.encode(), fp(buf), buf.size) == buf.size
        assert np.array_equal(buf, w[k].reshape(-1)), k
        got = np.zeros(w[k].size, np.float32)
        assert L.ssla_hip_npz_read(trained_dir.encode(), k.encode(), fp(got), got.size,
                                   None, None) == got.size
        assert np.array_equal(got, buf), k


def test_trained_head_matches_reference(trained_dir):
    """Real BN statistics and conv biases: the product's host head and the
    oracle's head against the reference's folded head."""
    R = O.load_ref()
    if R is None:
        pytest.skip("oracle/_ref not built (reference checkout absent)")
    head = O.head_from_npz(O.load_npz(trained_dir))
    rng = np.random.default_rng(8)
    for k in range(16):
        x = np.zeros(96, np.float32) if k == 0 else rng.normal(0, 1, 96).astype(np.float32)
        gx, gy = int(rng.integers(0, 10)), int(rng.integers(0, 8))
        ref = np.zeros(7, np.float32)
        assert R.ref_head_decode(trained_dir.encode(), gx, gy, fp(x), fp(ref)) == 7
        ours = grid.decode_cells(grid.head_row(trained_dir, x)[None], grid_w=10, gx0=gx, gy0=gy)[0]
        assert np.allclose(ours, ref, rtol=1e-5, atol=2e-5), (k, ours, ref)
        ora = grid.decode_cells(O.head_raw(head, x)[None], grid_w=10, gx0=gx, gy0=gy)[0]
        assert np.allclose(ora, ref, rtol=1e-5, atol=2e-5), (k, ora, ref)


def test_trained_dir_runs_through_oracle_stages(trained_dir):
    """The converted directory drives stages 0..3 of the oracle with the
    same layers as the weights it was made from."""
    from ssla_hip import stub
    w = O.load_npz(trained_dir)
    ref = stub.make_weights(3)
    got = O.layers_from_npz(w)
    want = O.layers_from_npz(ref)
    for a, b in zip(got, want):
        for f in ("qvgIn", "goW", "ln_gamma", "ln_beta"):
            assert np.array_equal(getattr(a, f), getattr(b, f)), f
