"""Shared fixtures.  Tests marked `gpu` need an MI355X; the rest run on CPU."""
import os
import sys
from pathlib import Path

import numpy as np
import pytest

ROOT = Path(__file__).resolve().parent.parent
for p in (str(ROOT), str(ROOT / "ssla-rt_amd")):
    if p not in sys.path:
        sys.path.insert(0, p)


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs a gfx950 GPU (run with -m gpu)")


@pytest.fixture(scope="session")
def stub_dir(tmp_path_factory):
    """Stub weight directory at 80x64, seed 1, tdrop 4 (the CPU-reference config)."""
    from ssla_hip import stub
    d = tmp_path_factory.mktemp("stub_80x64")
    stub.write_stub(str(d), height=64, width=80, seed=1, tdrop=4)
    return str(d)


@pytest.fixture(scope="session")
def stub_npz(stub_dir):
    from oracle import oracle
    return oracle.load_npz(stub_dir)


@pytest.fixture(scope="session")
def stub_w1_dir(tmp_path_factory):
    """Stub weight directory at 80x64, seed 5, tdrop window 1: every record
    passes both gates, so every record has head outputs."""
    from ssla_hip import stub
    d = tmp_path_factory.mktemp("stub_80x64_w1")
    stub.write_stub(str(d), height=64, width=80, seed=5, tdrop=1)
    return str(d)


@pytest.fixture(scope="session")
def stub_640(tmp_path_factory):
    """Stub weight directory at 640x480 (s2 160 x 120), seed 1, tdrop 4."""
    from ssla_hip import stub
    d = tmp_path_factory.mktemp("stub_640x480")
    stub.write_stub(str(d), height=480, width=640, seed=1, tdrop=4)
    return str(d)


def make_trained_checkpoint(path, seed: int = 3, tdrop: int = 6, with_ema: bool = True):
    """A Lightning-style checkpoint with the tensor names of a trained SSLA-S
    model: SSLA layers at slots 0,1,4,5,8,9,12,13, 4-D head convs with
    biases, BatchNorm statistics away from (0, 1), pixel2patch_lut buffers,
    num_batches_tracked counters, one stray layer slot and one unknown key.
    Returns (checkpoint dict, expected weight-directory tensors of the EMA
    and of the live state dict)."""
    import torch
    from ssla_hip import stub
    rng = np.random.default_rng(seed + 100)
    w = stub.make_weights(seed)
    deploy_to_slot = {0: 0, 1: 1, 2: 4, 3: 5, 4: 8, 5: 9, 6: 12, 7: 13}
    for br in ("cls_convs", "reg_convs"):
        base = f"head/{br}/0"
        w[f"{base}/0/weight"] = w[f"{base}/0/weight"].reshape(96, 96, 1, 1)
        w[f"{base}/0/bias"] = rng.normal(0, 0.1, 96).astype(np.float32)
        w[f"{base}/1/running_mean"] = rng.normal(0, 0.2, 96).astype(np.float32)
        w[f"{base}/1/running_var"] = rng.uniform(0.3, 2.5, 96).astype(np.float32)
    live = {k: (v + rng.normal(0, 0.01, v.shape)).astype(np.float32) for k, v in w.items()}
    for k in live:
        if k.endswith("running_var"):
            live[k] = np.abs(live[k]) + 0.1

    def state_dict(src):
        sd = {}
        for k, v in src.items():
            parts = k.split("/")
            if parts[0] == "layers":
                parts[1] = str(deploy_to_slot[int(parts[1])])
            sd[".".join(parts)] = torch.from_numpy(v.copy())
        for slot in (1, 5, 9, 13):
            sd[f"layers.{slot}.pixel2patch_lut"] = torch.arange(9, dtype=torch.int64)
        sd["head.cls_convs.0.1.num_batches_tracked"] = torch.tensor(1000)
        sd["head.reg_convs.0.1.num_batches_tracked"] = torch.tensor(1000)
        sd["layers.2.scale"] = torch.ones(3)
        sd["criterion.weight"] = torch.ones(2)
        return sd

    ck = {"epoch": 7, "global_step": 1234, "state_dict": state_dict(live),
          "hyper_parameters": {"num_classes": 2, "height": 430, "width": 640,
                               "stages": [{"layers": [{"type": "ssla"}, {"type": "ssla"}]},
                                          {"layers": [{"type": "spatial_downsample"},
                                                      {"type": "temporal_dropout",
                                                       "window": tdrop}]}]}}
    if with_ema:
        ck["ema_state_dict"] = state_dict(w)
    torch.save(ck, str(path))
    return ck, w, live


@pytest.fixture(scope="session")
def trained_dir(tmp_path_factory):
    """Weight directory (80x64) converted from a synthetic trained
    checkpoint with conv biases and real BatchNorm statistics."""
    from ssla_hip import convert
    d = tmp_path_factory.mktemp("trained")
    make_trained_checkpoint(d / "model.ckpt")
    convert.convert(str(d / "model.ckpt"), str(d / "weights"), h=64, w=80)
    return str(d / "weights")


@pytest.fixture(scope="session")
def headless_dir(tmp_path_factory):
    """Stub weight directory at 80x64, seed 1, tdrop 4 with no head keys
    (make_ssla_stub --num-head-levels 0): the layers equal stub_dir's, and
    the reference's live runner falls back to a single-linear head."""
    from ssla_hip import stub
    d = tmp_path_factory.mktemp("stub_80x64_headless")
    stub.write_stub(str(d), height=64, width=80, seed=1, tdrop=4, num_head_levels=0)
    return str(d)
