"""Random stub weight directory in the SSLA-S export schema.

Writes <dir>/weights.npz (stored, uncompressed) and <dir>/meta.json with the
keys, shapes, scales and random-draw order of tools/make_ssla_stub.py:29-149,
so a directory made here with seed s holds the same tensors the reference
tool writes with --seed s (same numpy Generator stream).

Layer schema (tools/make_ssla_stub.py:29-49), for layer li with (in, out, K):
  layers/li/W_in_cat           (in, K*K*out)   N(0, 0.3)
  layers/li/W_out_cat          (K*K*out, out)  N(0, 0.3)
  layers/li/{q,v,g,o}_proj/weight (out, out)   N(0, 0.3)
  layers/li/input_proj/weight  (out, in)       N(0, 0.3), only if in != out
  layers/li/norm/weight        (out,)          1 + N(0, 0.1)
  layers/li/norm/bias          (out,)          N(0, 0.1)
Head level k (tools/make_ssla_stub.py:52-81): conv 1x1 N(0, 0.1), BN gamma
1 + N(0, 0.05), beta N(0, 0.05), running mean 0, var 1 for cls_convs and
reg_convs, then cls/reg/obj preds N(0, 0.05).
"""
from __future__ import annotations

import argparse
import json
import os
from typing import Dict

import numpy as np

IN_DIM = 2
CHANNELS = (12, 24, 48, 96)

# (in, out, K) of the 8 SSLA-S layers, two per stage
LAYERS = ((2, 12, 1), (12, 12, 3), (12, 24, 3), (24, 24, 3),
          (24, 48, 3), (48, 48, 3), (48, 96, 3), (96, 96, 3))


def _layer(rng: np.random.Generator, name: str, i: int, o: int, k: int,
           w: Dict[str, np.ndarray]) -> None:
    a = k * k
    f32 = np.float32
    w[f"{name}/W_in_cat"] = rng.normal(scale=0.3, size=(i, a * o)).astype(f32)
    w[f"{name}/W_out_cat"] = rng.normal(scale=0.3, size=(a * o, o)).astype(f32)
    for proj in ("q", "v", "g", "o"):
        w[f"{name}/{proj}_proj/weight"] = rng.normal(scale=0.3, size=(o, o)).astype(f32)
    if i != o:
        w[f"{name}/input_proj/weight"] = rng.normal(scale=0.3, size=(o, i)).astype(f32)
    w[f"{name}/norm/weight"] = (rng.normal(scale=0.1, size=(o,)) + 1.0).astype(f32)
    w[f"{name}/norm/bias"] = rng.normal(scale=0.1, size=(o,)).astype(f32)


def _head_level(rng: np.random.Generator, k: int, c_in: int, c_hid: int, n_cls: int,
                w: Dict[str, np.ndarray]) -> None:
    f32 = np.float32
    for branch in ("cls_convs", "reg_convs"):
        base = f"head/{branch}/{k}"
        w[f"{base}/0/weight"] = rng.normal(scale=0.1, size=(c_hid, c_in)).astype(f32)
        w[f"{base}/1/weight"] = (rng.normal(scale=0.05, size=(c_hid,)) + 1.0).astype(f32)
        w[f"{base}/1/bias"] = rng.normal(scale=0.05, size=(c_hid,)).astype(f32)
        w[f"{base}/1/running_mean"] = np.zeros((c_hid,), dtype=f32)
        w[f"{base}/1/running_var"] = np.ones((c_hid,), dtype=f32)
    for pred, rows in (("cls_preds", n_cls), ("reg_preds", 4), ("obj_preds", 1)):
        w[f"head/{pred}/{k}/weight"] = rng.normal(scale=0.05, size=(rows, c_hid)).astype(f32)
        w[f"head/{pred}/{k}/bias"] = rng.normal(scale=0.05, size=(rows,)).astype(f32)


def make_weights(seed: int = 1, num_classes: int = 2,
                 num_head_levels: int = 1) -> Dict[str, np.ndarray]:
    rng = np.random.default_rng(seed)
    w: Dict[str, np.ndarray] = {}
    for li, (i, o, k) in enumerate(LAYERS):
        _layer(rng, f"layers/{li}", i, o, k, w)
    n_stages = len(CHANNELS)
    for k in range(num_head_levels):
        stage = n_stages - num_head_levels + k
        _head_level(rng, k, CHANNELS[stage], CHANNELS[-1], num_classes, w)
    return w


def write_stub(out_dir: str, *, height: int = 64, width: int = 80,
               num_classes: int = 2, tdrop: int = 4, seed: int = 1,
               num_head_levels: int = 1) -> str:
    os.makedirs(out_dir, exist_ok=True)
    w = make_weights(seed, num_classes, num_head_levels)
    np.savez(os.path.join(out_dir, "weights.npz"), **w)
    meta = {
        "schema_version": 1,
        "model": "ssla_s_yolox_det",
        "method": "ssla",
        "height": height,
        "width": width,
        "num_classes": num_classes,
        "num_anchors": 1,
        "ssla_tdrop_window": tdrop,
        "dtype": "float32",
        "layout": "C_order_row_major",
        "key_separator": "/",
        "checkpoint": "stub_random",
        "total_params": int(sum(int(np.prod(a.shape)) for a in w.values())),
    }
    with open(os.path.join(out_dir, "meta.json"), "w") as f:
        json.dump(meta, f, indent=2)
    return out_dir


def main() -> None:
    ap = argparse.ArgumentParser(description=__doc__.splitlines()[0])
    ap.add_argument("out_dir")
    ap.add_argument("--h", type=int, default=64)
    ap.add_argument("--w", type=int, default=80)
    ap.add_argument("--num-classes", type=int, default=2)
    ap.add_argument("--tdrop", type=int, default=4)
    ap.add_argument("--seed", type=int, default=1)
    ap.add_argument("--num-head-levels", type=int, default=1)
    a = ap.parse_args()
    write_stub(a.out_dir, height=a.h, width=a.w, num_classes=a.num_classes,
               tdrop=a.tdrop, seed=a.seed, num_head_levels=a.num_head_levels)


if __name__ == "__main__":
    main()
