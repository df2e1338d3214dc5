"""Trained SSLA-S checkpoint -> weight directory (weights.npz + meta.json).

Same job, arguments and output schema as tools/convert_dsec_ckpt.py:
  * the checkpoint keeps its SSLA layers at indices 0,1,4,5,8,9,12,13 (the
    slots between hold parameter-free downsample / temporal-dropout ops);
    they become layers 0..7 of the weight directory (:26);
  * ema_state_dict is used when present unless use_ema is off (:46-52);
  * pixel2patch_lut buffers and BatchNorm num_batches_tracked counters are
    dropped (:29, :68-71); every other head tensor -- conv biases and the
    real BatchNorm running statistics included -- is kept under its
    '/'-separated name (:88-91);
  * the temporal-dropout window is the first one named in
    hyper_parameters.stages[*].layers[*] (default 4), num_classes defaults
    to 2 (:56-63);
  * weights.npz is written uncompressed, as the weight-directory readers
    require, and meta.json carries the keys of :100-119.

One difference on purpose: the checkpoint is opened with
torch.load(weights_only=True), which executes nothing from the file.  A
checkpoint that needs arbitrary Python objects to load is refused with a
ValueError naming what the safe loader rejected.
"""
from __future__ import annotations

import argparse
import json
import os
import sys
from dataclasses import dataclass, field
from typing import Dict, List, Mapping, Optional, Tuple

import numpy as np

# checkpoint layer slot -> weight-directory layer index
CKPT_TO_DEPLOY_IDX = {0: 0, 1: 1, 4: 2, 5: 3, 8: 4, 9: 5, 12: 6, 13: 7}
SKIP_SUFFIXES = ("pixel2patch_lut", "num_batches_tracked")


@dataclass
class ConvertReport:
    source: str
    num_classes: int
    tdrop_window: int
    n_layer: int = 0
    n_head: int = 0
    n_skipped: int = 0
    warnings: List[str] = field(default_factory=list)


def load_checkpoint(path: str) -> dict:
    """torch.load(path, weights_only=True) on the CPU."""
    import torch
    try:
        return torch.load(path, map_location="cpu", weights_only=True)
    except Exception as e:   # UnpicklingError and friends name the rejected global
        raise ValueError(f"{path}: the weights-only loader refused the checkpoint ({e}); "
                         "re-save it with plain tensors and containers") from e


def _to_f32(t) -> np.ndarray:
    if hasattr(t, "detach"):
        import torch
        return t.detach().cpu().to(torch.float32).numpy()
    return np.asarray(t, dtype=np.float32)


def tdrop_window(hparams: Mapping) -> int:
    for stage in hparams.get("stages", []) or []:
        for layer in stage.get("layers", []) or []:
            if layer.get("type") == "temporal_dropout":
                return int(layer["window"])
    return 4


def remap_state_dict(sd: Mapping, report: ConvertReport) -> Dict[str, np.ndarray]:
    """Checkpoint tensor names -> weight-directory keys (dots become '/';
    layer slots renumbered by CKPT_TO_DEPLOY_IDX)."""
    out: Dict[str, np.ndarray] = {}
    for name, tensor in sd.items():
        if name.endswith(SKIP_SUFFIXES):
            report.n_skipped += 1
            continue
        parts = name.split(".")
        if parts[0] == "layers" and len(parts) > 2:
            slot = int(parts[1])
            if slot not in CKPT_TO_DEPLOY_IDX:
                report.warnings.append(f"skipping {name} (layer slot {slot} holds no SSLA layer)")
                continue
            out["/".join(["layers", str(CKPT_TO_DEPLOY_IDX[slot])] + parts[2:])] = _to_f32(tensor)
            report.n_layer += 1
        elif parts[0] == "head":
            out["/".join(parts)] = _to_f32(tensor)
            report.n_head += 1
        else:
            report.warnings.append(f"unrecognized key {name}; skipping")
            report.n_skipped += 1
    return out


def convert(ckpt, out_dir: str, h: int = 120, w: int = 160, use_ema: bool = True,
            ckpt_path: Optional[str] = None) -> Tuple[ConvertReport, dict]:
    """ckpt: a path or an already loaded checkpoint dict.  Writes
    out_dir/weights.npz and out_dir/meta.json; returns (report, meta)."""
    if isinstance(ckpt, (str, os.PathLike)):
        ckpt_path = str(ckpt)
        ck = load_checkpoint(ckpt_path)
    else:
        ck = ckpt
    sd = ck.get("ema_state_dict") if use_ema else None
    src = "ema_state_dict"
    if sd is None:
        sd, src = ck["state_dict"], "state_dict"
    hp = ck.get("hyper_parameters", {}) or {}
    report = ConvertReport(src, int(hp.get("num_classes", 2)), tdrop_window(hp))
    weights = remap_state_dict(sd, report)

    os.makedirs(out_dir, exist_ok=True)
    np.savez(os.path.join(out_dir, "weights.npz"), **weights)
    meta = {
        "schema_version": 1,
        "model": hp.get("model", "ssla_s_yolox_det"),
        "method": "ssla",
        "height": int(h),
        "width": int(w),
        "num_classes": report.num_classes,
        "num_anchors": 1,
        "ssla_tdrop_window": report.tdrop_window,
        "dtype": "float32",
        "layout": "C_order_row_major",
        "key_separator": "/",
        "checkpoint": os.path.abspath(ckpt_path) if ckpt_path else "",
        "ckpt_epoch": int(ck.get("epoch", -1)),
        "ckpt_global_step": int(ck.get("global_step", -1)),
        "source_state_dict": src,
        "ckpt_native_h": int(hp.get("height", 0)),
        "ckpt_native_w": int(hp.get("width", 0)),
        "total_params": int(sum(int(np.prod(a.shape)) for a in weights.values())),
    }
    with open(os.path.join(out_dir, "meta.json"), "w") as f:
        json.dump(meta, f, indent=2)
    return report, meta


def main(argv: Optional[List[str]] = None) -> int:
    ap = argparse.ArgumentParser(description=__doc__.splitlines()[0])
    ap.add_argument("ckpt", help="Lightning .ckpt file")
    ap.add_argument("out_dir")
    ap.add_argument("--h", type=int, default=120, help="runtime input height")
    ap.add_argument("--w", type=int, default=160, help="runtime input width")
    ap.add_argument("--use-ema", dest="use_ema", action="store_true", default=True)
    ap.add_argument("--no-ema", dest="use_ema", action="store_false")
    a = ap.parse_args(argv)
    report, meta = convert(a.ckpt, a.out_dir, a.h, a.w, a.use_ema)
    for wmsg in report.warnings:
        print(f"[convert] WARN: {wmsg}", file=sys.stderr)
    print(f"[convert] {report.source}: kept {report.n_layer} layer + {report.n_head} head "
          f"tensors, skipped {report.n_skipped}; num_classes={report.num_classes} "
          f"tdrop={report.tdrop_window} total_params={meta['total_params']}")
    return 0


if __name__ == "__main__":
    sys.exit(main())
