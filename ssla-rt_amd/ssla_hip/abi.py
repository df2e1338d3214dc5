"""numpy / ctypes mirrors of include/ssla_abi.h.

The record, output-slot and timing layouts are the ones existing producers
and harnesses use (orin/orin/hybrid_common.py:30-123); the config struct is
the ctypes form of HybridS2S3Config (orin/kernels/ssla_s2_s3_head_celled.cuh
:84-127).  lib.check_layout() compares these sizes with the compiled library.
"""
from __future__ import annotations

import ctypes

import numpy as np

C1, C2, C3 = 24, 48, 96
HEAD_OUT = 7
MAX_BLOCKS = 16

INPUT_DTYPE = np.dtype([
    ("seq_done", "<u8"),
    ("t", "<f4"),
    ("x", "<u2"),
    ("y", "<u2"),
    ("feat1", "<f4", (C1,)),
    ("t_push_ns", "<u8"),
    ("t_emit_ns", "<u8"),
])

OUTPUT_DTYPE = np.dtype([
    ("pass2", "<i4"),
    ("pass3", "<i4"),
    ("s3_feat", "<f4", (C3,)),
])

TIMING_DTYPE = np.dtype([
    ("t_pop_clk", "<u8"),
    ("t_done_clk", "<u8"),
    ("seq", "<u4"),
    ("owner", "<u4"),
    ("t_push_ns", "<u8"),
    ("t_emit_ns", "<u8"),
])

assert INPUT_DTYPE.itemsize == 128
assert OUTPUT_DTYPE.itemsize == 392
assert TIMING_DTYPE.itemsize == 40


class HybridStrip(ctypes.Structure):
    _fields_ = [
        ("owned_lo", ctypes.c_int32), ("owned_hi", ctypes.c_int32),
        ("s3_owned_lo", ctypes.c_int32), ("s3_owned_hi", ctypes.c_int32),
        ("owned_y_lo", ctypes.c_int32), ("owned_y_hi", ctypes.c_int32),
        ("s3_owned_y_lo", ctypes.c_int32), ("s3_owned_y_hi", ctypes.c_int32),
    ]


class LayerWeightsS2S3(ctypes.Structure):
    _fields_ = [(n, ctypes.c_void_p) for n in
                ("qvgIn", "goW", "input_proj", "ln_gamma", "ln_beta")]


# pointers of the two-branch YOLOX head in HybridS2S3Config
HEAD_FIELDS = ("head_cls_conv_W", "head_cls_conv_b", "head_cls_pred_W",
               "head_cls_pred_b", "head_reg_conv_W", "head_reg_conv_b",
               "head_reg_pred_W", "head_reg_pred_b", "head_obj_pred_W",
               "head_obj_pred_b")


class HybridS2S3Config(ctypes.Structure):
    _fields_ = [
        ("H2", ctypes.c_int32), ("W2", ctypes.c_int32),
        ("H3", ctypes.c_int32), ("W3", ctypes.c_int32),
        ("tdrop_window", ctypes.c_int32),
        ("head_out_dim", ctypes.c_int32),
        ("n_blocks", ctypes.c_int32),
        ("_pad_nblocks", ctypes.c_int32),
        ("strip", HybridStrip * MAX_BLOCKS),
        ("layers", (LayerWeightsS2S3 * 4) * MAX_BLOCKS),
        ("hidden", (ctypes.c_void_p * 4) * MAX_BLOCKS),
        ("tdrop_s2", ctypes.c_void_p * MAX_BLOCKS),
        ("tdrop_s3", ctypes.c_void_p * MAX_BLOCKS),
        ("head_W", ctypes.c_void_p),
        ("head_b", ctypes.c_void_p),
    ] + [(n, ctypes.c_void_p) for n in HEAD_FIELDS] + [
        ("preds", ctypes.c_void_p * MAX_BLOCKS),
        ("version", ctypes.c_void_p * MAX_BLOCKS),
        ("timing", ctypes.c_void_p * MAX_BLOCKS),
        ("timing_mask", ctypes.c_uint32),
        ("_pad_timing", ctypes.c_uint32),
        ("kernel_start_clk", ctypes.c_void_p * MAX_BLOCKS),
        ("kernel_end_clk", ctypes.c_void_p * MAX_BLOCKS),
    ]


class SslaHipModelInfo(ctypes.Structure):
    _fields_ = [(n, ctypes.c_int) for n in
                ("height", "width", "num_classes", "tdrop_window",
                 "H2", "W2", "H3", "W3", "has_head")]


class SslaHipDrainOpts(ctypes.Structure):
    _fields_ = [
        ("stream", ctypes.c_void_p),
        ("sync", ctypes.c_int),
        ("batch", ctypes.c_int),
        ("head_outs", ctypes.POINTER(ctypes.c_void_p)),
        ("phase_ms", ctypes.POINTER(ctypes.c_float)),
        ("batch_phase_us", ctypes.POINTER(ctypes.c_double)),
        ("group", ctypes.c_int),
        ("phase_mask", ctypes.c_ulonglong),
    ]


class SslaHipLiveOpts(ctypes.Structure):
    _fields_ = [("max_batch", ctypes.c_int), ("idle_timeout_ms", ctypes.c_uint),
                ("phase_us", ctypes.POINTER(ctypes.c_double)), ("group", ctypes.c_int),
                ("stages", ctypes.c_int)]


class SslaHipOevaDiff(ctypes.Structure):
    _fields_ = [("ok", ctypes.c_int), ("n_cp", ctypes.c_size_t),
                ("max_abs_delta", ctypes.c_double), ("n_mismatched_cp", ctypes.c_size_t)]


# return codes of the C ABI (include/ssla_hip.h)
SSLA_OK, SSLA_ERR_ARG, SSLA_ERR_HIP, SSLA_ERR_IO, SSLA_ERR_FORMAT, SSLA_ERR_STATE = 0, -1, -2, -3, -4, -5

PRED_BUSY = 0x80000000
OEVA_MAGIC = 0x4F455641
OEVA_VERSION = 1


DRAIN_PHASES = ("order",
                "L4.proj", "L4.sum", "L4.carry", "L4.apply", "L4.out",
                "L5.proj", "L5.sum", "L5.carry", "L5.apply", "L5.out",
                "L6.proj", "L6.sum", "L6.carry", "L6.apply", "L6.out",
                "L7.proj", "L7.sum", "L7.carry", "L7.apply", "L7.out",
                "head", "emit")

# in-kernel profile of the batch-mode and live drains (SSLA_BATCH_PHASES);
# times in microseconds except the two trailing counts
BATCH_PHASES = ("load", "tdrop2", "pairs2",
                "L4.proj", "L4.scan", "L4.out", "L4.ln", "L5.proj", "L5.scan", "L5.out", "L5.ln",
                "tdrop3", "pairs3",
                "L6.proj", "L6.scan", "L6.out", "L6.ln", "L7.proj", "L7.scan", "L7.out", "L7.ln",
                "head.hidden", "head.out", "preds", "publish", "batches", "records",
                "L4.xwait", "L5.xwait", "L6.xwait", "L7.xwait")
N_BATCH_PHASES = 32


assert ctypes.sizeof(HybridS2S3Config) == 4616
assert HybridS2S3Config.preds.offset == 3968
