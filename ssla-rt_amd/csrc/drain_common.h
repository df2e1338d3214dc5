// drain_common.h -- device-side definitions shared by the whole-ring drain
// (drain_scan.hip) and the batch / live drain (drain_live.hip).
#pragma once

#include <hip/hip_runtime.h>

#include <cstdint>

#include "ssla_abi.h"

namespace ssla {

constexpr int kPatch = 9;   // 3x3 patch positions, delta = (1-dy)*3 + (1-dx)

struct Geometry {
    int H2, W2, H3, W3;
    int C2, C3;          // cells per block at s2 / s3
    int nb;              // blocks
    int window;
};

// Two-branch YOLOX head, BN folded, (IN, OUT) layouts (ssla_abi.h).
struct HeadPtrs {
    const float *cls_conv_W, *cls_conv_b, *cls_pred_W, *cls_pred_b;
    const float *reg_conv_W, *reg_conv_b, *reg_pred_W, *reg_pred_b;
    const float *obj_pred_W, *obj_pred_b;
};

__device__ __forceinline__ float sigmoid_fast(float x) {
    return __fdividef(1.0f, 1.0f + __expf(-x));
}

}  // namespace ssla
