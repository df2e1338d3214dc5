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

// Bit 31 of a prediction cell's version marks a write in progress.
constexpr unsigned kPredBusy = 0x80000000u;

// Publishes one prediction-grid cell (fine-grained host memory) for
// concurrent host readers: the version's busy bit is set, the seven values
// are stored between two system-scope fences, and the version ends at
// old + count with the bit clear -- so a reader that sees the same version
// before and after copying a cell, without the bit, has a whole cell.
__device__ __forceinline__ void publish_pred(float* preds7, unsigned* version, const float* v7,
                                             unsigned count) {
    unsigned old = 0;
    if (version) {
        old = __hip_atomic_load(version, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_SYSTEM) & ~kPredBusy;
        __hip_atomic_store(version, old | kPredBusy, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_SYSTEM);
        __threadfence_system();
    }
    if (preds7) {
        #pragma unroll
        for (int q = 0; q < 7; ++q) preds7[q] = v7[q];
    }
    if (version) {
        __threadfence_system();
        __hip_atomic_store(version, (old + count) & ~kPredBusy, __ATOMIC_RELAXED,
                           __HIP_MEMORY_SCOPE_SYSTEM);
    }
}

}  // namespace ssla
