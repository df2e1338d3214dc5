// drain_common.h -- device-side definitions shared by the whole-ring drain
// (drain_scan.hip) and the batch / live drain (drain_live.hip).
#pragma once

#include <hip/hip_runtime.h>

#include <cstdint>

#include "ssla_abi.h"

namespace ssla {

// Global-memory accesses through address-space-1 pointers: pointers that
// reach device code as generic values (loaded from descriptor tables) would
// otherwise compile to flat instructions, which also count against the LDS
// counter, so every later LDS wait would wait for them as well (a host-ring
// read or a counter store for a PCIe or L2 round trip).
#define SSLA_GLOBAL __attribute__((address_space(1)))

template <class T>
__device__ __forceinline__ SSLA_GLOBAL T* gmem(T* p) {
    return (SSLA_GLOBAL T*)p;
}

constexpr int kPatch = 9;   // 3x3 patch positions, delta = (1-dy)*3 + (1-dx)

struct Geometry {
    int H2, W2, H3, W3;
    int C2, C3;          // cells per block at s2 / s3
    int nb;              // blocks
    int window;
};

// Head of a configuration (orin/kernels/ssla_s2_s3_head_celled.cuh:1462-1500,
// 1715-1751): the two-branch YOLOX head when head_cls_conv_W is set, else
// the single-linear head raw7 = head_W^T x + head_b when head_W is set,
// else none.
enum HeadKind : int { kHeadNone = 0, kHeadYolox = 1, kHeadLinear = 2 };

// Head weights, (IN, OUT) layouts (ssla_abi.h): the two-branch YOLOX head
// with BN folded, and the single-linear head (lin_W (C3, 7), lin_b (7)).
struct HeadPtrs {
    const float *cls_conv_W, *cls_conv_b, *cls_pred_W, *cls_pred_b;
    const float *reg_conv_W, *reg_conv_b, *reg_pred_W, *reg_pred_b;
    const float *obj_pred_W, *obj_pred_b;
    const float *lin_W, *lin_b;
};

inline int head_kind(const HybridS2S3Config* cfg) {
    if (cfg->head_cls_conv_W) return kHeadYolox;
    return cfg->head_W ? kHeadLinear : kHeadNone;
}

inline HeadPtrs head_ptrs(const HybridS2S3Config* cfg) {
    return HeadPtrs{cfg->head_cls_conv_W, cfg->head_cls_conv_b, cfg->head_cls_pred_W,
                    cfg->head_cls_pred_b, cfg->head_reg_conv_W, cfg->head_reg_conv_b,
                    cfg->head_reg_pred_W, cfg->head_reg_pred_b, cfg->head_obj_pred_W,
                    cfg->head_obj_pred_b, cfg->head_W, cfg->head_b};
}

// Which head weights a configuration must have bound for its kind; the
// message names the first one missing, or is null.
inline const char* head_missing(const HybridS2S3Config* cfg) {
    const int k = head_kind(cfg);
    if (k == kHeadLinear && !cfg->head_b) return "head_W is set but head_b is not";
    if (k == kHeadYolox) {
        const float* const need[9] = {cfg->head_cls_conv_b, cfg->head_cls_pred_W, cfg->head_cls_pred_b,
                                      cfg->head_reg_conv_W, cfg->head_reg_conv_b, cfg->head_reg_pred_W,
                                      cfg->head_reg_pred_b, cfg->head_obj_pred_W, cfg->head_obj_pred_b};
        for (const float* p : need)
            if (!p) return "head_cls_conv_W is set but another two-branch head weight is not";
    }
    return nullptr;
}

__device__ __forceinline__ float sigmoid_fast(float x) {
    return __fdividef(1.0f, 1.0f + __expf(-x));
}

// Bit 31 of a prediction cell's version marks a write in progress.
constexpr unsigned kPredBusy = 0x80000000u;

// A prediction cell's version word (fine-grained host memory) without the
// busy bit, or 0 for none.
__device__ __forceinline__ unsigned pred_version(const unsigned* version) {
    return version ? __hip_atomic_load(gmem(const_cast<unsigned*>(version)), __ATOMIC_RELAXED,
                                       __HIP_MEMORY_SCOPE_SYSTEM) & ~kPredBusy
                   : 0u;
}

// Publishes one prediction-grid cell (fine-grained host memory) for
// concurrent host readers: the version's busy bit is set, the seven values
// are stored between two system-scope fences, and the version ends at
// old + count with the bit clear -- so a reader that sees the same version
// before and after copying a cell, without the bit, has a whole cell.
// `old` is the cell's version read beforehand (pred_version): the device is
// the cell's only writer, so the word cannot change in between.
__device__ __forceinline__ void publish_pred_at(float* preds7, unsigned* version, const float* v7,
                                                unsigned count, unsigned old) {
    if (version) {
        __hip_atomic_store(gmem(version), old | kPredBusy, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_SYSTEM);
        __threadfence_system();
    }
    if (preds7) {
        #pragma unroll
        for (int q = 0; q < 7; ++q) gmem(preds7)[q] = v7[q];
    }
    if (version) {
        __threadfence_system();
        __hip_atomic_store(gmem(version), (old + count) & ~kPredBusy, __ATOMIC_RELAXED,
                           __HIP_MEMORY_SCOPE_SYSTEM);
    }
}

__device__ __forceinline__ void publish_pred(float* preds7, unsigned* version, const float* v7,
                                             unsigned count) {
    publish_pred_at(preds7, version, v7, count, pred_version(version));
}

}  // namespace ssla
