/*
 * ssla_abi.h -- binary contracts of the SSLA-S s2+s3+head drain path.
 *
 * These layouts are shared with existing producers and harnesses, so they
 * are kept byte-identical to the reference:
 *   HybridInputRec        orin/kernels/ssla_s2_s3_head_celled.cuh:129-137,
 *                         src/lib_stage01_to_gpu.cpp:51-60 (128 B)
 *   HybridStrip           ...celled.cuh:53-64 (32 B)
 *   LayerWeightsS2S3      ...celled.cuh:45-51 (40 B)
 *   HybridS2S3Config      ...celled.cuh:84-127, ctypes mirror
 *                         orin/orin/hybrid_common.py:76-111 (4616 B,
 *                         preds at offset 3968)
 *   HybridS2S3OutputSlot  ...celled.cuh:139-143 (392 B)
 *   GpuTimingSlot         ...celled.cuh:66-76 (40 B)
 *
 * Device weight layouts referenced by LayerWeightsS2S3 (per layer, A = 9
 * patch positions "delta", delta = (1-dy)*3 + (1-dx)):
 *   qvgIn      (9, IN, 3*OUT) row-major; each row is [q | v | g]
 *   goW        (9, OUT_in, OUT_out) row-major; contrib[o] = sum_i goW[i][o]*qh[i]
 *   input_proj (IN, OUT) row-major, or NULL when IN == OUT
 *   ln_gamma, ln_beta (OUT)
 * Head weights are stored (IN, OUT) row-major with BatchNorm folded in.
 * Hidden state hidden[b][li] is (Hl*Wl, OUT) fp32, cell-major.
 * tdrop_s2[b] / tdrop_s3[b] are uint8 counters of H2*W2 / H3*W3 cells.
 */
#ifndef SSLA_ABI_H
#define SSLA_ABI_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define SSLA_C1 24
#define SSLA_C2 48
#define SSLA_C3 96
#define SSLA_HEAD_OUT 7
#define SSLA_MAX_BLOCKS 16

typedef struct LayerWeightsS2S3 {
    const float* qvgIn;
    const float* goW;
    const float* input_proj;
    const float* ln_gamma;
    const float* ln_beta;
} LayerWeightsS2S3;

typedef struct HybridStrip {
    int owned_lo;          /* s2-x owned range [lo, hi) */
    int owned_hi;
    int s3_owned_lo;       /* s3-x owned range */
    int s3_owned_hi;
    int owned_y_lo;        /* s2-y owned range */
    int owned_y_hi;
    int s3_owned_y_lo;     /* s3-y owned range */
    int s3_owned_y_hi;
} HybridStrip;

typedef struct GpuTimingSlot {
    unsigned long long t_pop_clk;
    unsigned long long t_done_clk;
    unsigned int       seq;
    unsigned int       owner;      /* 1 iff owner && pass2 && pass3 */
    unsigned long long t_push_ns;
    unsigned long long t_emit_ns;
} GpuTimingSlot;

typedef struct HybridS2S3Config {
    int H2, W2;
    int H3, W3;
    int tdrop_window;
    int head_out_dim;
    int n_blocks;
    int _pad_nblocks;
    HybridStrip      strip[SSLA_MAX_BLOCKS];
    LayerWeightsS2S3 layers[SSLA_MAX_BLOCKS][4];
    float*           hidden[SSLA_MAX_BLOCKS][4];
    unsigned char*   tdrop_s2[SSLA_MAX_BLOCKS];
    unsigned char*   tdrop_s3[SSLA_MAX_BLOCKS];
    const float*     head_W;            /* single-linear head (C3, 7) */
    const float*     head_b;
    const float*     head_cls_conv_W;   /* (C3, C3) */
    const float*     head_cls_conv_b;
    const float*     head_cls_pred_W;   /* (C3, 2)  */
    const float*     head_cls_pred_b;
    const float*     head_reg_conv_W;   /* (C3, C3) */
    const float*     head_reg_conv_b;
    const float*     head_reg_pred_W;   /* (C3, 4)  */
    const float*     head_reg_pred_b;
    const float*     head_obj_pred_W;   /* (C3, 1)  */
    const float*     head_obj_pred_b;
    float*           preds[SSLA_MAX_BLOCKS];     /* (s3 owned cells, 7) */
    unsigned int*    version[SSLA_MAX_BLOCKS];   /* (s3 owned cells,)   */
    GpuTimingSlot*   timing[SSLA_MAX_BLOCKS];
    unsigned int     timing_mask;
    unsigned int     _pad_timing;
    unsigned long long* kernel_start_clk[SSLA_MAX_BLOCKS];
    unsigned long long* kernel_end_clk[SSLA_MAX_BLOCKS];
} HybridS2S3Config;

typedef struct HybridInputRec {
    unsigned long long seq_done;   /* publish tag: slot + 1 */
    float              t;
    unsigned short     x;          /* s2 coordinates */
    unsigned short     y;
    float              feat1[SSLA_C1];
    unsigned long long t_push_ns;
    unsigned long long t_emit_ns;
} HybridInputRec;

typedef struct HybridS2S3OutputSlot {
    int   pass2;                   /* 1 / 0 owner decision, -1 halo record */
    int   pass3;
    float s3_feat[SSLA_C3];
} HybridS2S3OutputSlot;

#ifdef __cplusplus
}  /* extern "C" */
static_assert(sizeof(HybridInputRec) == 128, "HybridInputRec must be 128 B");
static_assert(offsetof(HybridInputRec, feat1) == 16, "feat1 offset");
static_assert(offsetof(HybridInputRec, t_push_ns) == 112, "t_push_ns offset");
static_assert(sizeof(HybridStrip) == 32, "HybridStrip size");
static_assert(sizeof(LayerWeightsS2S3) == 40, "LayerWeightsS2S3 size");
static_assert(sizeof(GpuTimingSlot) == 40, "GpuTimingSlot size");
static_assert(sizeof(HybridS2S3OutputSlot) == 392, "HybridS2S3OutputSlot size");
static_assert(sizeof(HybridS2S3Config) == 4616, "HybridS2S3Config size");
static_assert(offsetof(HybridS2S3Config, preds) == 3968, "preds offset");
#endif

#endif /* SSLA_ABI_H */
