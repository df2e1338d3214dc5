/*
 * ssla_oracle.h -- CPU restatement of the SSLA-S s2+s3+head drain path.
 *
 * TEST INFRASTRUCTURE ONLY.  Only tests/, __graft_entry__.smoke() and the
 * cpu_baseline leg of bench.py may load this library, and only as the
 * checker (or, for cpu_baseline, as the timed CPU comparison).  The product
 * path (libssla_hip.so) never links or calls it.
 *
 * What it restates (reference file:line):
 *   - oracle_reshape_layer     orin/orin/weights_ssla.py:24-88 and
 *                              src/ssla_kernels.cpp:73-153 (load_layer)
 *   - oracle_layer_step_f64    orin/orin/ssla_ref.py:17-93 (layer_step)
 *   - oracle_layer_step_f32    src/ssla_kernels.cpp:315-385 (layer_forward_ct,
 *                              generic fp32 path) with vendor/openeva/prim/
 *                              linear.h:80-101, rnn.h:79-90, layernorm.h:40-60,
 *                              activation.h:16-20
 *   - oracle_tdrop             orin/orin/ssla_ref.py:190-195
 *   - oracle_s2s3_run          orin/bench_s2_s3_head_celled.py:53-86 (cpu_oracle
 *                              schedule: L4, L5, tdrop_s2, L6, L7, tdrop_s3)
 *   - oracle_head_raw          orin/kernels/ssla_s2_s3_head_celled.cuh:841-902
 *                              (raw [reg4, obj, cls2] of the 2-branch head)
 *                              and :1462-1500, 1715-1751 (single-linear head:
 *                              matvec_w<C3, 7> of orin/kernels/
 *                              proto_layer_pair.cuh:39-58 plus head_b)
 *   - oracle_fuse_conv_bn      orin/orin/hybrid_common.py:327-349
 *   - oracle_s01_run           one producer shard: preprocess
 *                              (src/ssla_kernels.cpp:288-309), stages 0 and 1
 *                              of step_ref (orin/orin/ssla_ref.py:119-170),
 *                              halo events stage 0 only
 *                              (src/lib_stage01_to_gpu.cpp:210-330)
 *
 * Pinning (see tests/): tdrop + schedule by the published P1 pass counts;
 * reshape by the per-position module forward identity; layer_step by the
 * module forward + LayerNorm closed forms; head by the reference's own
 * YOLOX decode compiled into oracle/_ref; the single-linear head by one-hot
 * and zero-feature closed forms (row i of lin_W plus lin_b, lin_b) and the
 * reference's prim::matvec_ct compiled into oracle/_ref.
 */
#ifndef SSLA_ORACLE_H
#define SSLA_ORACLE_H

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* One SSLA layer in the oracle (reference) layout.
 *   qvgIn      (A, 3*OUT, IN) row-major, rows split [q | v | g]
 *   goW        (A, OUT, OUT)  row-major, contrib = goW[p] @ qh
 *   input_proj (OUT, IN) or NULL (then IN == OUT, identity residual)
 *   A = K*K (1 or 9)                                                      */
typedef struct {
    const float* qvgIn;
    const float* goW;
    const float* input_proj;
    const float* ln_gamma;
    const float* ln_beta;
    int in_dim;
    int out_dim;
    int K;
    /* Optional copies of qvgIn and goW with the last two axes swapped
     * ((A, in, 3D) and (A, D, D) input-major), or NULL.  The fp64 step then
     * runs its dot products over these; every sum keeps the same terms in
     * the same order, so the results are identical either way. */
    const float* qvgInT;
    const float* goWT;
} OracleLayer;

/* Head of the drain.  Two-branch YOLOX head (BN already folded, PyTorch
 * (out, in) layouts) when cls_conv_W is set; otherwise the single-linear
 * head of the reference's persistent kernels (lin_W in the device's
 * (IN, OUT) = (C, 7) layout):  raw7[o] = lin_b[o] + sum_i lin_W[i*7+o] x[i]. */
typedef struct {
    const float* cls_conv_W;   /* (C, C)  */
    const float* cls_conv_b;   /* (C,)    */
    const float* cls_pred_W;   /* (2, C)  */
    const float* cls_pred_b;   /* (2,)    */
    const float* reg_conv_W;   /* (C, C)  */
    const float* reg_conv_b;   /* (C,)    */
    const float* reg_pred_W;   /* (4, C)  */
    const float* reg_pred_b;   /* (4,)    */
    const float* obj_pred_W;   /* (1, C)  */
    const float* obj_pred_b;   /* (1,)    */
    int C;                     /* 96 */
    const float* lin_W;        /* (C, 7)  single-linear head, or NULL */
    const float* lin_b;        /* (7,)    */
} OracleHead;

/* State of one s2+s3 instance.  H[li] is (Hl*Wl, OUT) fp32, read and
 * written; td2 (H2*W2) and td3 (H3*W3) are the uint8 tdrop counters.     */
typedef struct {
    OracleLayer L[4];          /* L4, L5, L6, L7 */
    float*   H[4];
    uint8_t* td2;
    uint8_t* td3;
    int H2, W2, H3, W3;
    int window;
    const OracleHead* head;    /* NULL: no head outputs */
} OracleS2S3;

/* fp32 reshape following load_layer's loop structure.  W_in_cat is
 * (in_dim, win_cols), W_out_cat is (wout_rows, D); q/v/g/oW are (D, D).
 * Writes qvgIn (A, 3D, in_dim) and goW (A, D, D); returns A or -1.        */
int oracle_reshape_layer(const float* W_in_cat, int win_cols,
                         const float* W_out_cat, int wout_rows,
                         const float* qW, const float* vW,
                         const float* gW, const float* oW,
                         int in_dim, int D,
                         float* qvgIn, float* goW);

/* One layer forward for one event at (ev_x, ev_y) on an (Hl, Wl) grid.
 * Mutates H_all at the patch cells; writes out (OUT,).                   */
void oracle_layer_step_f64(const OracleLayer* L, const float* in,
                           float* H_all, int ev_x, int ev_y,
                           int Hl, int Wl, float* out);
void oracle_layer_step_f32(const OracleLayer* L, const float* in,
                           float* H_all, int ev_x, int ev_y,
                           int Hl, int Wl, float* out);

/* pre = c[idx]; c[idx] = pre+1 (mod 256); pass = window<=1 || pre%window==0 */
int oracle_tdrop(uint8_t* counter, int window, int idx);

/* The drain schedule over n ring records (s2 coordinates).
 *   precision: 64 (golden, layer_step semantics) or 32 (generic C++ path)
 *   owner:     per-record ownership flag or NULL (all owned)
 * Outputs (any may be NULL):
 *   pass2[i], pass3[i]  1/0 (pass3 = 0 when pass2 = 0); -2 for records
 *                       outside the s2 grid
 *   s3_feat[i*96..]     L7 output for pass3 records, zeros otherwise
 *   head7[i*7..]        raw head output for owner & pass3 records, zeros
 *                       otherwise (needs st->head)
 * Records with x >= W2 or y >= H2 are skipped (no state change).
 * Returns the number of pass3 records, or -1 on bad arguments.           */
int oracle_s2s3_run(OracleS2S3* st, const uint16_t* xs, const uint16_t* ys,
                    const float* feat1, const uint8_t* owner, int n,
                    int precision, int8_t* pass2, int8_t* pass3,
                    float* s3_feat, float* head7);

/* Decisions only (no features): the same tdrop schedule as
 * oracle_s2s3_run, for full-size checks.  Returns pass3 count.           */
int oracle_s2s3_decisions(uint8_t* td2, uint8_t* td3, int H2, int W2,
                          int window, const uint16_t* xs, const uint16_t* ys,
                          int n, int8_t* pass2, int8_t* pass3);

/* One producer shard over stages 0 + 1: layers L0..L3 (L0 with K = 1),
 * hidden state H[li] (cells x OUT on the full or half grid), tdrop counters td0
 * (height/2 * width/2) and td1 (height/4 * width/4), per-pixel last event time last_t (height * width,
 * initialised to -1).                                                     */
typedef struct {
    OracleLayer L[4];
    float*   H[4];
    uint8_t* td0;
    uint8_t* td1;
    double*  last_t;
    int height, width;
    int window;
} OracleS01;

/* feat = [dt_norm, p] with dt_norm = clamp((t - last_t[pixel]) / 1e5, 0, 1)
 * (1 for a pixel's first event); updates last_t; zeros outside the sensor. */
void oracle_preprocess(double* last_t, int height, int width, float t_us,
                       int x, int y, float p, float feat[2]);

/* Events ev[i] = (t_us, x, y, p).  owner[i] = 0 marks a halo event (stage
 * 0 for its state only, no tdrop); NULL = all owned.  Outputs (any NULL):
 *   pass0[i], pass1[i]  1/0 (pass1 = 0 when pass0 = 0), -1 for halo
 *                       events, -2 for events outside the sensor
 *   feat1[i*24..]       L3 output when pass1, zeros otherwise
 *   x2[i], y2[i]        s2 coordinates (x >> 2, y >> 2) when pass1
 * Returns the number of pass1 events, or -1 on bad arguments.            */
int oracle_s01_run(OracleS01* st, const float* ev, const uint8_t* owner, int n,
                   int precision, int8_t* pass0, int8_t* pass1, float* feat1,
                   uint16_t* x2, uint16_t* y2);

/* Raw head output [reg0..3, obj, cls0, cls1] for one 96-float feature
 * (either head kind of OracleHead).                                       */
void oracle_head_raw_f64(const OracleHead* h, const float* x, float out7[7]);
void oracle_head_raw_f32(const OracleHead* h, const float* x, float out7[7]);

/* Fold eval-mode BatchNorm into a 1x1 conv (out, in):
 *   scale = g / sqrt(var + eps); shift = b - scale*mu
 *   W' = W * scale[:, None];     b' = b_conv*scale + shift              */
void oracle_fuse_conv_bn(const float* W, const float* b_conv_or_null,
                         const float* bn_w, const float* bn_b,
                         const float* bn_mu, const float* bn_var,
                         int c_out, int c_in, float eps,
                         float* W_out, float* b_out);

#ifdef __cplusplus
}
#endif

#endif /* SSLA_ORACLE_H */
