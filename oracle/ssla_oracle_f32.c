/*
 * ssla_oracle_f32.c -- the fp32 "reference CPU path" of the oracle.
 *
 * TEST INFRASTRUCTURE ONLY.  Restates the generic fp32 layer of
 * src/ssla_kernels.cpp:315-385 (layer_forward_ct) built from the scalar
 * primitives vendor/openeva/prim/linear.h:80-101 (matvec_ct,
 * matvec_accum_ct), rnn.h:79-90 (lru_step), activation.h:16-20
 * (sigmoid = 1/(1+exp(-x))), elementwise.h:11-14 (add_inplace) and
 * layernorm.h:40-60 (fp64 LayerNorm).  Compiled with -ffast-math like the
 * reference CPU build (CMakeLists.txt:18-25); this is the timed CPU baseline.
 */
#include "ssla_oracle.h"

#include <math.h>
#include <string.h>

#define MAXD 96

static inline float sigmoid_f(float x) { return 1.0f / (1.0f + expf(-x)); }

/* y[o] = sum_i W[o*IN + i] * x[i] (acc from 0, i ascending) */
static inline void matvec_f32(const float* x, const float* W, int IN, int OUT,
                              float* y) {
    for (int o = 0; o < OUT; ++o) {
        const float* w = W + (size_t)o * IN;
        float acc = 0.0f;
        for (int i = 0; i < IN; ++i) acc += w[i] * x[i];
        y[o] = acc;
    }
}

static inline void matvec_accum_f32(const float* x, const float* W, int IN,
                                    int OUT, float* y) {
    for (int o = 0; o < OUT; ++o) {
        const float* w = W + (size_t)o * IN;
        float acc = 0.0f;
        for (int i = 0; i < IN; ++i) acc += w[i] * x[i];
        y[o] += acc;
    }
}

static void layernorm_ct(float* x, int D, const float* gamma, const float* beta) {
    double sum = 0.0;
    for (int i = 0; i < D; ++i) sum += (double)x[i];
    const double mean = sum / (double)D;
    double var = 0.0;
    for (int i = 0; i < D; ++i) {
        const double d = (double)x[i] - mean;
        var += d * d;
    }
    var /= (double)D;
    const double inv = 1.0 / sqrt(var + (double)1e-5f);
    for (int i = 0; i < D; ++i) {
        const double v = ((double)x[i] - mean) * inv;
        x[i] = (float)(v * (double)gamma[i] + (double)beta[i]);
    }
}

static void process_patch(const OracleLayer* L, const float* in, float* h,
                          int pos, float* out) {
    const int IN = L->in_dim, D = L->out_dim;
    float qvg[3 * MAXD], qh[MAXD];
    matvec_f32(in, L->qvgIn + (size_t)pos * 3 * D * IN, IN, 3 * D, qvg);
    const float* q = qvg;
    const float* v = qvg + D;
    const float* g = qvg + 2 * D;
    for (int c = 0; c < D; ++c) {
        const float gc = sigmoid_f(g[c]);
        const float hc = gc * h[c] + v[c];
        h[c] = hc;
        qh[c] = q[c] * hc;
    }
    matvec_accum_f32(qh, L->goW + (size_t)pos * D * D, D, D, out);
}

void oracle_layer_step_f32(const OracleLayer* L, const float* in,
                           float* H_all, int ev_x, int ev_y, int Hl, int Wl,
                           float* out) {
    const int IN = L->in_dim, D = L->out_dim;
    float residual[MAXD];
    if (L->input_proj) matvec_f32(in, L->input_proj, IN, D, residual);
    else memcpy(residual, in, sizeof(float) * D);
    memset(out, 0, sizeof(float) * D);

    const int base = ev_y * Wl + ev_x;
    if (L->K == 1) {
        process_patch(L, in, H_all + (size_t)base * D, 0, out);
    } else if (ev_x > 0 && ev_x + 1 < Wl && ev_y > 0 && ev_y + 1 < Hl) {
        /* interior order of ssla_kernels.cpp:349-358 */
        process_patch(L, in, H_all + (size_t)(base - Wl - 1) * D, 8, out);
        process_patch(L, in, H_all + (size_t)(base - Wl) * D, 7, out);
        process_patch(L, in, H_all + (size_t)(base - Wl + 1) * D, 6, out);
        process_patch(L, in, H_all + (size_t)(base - 1) * D, 5, out);
        process_patch(L, in, H_all + (size_t)(base) * D, 4, out);
        process_patch(L, in, H_all + (size_t)(base + 1) * D, 3, out);
        process_patch(L, in, H_all + (size_t)(base + Wl - 1) * D, 2, out);
        process_patch(L, in, H_all + (size_t)(base + Wl) * D, 1, out);
        process_patch(L, in, H_all + (size_t)(base + Wl + 1) * D, 0, out);
    } else {
        for (int dy = -1; dy <= 1; ++dy) {
            const int py = ev_y + dy;
            if (py < 0 || py >= Hl) continue;
            for (int dx = -1; dx <= 1; ++dx) {
                const int px = ev_x + dx;
                if (px < 0 || px >= Wl) continue;
                process_patch(L, in, H_all + (size_t)(py * Wl + px) * D,
                              (1 - dy) * 3 + (1 - dx), out);
            }
        }
    }
    for (int o = 0; o < D; ++o) out[o] += residual[o];
    layernorm_ct(out, D, L->ln_gamma, L->ln_beta);
}

/* fp32 head: matvec with bias, SiLU = x * sigmoid(x) (activation.h:19);
 * the single-linear head accumulates in channel order as matvec_w does
 * (proto_layer_pair.cuh:39-58), then adds head_b (…celled.cuh:1481). */
void oracle_head_raw_f32(const OracleHead* h, const float* x, float out7[7]) {
    const int C = h->C;
    if (!h->cls_conv_W) {
        for (int o = 0; o < 7; ++o) {
            float s = 0.0f;
            for (int i = 0; i < C; ++i) s += h->lin_W[(size_t)i * 7 + o] * x[i];
            out7[o] = s + h->lin_b[o];
        }
        return;
    }
    float yc[MAXD], yr[MAXD];
    for (int o = 0; o < C; ++o) {
        float a = h->cls_conv_b[o], b = h->reg_conv_b[o];
        const float* wc = h->cls_conv_W + (size_t)o * C;
        const float* wr = h->reg_conv_W + (size_t)o * C;
        for (int i = 0; i < C; ++i) {
            a += wc[i] * x[i];
            b += wr[i] * x[i];
        }
        yc[o] = a * sigmoid_f(a);
        yr[o] = b * sigmoid_f(b);
    }
    for (int k = 0; k < 4; ++k) {
        float s = h->reg_pred_b[k];
        for (int i = 0; i < C; ++i) s += h->reg_pred_W[(size_t)k * C + i] * yr[i];
        out7[k] = s;
    }
    {
        float s = h->obj_pred_b[0];
        for (int i = 0; i < C; ++i) s += h->obj_pred_W[i] * yr[i];
        out7[4] = s;
    }
    for (int k = 0; k < 2; ++k) {
        float s = h->cls_pred_b[k];
        for (int i = 0; i < C; ++i) s += h->cls_pred_W[(size_t)k * C + i] * yc[i];
        out7[5 + k] = s;
    }
}
