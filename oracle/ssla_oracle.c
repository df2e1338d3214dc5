/*
 * ssla_oracle.c -- CPU restatement of the SSLA-S s2+s3+head drain path.
 *
 * TEST INFRASTRUCTURE ONLY (see ssla_oracle.h for the rules and the list of
 * reference files each function follows).  Built by oracle/Makefile into
 * oracle/libssla_oracle.so with the reference CPU build's flags
 * (CMakeLists.txt:18-25: -O3 -march=native -ffast-math) for the fp32 path;
 * the fp64 path is compiled in a separate translation unit without
 * -ffast-math so its summation order is the one written here.
 */
#include "ssla_oracle.h"

#include <math.h>
#include <stdlib.h>
#include <string.h>

#define MAXD 96          /* largest channel count on the path (C3) */

/* ------------------------------------------------------------------------ */
/* reshape (weights_ssla.py:24-88, ssla_kernels.cpp:73-153)                 */
/* ------------------------------------------------------------------------ */

/* C = B @ A with B (bo, bi), A (bi, ai); k-outer accumulation in fp32 as in
 * vendor/openeva/prim/matmul.h:22-38.                                       */
static void mm_f32(const float* B, int bo, int bi, const float* A, int ai,
                   float* C) {
    for (int o = 0; o < bo; ++o) {
        float* cr = C + (size_t)o * ai;
        for (int i = 0; i < ai; ++i) cr[i] = 0.0f;
        for (int k = 0; k < bi; ++k) {
            const float bv = B[(size_t)o * bi + k];
            const float* ar = A + (size_t)k * ai;
            for (int i = 0; i < ai; ++i) cr[i] += bv * ar[i];
        }
    }
}

int oracle_reshape_layer(const float* W_in_cat, int win_cols,
                         const float* W_out_cat, int wout_rows,
                         const float* qW, const float* vW,
                         const float* gW, const float* oW,
                         int in_dim, int D, float* qvgIn, float* goW) {
    if (D <= 0 || D > MAXD || in_dim <= 0 || in_dim > MAXD) return -1;
    if (win_cols % D != 0 || wout_rows % D != 0) return -1;
    const int n_in = win_cols / D, n_out = wout_rows / D;
    const int A = n_in > n_out ? n_in : n_out;
    float* scatter = (float*)malloc(sizeof(float) * D * in_dim);
    float* gather = (float*)malloc(sizeof(float) * D * D);
    if (!scatter || !gather) { free(scatter); free(gather); return -1; }
    for (int p = 0; p < A; ++p) {
        const int pin = (n_in == 1) ? 0 : p;
        const int pout = (n_out == 1) ? 0 : p;
        /* scatter[d, c] = W_in_cat[c, pin*D + d] */
        for (int d = 0; d < D; ++d)
            for (int c = 0; c < in_dim; ++c)
                scatter[(size_t)d * in_dim + c] =
                    W_in_cat[(size_t)c * win_cols + (size_t)pin * D + d];
        /* gather[i, j] = W_out_cat[pout*D + j, i] */
        for (int i = 0; i < D; ++i)
            for (int j = 0; j < D; ++j)
                gather[(size_t)i * D + j] =
                    W_out_cat[((size_t)pout * D + j) * D + i];
        float* qvg = qvgIn + (size_t)p * 3 * D * in_dim;
        mm_f32(qW, D, D, scatter, in_dim, qvg);
        mm_f32(vW, D, D, scatter, in_dim, qvg + (size_t)D * in_dim);
        mm_f32(gW, D, D, scatter, in_dim, qvg + (size_t)2 * D * in_dim);
        mm_f32(gather, D, D, oW, D, goW + (size_t)p * D * D);
    }
    free(scatter);
    free(gather);
    return A;
}

/* ------------------------------------------------------------------------ */
/* patch walk shared by both precisions                                     */
/* ------------------------------------------------------------------------ */

/* Fills (cell index, delta) for the in-bounds patch cells of an event, in
 * the order the reference visits them: interior events use the fixed
 * delta 8..0 table (ssla_ref.py:72-77, ssla_kernels.cpp:349-358); events on
 * the border walk dy, dx = -1..1 with delta = (1-dy)*3 + (1-dx)
 * (ssla_ref.py:79-86).  K = 1 visits only the centre with delta 0.         */
static int patch_list(int K, int ev_x, int ev_y, int Hl, int Wl,
                      int cells[9], int deltas[9]) {
    if (K == 1) {
        cells[0] = ev_y * Wl + ev_x;
        deltas[0] = 0;
        return 1;
    }
    const int base = ev_y * Wl + ev_x;
    const int interior = ev_x > 0 && ev_x + 1 < Wl && ev_y > 0 && ev_y + 1 < Hl;
    if (interior) {
        const int offs[9] = {-Wl - 1, -Wl, -Wl + 1, -1, 0, 1, Wl - 1, Wl, Wl + 1};
        for (int k = 0; k < 9; ++k) {
            cells[k] = base + offs[k];
            deltas[k] = 8 - k;
        }
        return 9;
    }
    int n = 0;
    for (int dy = -1; dy <= 1; ++dy) {
        const int py = ev_y + dy;
        if (py < 0 || py >= Hl) continue;
        for (int dx = -1; dx <= 1; ++dx) {
            const int px = ev_x + dx;
            if (px < 0 || px >= Wl) continue;
            cells[n] = py * Wl + px;
            deltas[n] = (1 - dy) * 3 + (1 - dx);
            ++n;
        }
    }
    return n;
}

/* fp64 LayerNorm over OUT values with eps = 1e-5, affine in fp64 then cast
 * (ssla_ref.py:88-93; layernorm.h:40-60 does the same in fp64).            */
static void layernorm_f64(const double* y, int D, const float* gamma,
                          const float* beta, float* out) {
    double sum = 0.0;
    for (int i = 0; i < D; ++i) sum += y[i];
    const double mean = sum / (double)D;
    double var = 0.0;
    for (int i = 0; i < D; ++i) {
        const double d = y[i] - mean;
        var += d * d;
    }
    var /= (double)D;
    const double inv = 1.0 / sqrt(var + 1e-5);
    for (int i = 0; i < D; ++i)
        out[i] = (float)((y[i] - mean) * inv * (double)gamma[i] + (double)beta[i]);
}

/* ------------------------------------------------------------------------ */
/* layer_step, fp64 (ssla_ref.py:17-93)                                     */
/* ------------------------------------------------------------------------ */

/* out[r] = sum_i W[r*IN + i] * x[i] for r < rows, each sum taken in fp64 in
 * index order i = 0..IN-1.  Eight rows run side by side so their eight
 * dependency chains overlap; the order of every single sum is unchanged.  */
#define ROWS_DOT_F64(NAME, XT)                                                \
static void NAME(const float* W, int rows, int IN, const XT* x, double* out) { \
    int r = 0;                                                                \
    for (; r + 8 <= rows; r += 8) {                                           \
        const float* w0 = W + (size_t)r * IN;                                 \
        const float *w1 = w0 + IN, *w2 = w1 + IN, *w3 = w2 + IN;              \
        const float *w4 = w3 + IN, *w5 = w4 + IN, *w6 = w5 + IN, *w7 = w6 + IN; \
        double s0 = 0.0, s1 = 0.0, s2 = 0.0, s3 = 0.0;                        \
        double s4 = 0.0, s5 = 0.0, s6 = 0.0, s7 = 0.0;                        \
        for (int i = 0; i < IN; ++i) {                                        \
            const double xi = (double)x[i];                                   \
            s0 += (double)w0[i] * xi; s1 += (double)w1[i] * xi;               \
            s2 += (double)w2[i] * xi; s3 += (double)w3[i] * xi;               \
            s4 += (double)w4[i] * xi; s5 += (double)w5[i] * xi;               \
            s6 += (double)w6[i] * xi; s7 += (double)w7[i] * xi;               \
        }                                                                     \
        out[r] = s0; out[r + 1] = s1; out[r + 2] = s2; out[r + 3] = s3;       \
        out[r + 4] = s4; out[r + 5] = s5; out[r + 6] = s6; out[r + 7] = s7;   \
    }                                                                         \
    for (; r < rows; ++r) {                                                   \
        double s = 0.0;                                                       \
        const float* w = W + (size_t)r * IN;                                  \
        for (int i = 0; i < IN; ++i) s += (double)w[i] * (double)x[i];        \
        out[r] = s;                                                           \
    }                                                                         \
}
ROWS_DOT_F64(rows_dot_f32in, float)
ROWS_DOT_F64(rows_dot_f64in, double)

/* The same sums over the input-major copy WT[i*rows + r]: the loop over r
 * is innermost, so the compiler can run it on vector lanes, while each
 * out[r] still adds its terms in the order i = 0..IN-1.                    */
#define COLS_DOT_F64(NAME, XT)                                                \
static void NAME(const float* WT, int rows, int IN, const XT* x, double* out) { \
    for (int r = 0; r < rows; ++r) out[r] = 0.0;                              \
    for (int i = 0; i < IN; ++i) {                                            \
        const double xi = (double)x[i];                                       \
        const float* w = WT + (size_t)i * rows;                               \
        for (int r = 0; r < rows; ++r) out[r] += (double)w[r] * xi;           \
    }                                                                         \
}
COLS_DOT_F64(cols_dot_f32in, float)
COLS_DOT_F64(cols_dot_f64in, double)

void oracle_layer_step_f64(const OracleLayer* L, const float* in,
                           float* H_all, int ev_x, int ev_y, int Hl, int Wl,
                           float* out) {
    const int IN = L->in_dim, D = L->out_dim;
    double acc[MAXD], res[MAXD], qvg[3 * MAXD], qh[MAXD];
    if (L->input_proj) {
        rows_dot_f32in(L->input_proj, D, IN, in, res);
    } else {
        for (int o = 0; o < D; ++o) res[o] = (double)in[o];
    }
    for (int o = 0; o < D; ++o) acc[o] = 0.0;

    int cells[9], deltas[9];
    const int np = patch_list(L->K, ev_x, ev_y, Hl, Wl, cells, deltas);
    for (int k = 0; k < np; ++k) {
        const int p = deltas[k];
        if (L->qvgInT)
            cols_dot_f32in(L->qvgInT + (size_t)p * 3 * D * IN, 3 * D, IN, in, qvg);
        else
            rows_dot_f32in(L->qvgIn + (size_t)p * 3 * D * IN, 3 * D, IN, in, qvg);
        float* h = H_all + (size_t)cells[k] * D;
        for (int o = 0; o < D; ++o) {
            const double gc = 1.0 / (1.0 + exp(-qvg[2 * D + o]));
            const double hn = gc * (double)h[o] + qvg[D + o];
            h[o] = (float)hn;              /* stored back as fp32 */
            qh[o] = qvg[o] * hn;           /* q * h_new in fp64 */
        }
        double go[MAXD];
        if (L->goWT)
            cols_dot_f64in(L->goWT + (size_t)p * D * D, D, D, qh, go);
        else
            rows_dot_f64in(L->goW + (size_t)p * D * D, D, D, qh, go);
        for (int o = 0; o < D; ++o) acc[o] += go[o];
    }
    for (int o = 0; o < D; ++o) acc[o] += res[o];
    layernorm_f64(acc, D, L->ln_gamma, L->ln_beta, out);
}

/* ------------------------------------------------------------------------ */
/* tdrop (ssla_ref.py:190-195, ssla_kernels.cpp:912-921)                    */
/* ------------------------------------------------------------------------ */

int oracle_tdrop(uint8_t* counter, int window, int idx) {
    const uint8_t pre = counter[idx];
    counter[idx] = (uint8_t)(pre + 1u);
    if (window <= 1) return 1;
    return (pre % (unsigned)window) == 0u;
}

/* ------------------------------------------------------------------------ */
/* head (…celled.cuh:841-902): y = SiLU(Wc x + bc) -> cls; y' = SiLU(Wr x +
 * br) -> reg, obj; output [reg0..3, obj, cls0, cls1]                       */
/* ------------------------------------------------------------------------ */

/* single-linear head (…celled.cuh:1476-1481): matvec_w<C3, 7>
 * (proto_layer_pair.cuh:39-58) reads W[i*7 + o], then head_b is added     */
static void head_linear_f64(const OracleHead* h, const float* x, float out7[7]) {
    for (int o = 0; o < 7; ++o) {
        double s = 0.0;
        for (int i = 0; i < h->C; ++i) s += (double)h->lin_W[(size_t)i * 7 + o] * (double)x[i];
        out7[o] = (float)(s + (double)h->lin_b[o]);
    }
}

void oracle_head_raw_f64(const OracleHead* h, const float* x, float out7[7]) {
    if (!h->cls_conv_W) {
        head_linear_f64(h, x, out7);
        return;
    }
    const int C = h->C;
    double yc[MAXD], yr[MAXD];
    for (int o = 0; o < C; ++o) {
        double a = (double)h->cls_conv_b[o], b = (double)h->reg_conv_b[o];
        const float* wc = h->cls_conv_W + (size_t)o * C;
        const float* wr = h->reg_conv_W + (size_t)o * C;
        for (int i = 0; i < C; ++i) {
            a += (double)wc[i] * (double)x[i];
            b += (double)wr[i] * (double)x[i];
        }
        yc[o] = a / (1.0 + exp(-a));
        yr[o] = b / (1.0 + exp(-b));
    }
    for (int k = 0; k < 4; ++k) {
        double s = (double)h->reg_pred_b[k];
        for (int i = 0; i < C; ++i) s += (double)h->reg_pred_W[(size_t)k * C + i] * yr[i];
        out7[k] = (float)s;
    }
    {
        double s = (double)h->obj_pred_b[0];
        for (int i = 0; i < C; ++i) s += (double)h->obj_pred_W[i] * yr[i];
        out7[4] = (float)s;
    }
    for (int k = 0; k < 2; ++k) {
        double s = (double)h->cls_pred_b[k];
        for (int i = 0; i < C; ++i) s += (double)h->cls_pred_W[(size_t)k * C + i] * yc[i];
        out7[5 + k] = (float)s;
    }
}

/* ------------------------------------------------------------------------ */
/* decisions (bench_s2_s3_head_celled.py:70-84)                             */
/* ------------------------------------------------------------------------ */

static int in_grid(int x, int y, int H, int W) {
    return x >= 0 && x < W && y >= 0 && y < H;
}

int oracle_s2s3_decisions(uint8_t* td2, uint8_t* td3, int H2, int W2,
                          int window, const uint16_t* xs, const uint16_t* ys,
                          int n, int8_t* pass2, int8_t* pass3) {
    if (n < 0 || H2 <= 0 || W2 <= 0) return -1;
    const int W3 = W2 >> 1;
    int n3 = 0;
    for (int i = 0; i < n; ++i) {
        const int x = xs[i], y = ys[i];
        int p2 = -2, p3 = -2;
        if (in_grid(x, y, H2, W2)) {
            p2 = oracle_tdrop(td2, window, y * W2 + x);
            p3 = 0;
            if (p2) {
                p3 = oracle_tdrop(td3, window, (y >> 1) * W3 + (x >> 1));
                n3 += p3;
            }
        }
        if (pass2) pass2[i] = (int8_t)p2;
        if (pass3) pass3[i] = (int8_t)p3;
    }
    return n3;
}

/* ------------------------------------------------------------------------ */
/* full schedule, both precisions                                           */
/* ------------------------------------------------------------------------ */

typedef void (*layer_fn)(const OracleLayer*, const float*, float*, int, int,
                         int, int, float*);

int oracle_s2s3_run(OracleS2S3* st, const uint16_t* xs, const uint16_t* ys,
                    const float* feat1, const uint8_t* owner, int n,
                    int precision, int8_t* pass2, int8_t* pass3,
                    float* s3_feat, float* head7) {
    if (!st || n < 0 || (precision != 32 && precision != 64)) return -1;
    if (st->H2 <= 0 || st->W2 <= 0 || (st->H2 & 1) || (st->W2 & 1)) return -1;
    if (head7 && !st->head) return -1;
    const layer_fn step = (precision == 64) ? oracle_layer_step_f64
                                            : oracle_layer_step_f32;
    const int H2 = st->H2, W2 = st->W2, H3 = st->H3, W3 = st->W3;
    float b4[MAXD], b5[MAXD], b6[MAXD], b7[MAXD];
    int n3 = 0;
    for (int i = 0; i < n; ++i) {
        const int x = xs[i], y = ys[i];
        int p2 = -2, p3 = -2;
        if (s3_feat) memset(s3_feat + (size_t)i * 96, 0, sizeof(float) * 96);
        if (head7) memset(head7 + (size_t)i * 7, 0, sizeof(float) * 7);
        if (in_grid(x, y, H2, W2)) {
            const float* f = feat1 + (size_t)i * 24;
            step(&st->L[0], f, st->H[0], x, y, H2, W2, b4);
            step(&st->L[1], b4, st->H[1], x, y, H2, W2, b5);
            p2 = oracle_tdrop(st->td2, st->window, y * W2 + x);
            p3 = 0;
            if (p2) {
                const int sx = x >> 1, sy = y >> 1;
                step(&st->L[2], b5, st->H[2], sx, sy, H3, W3, b6);
                step(&st->L[3], b6, st->H[3], sx, sy, H3, W3, b7);
                p3 = oracle_tdrop(st->td3, st->window, sy * W3 + sx);
                if (p3) {
                    ++n3;
                    if (s3_feat) memcpy(s3_feat + (size_t)i * 96, b7, sizeof(float) * 96);
                    if (head7 && (!owner || owner[i])) {
                        if (precision == 64) oracle_head_raw_f64(st->head, b7, head7 + (size_t)i * 7);
                        else oracle_head_raw_f32(st->head, b7, head7 + (size_t)i * 7);
                    }
                }
            }
        }
        if (pass2) pass2[i] = (int8_t)p2;
        if (pass3) pass3[i] = (int8_t)p3;
    }
    return n3;
}

/* ------------------------------------------------------------------------ */
/* One producer shard, stages 0 + 1                                          */
/* ------------------------------------------------------------------------ */

/* dt_norm = clamp((t - last) / 1e5, 0, 1), 1 for a pixel's first event;
 * zeros outside the sensor (src/ssla_kernels.cpp:288-309). */
void oracle_preprocess(double* last_t, int height, int width, float t_us, int x, int y,
                       float p, float feat[2]) {
    if (!in_grid(x, y, height, width)) {
        feat[0] = feat[1] = 0.0f;
        return;
    }
    const int pix = y * width + x;
    const double prev = last_t[pix];
    float dt = 1.0f;
    if (prev >= 0.0) {
        double v = ((double)t_us - prev) / 1e5;
        if (v < 0.0) v = 0.0;
        if (v > 1.0) v = 1.0;
        dt = (float)v;
    }
    last_t[pix] = (double)t_us;
    feat[0] = dt;
    feat[1] = p;
}

int oracle_s01_run(OracleS01* st, const float* ev, const uint8_t* owner, int n,
                   int precision, int8_t* pass0, int8_t* pass1, float* feat1,
                   uint16_t* x2, uint16_t* y2) {
    if (!st || !ev || n < 0 || (precision != 32 && precision != 64)) return -1;
    if (st->height <= 0 || st->width <= 0 || (st->height & 3) || (st->width & 3)) return -1;
    const layer_fn step = (precision == 64) ? oracle_layer_step_f64
                                            : oracle_layer_step_f32;
    const int H0 = st->height, W0 = st->width, H1 = H0 >> 1, W1 = W0 >> 1, W2 = W0 >> 2;
    float in[2], b0[MAXD], b1[MAXD], b2[MAXD], b3[MAXD];
    int n1 = 0;
    for (int i = 0; i < n; ++i) {
        const float* e = ev + (size_t)i * 4;
        const int x = (int)e[1], y = (int)e[2];
        int p0 = -2, p1 = -2;
        if (feat1) memset(feat1 + (size_t)i * 24, 0, sizeof(float) * 24);
        if (x2) x2[i] = 0;
        if (y2) y2[i] = 0;
        if (in_grid(x, y, H0, W0)) {
            oracle_preprocess(st->last_t, H0, W0, e[0], x, y, e[3], in);
            step(&st->L[0], in, st->H[0], x, y, H0, W0, b0);
            step(&st->L[1], b0, st->H[1], x, y, H0, W0, b1);
            if (owner && !owner[i]) {
                p0 = p1 = -1;
            } else {
                const int sx = x >> 1, sy = y >> 1;
                p0 = oracle_tdrop(st->td0, st->window, sy * W1 + sx);
                p1 = 0;
                if (p0) {
                    step(&st->L[2], b1, st->H[2], sx, sy, H1, W1, b2);
                    step(&st->L[3], b2, st->H[3], sx, sy, H1, W1, b3);
                    p1 = oracle_tdrop(st->td1, st->window, (sy >> 1) * W2 + (sx >> 1));
                    if (p1) {
                        ++n1;
                        if (feat1) memcpy(feat1 + (size_t)i * 24, b3, sizeof(float) * 24);
                        if (x2) x2[i] = (uint16_t)(sx >> 1);
                        if (y2) y2[i] = (uint16_t)(sy >> 1);
                    }
                }
            }
        }
        if (pass0) pass0[i] = (int8_t)p0;
        if (pass1) pass1[i] = (int8_t)p1;
    }
    return n1;
}

/* ------------------------------------------------------------------------ */
/* BN fold (hybrid_common.py:327-349)                                       */
/* ------------------------------------------------------------------------ */

void oracle_fuse_conv_bn(const float* W, const float* b_conv_or_null,
                         const float* bn_w, const float* bn_b,
                         const float* bn_mu, const float* bn_var,
                         int c_out, int c_in, float eps,
                         float* W_out, float* b_out) {
    for (int o = 0; o < c_out; ++o) {
        const float scale = bn_w[o] / sqrtf(bn_var[o] + eps);
        const float shift = bn_b[o] - scale * bn_mu[o];
        for (int i = 0; i < c_in; ++i)
            W_out[(size_t)o * c_in + i] = W[(size_t)o * c_in + i] * scale;
        const float bc = b_conv_or_null ? b_conv_or_null[o] : 0.0f;
        b_out[o] = bc * scale + shift;
    }
}
