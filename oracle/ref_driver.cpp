// ref_driver.cpp -- thin C entry points over the reference's own CPU sources.
//
// TEST INFRASTRUCTURE ONLY.  oracle/Makefile compiles this file together
// with the reference's vendor/src/weights_loader.cpp, straight from
// /root/reference, into oracle/_ref/libssla_ref.so.  Nothing here restates
// an algorithm: every function forwards to the reference implementation so
// the tests can pin the oracle and the product's host loader against it.
//
//   ref_meta        openeva::load_meta           vendor/src/weights_loader.cpp:162-252
//   ref_tensor      openeva::load_weights_npz    vendor/src/weights_loader.cpp:255-350
//   ref_head_decode openeva::heads::load_yolox_level + decode_yolox_cell_ct
//                                                vendor/openeva/heads/async_yolox.h:81-143,203-254
//   ref_layernorm   openeva::prim::layernorm_ct  vendor/openeva/prim/layernorm.h:40-60
//   ref_lru_step    openeva::prim::lru_step      vendor/openeva/prim/rnn.h:79-90
//   ref_mm          openeva::prim::mm            vendor/openeva/prim/matmul.h:22-38
//   ref_matvec96x7  openeva::prim::matvec_ct<96, 7>  vendor/openeva/prim/linear.h:80-91
//   ref_oeva_record deploy::OracleRecorder       include/oracle.h:35-89
//   ref_oeva_diff   deploy::diff_dumps           include/oracle.h:90-150
#include <cstring>
#include <exception>
#include <string>
#include <unordered_map>
#include <vector>

#include "openeva/output.h"
#include "openeva/heads/async_yolox.h"
#include "openeva/prim/layernorm.h"
#include "openeva/prim/linear.h"
#include "openeva/prim/matmul.h"
#include "openeva/prim/rnn.h"
#include "src/weights_loader.h"
#include "include/oracle.h"

extern "C" {

// out[0..3] = height, width, num_classes, ssla_tdrop_window; returns 0 / -1.
int ref_meta(const char* dir, int* out) {
    try {
        const openeva::ModelMeta m = openeva::load_meta(dir);
        out[0] = m.height;
        out[1] = m.width;
        out[2] = m.num_classes;
        out[3] = m.ssla_tdrop_window;
        return 0;
    } catch (const std::exception&) {
        return -1;
    }
}

// Copies tensor `key` of <dir>/weights.npz into out (cap floats).  Returns
// numel, -1 if the key is missing or the load fails, -2 if cap is short.
int ref_tensor(const char* dir, const char* key, float* out, int cap) {
    try {
        const auto W = openeva::load_weights_npz(dir);
        const auto it = W.find(key);
        if (it == W.end()) return -1;
        const int n = static_cast<int>(it->second.data.size());
        if (n > cap) return -2;
        std::memcpy(out, it->second.data.data(), sizeof(float) * n);
        return n;
    } catch (const std::exception&) {
        return -1;
    }
}

// Decoded YOLOX row [cx, cy, w, h, obj, cls...] for one 96-channel stage-3
// feature at grid cell (gx, gy), with the level loaded and BN-folded by the
// reference loader.  Returns the row width or -1.
int ref_head_decode(const char* dir, int gx, int gy, const float* feat,
                    float* out_row) {
    try {
        const openeva::ModelMeta m = openeva::load_meta(dir);
        const auto W = openeva::load_weights_npz(dir);
        openeva::heads::YoloxLevel lvl;
        const int Hg = m.height / 8, Wg = m.width / 8;
        openeva::heads::load_yolox_level(W, lvl, 0, 96, 96, m.num_classes,
                                         m.height / Hg, m.width / Wg, Hg, Wg,
                                         "ref_driver");
        std::vector<float> cls_f, reg_f, cls_logits;
        openeva::heads::decode_yolox_cell_ct<96, 96>(lvl, gx, gy, feat, out_row,
                                                     cls_f, reg_f, cls_logits);
        return 5 + m.num_classes;
    } catch (const std::exception&) {
        return -1;
    }
}

int ref_layernorm(float* x, int D, const float* gamma, const float* beta) {
    switch (D) {
        case 12: openeva::prim::layernorm_ct<12>(x, gamma, beta); return 0;
        case 24: openeva::prim::layernorm_ct<24>(x, gamma, beta); return 0;
        case 48: openeva::prim::layernorm_ct<48>(x, gamma, beta); return 0;
        case 96: openeva::prim::layernorm_ct<96>(x, gamma, beta); return 0;
        default: return -1;
    }
}

int ref_lru_step(const float* g, const float* v, const float* q, float* h,
                 float* y, int D) {
    switch (D) {
        case 48: openeva::prim::lru_step<48>(g, v, q, h, y); return 0;
        case 96: openeva::prim::lru_step<96>(g, v, q, h, y); return 0;
        default: return -1;
    }
}

// C = B @ A, B (bo, bi), A (bi, ai).
int ref_mm(const float* B, int bo, int bi, const float* A, int ai, float* C) {
    try {
        std::vector<float> vb(B, B + static_cast<std::size_t>(bo) * bi);
        std::vector<float> va(A, A + static_cast<std::size_t>(bi) * ai);
        const auto vc = openeva::prim::mm(vb, bo, bi, va, bi, ai);
        std::memcpy(C, vc.data(), sizeof(float) * vc.size());
        return 0;
    } catch (const std::exception&) {
        return -1;
    }
}

// y (7) = W x + bias with W (7, 96) row-major (bias may be NULL).
int ref_matvec96x7(const float* x, const float* W, const float* bias, float* y) {
    openeva::prim::matvec_ct<96, 7>(x, W, bias, y);
    return 0;
}

// Feeds n (event_idx, predictions) pairs to an OracleRecorder(num_anchors,
// cols, every, path) as DetectionOutputs of num_anchors*cols floats
// (preds + i*per) -- or of `sizes[i]` floats when sizes is non-NULL -- then
// saves.  Returns the number of checkpoints kept, or -1.
int ref_oeva_record(const char* path, int num_anchors, int cols, unsigned long long every, int n,
                    const unsigned long long* event_idx, const float* preds, const int* sizes) {
    try {
        deploy::OracleRecorder rec(num_anchors, cols, every, path);
        const std::size_t per = static_cast<std::size_t>(num_anchors) * cols;
        for (int i = 0; i < n; ++i) {
            openeva::DetectionOutput det;
            const std::size_t sz = sizes ? static_cast<std::size_t>(sizes[i]) : per;
            det.predictions.shape = {sz};
            det.predictions.data.assign(preds + i * per, preds + i * per + sz);
            rec.record(event_idx[i], openeva::ModelOutput{det});
        }
        rec.save();
        return static_cast<int>(rec.num_checkpoints());
    } catch (const std::exception&) {
        return -1;
    }
}

// out = {ok, n_cp, max_abs_delta, n_mismatched_cp}; returns 0 or -1 (throw).
int ref_oeva_diff(const char* a, const char* b, double tol_abs, double* out) {
    try {
        const deploy::DiffReport r = deploy::diff_dumps(a, b, tol_abs);
        out[0] = r.ok ? 1.0 : 0.0;
        out[1] = static_cast<double>(r.n_cp);
        out[2] = r.max_abs_delta;
        out[3] = static_cast<double>(r.n_mismatched_cp);
        return 0;
    } catch (const std::exception&) {
        return -1;
    }
}

}  // extern "C"
