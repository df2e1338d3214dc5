// grid.cpp -- host-side consumer of the drain's prediction grid.
//
// Host code only (no HIP calls), so every entry point also runs where no
// GPU is present.  Covers what the reference does on the CPU after the
// device head has written a cell:
//   * torn-free reads of cells the device may be writing
//     (the reference reads the pinned preds/version views directly,
//     orin/hybrid_runner_multi.py:648-656, orin/orin/multi_block.py:229-253);
//   * the YOLOX grid/exp/stride decode
//     (vendor/openeva/heads/async_yolox.h:189-196);
//   * the live demo's box collection (orin/hybrid_runner_multi.py:163-207);
//   * the OEVA head-grid dump format and its diff (include/oracle.h:10-18,
//     57-77, 90-150).
#include <atomic>
#include <chrono>
#include <cmath>
#include <cstdint>
#include <cstdio>
#include <cstring>
#include <exception>
#include <string>
#include <vector>

#include "ssla_hip.h"

namespace ssla {
void set_error(const std::string& msg);
}  // namespace ssla

using ssla::set_error;

namespace {

constexpr unsigned kBusy = SSLA_PRED_BUSY;

inline unsigned load_acquire(const unsigned* p) {
    return __atomic_load_n(p, __ATOMIC_ACQUIRE);
}

// About a microsecond between two reads of a busy cell: the device's
// publish of one cell (two system fences over PCIe) takes microseconds, so
// back-to-back retries would all land inside one write.
inline void backoff() {
    const auto t0 = std::chrono::steady_clock::now();
    while (std::chrono::steady_clock::now() - t0 < std::chrono::microseconds(1)) __builtin_ia32_pause();
}

// One cell of `cols` floats read between two acquire loads of its version.
// Returns true when both loads agree and the busy bit is clear.
bool read_cell(const float* src, const unsigned* ver, int cols, float* dst, unsigned* vout) {
    const unsigned v1 = load_acquire(ver);
    if (v1 & kBusy) {
        *vout = v1;
        return false;
    }
    const uint32_t* s = reinterpret_cast<const uint32_t*>(src);
    for (int q = 0; q < cols; ++q) {
        const uint32_t bits = __atomic_load_n(s + q, __ATOMIC_RELAXED);
        std::memcpy(dst + q, &bits, 4);
    }
    std::atomic_thread_fence(std::memory_order_acquire);
    const unsigned v2 = load_acquire(ver);
    *vout = v2;
    return v1 == v2;
}

// decode_yolox_cell's transform (async_yolox.h:189-196) on one raw row.
inline void decode_row(const float* raw, int gx, int gy, int sw, int sh, int cols, float* out) {
    out[0] = (raw[0] + float(gx)) * float(sw);
    out[1] = (raw[1] + float(gy)) * float(sh);
    out[2] = std::exp(raw[2]) * float(sw);
    out[3] = std::exp(raw[3]) * float(sh);
    for (int c = 4; c < cols; ++c) out[c] = raw[c];
}

struct OevaFile {
    uint32_t na = 0, cols = 0, ncp = 0;
    std::vector<uint64_t> idx;
    std::vector<float> preds;   // ncp * na * cols
};

// Header + checkpoints as include/oracle.h:100-121 reads them: a short read
// of a checkpoint ends the read and leaves that checkpoint and the rest
// zero-filled.
int oeva_load(const char* path, OevaFile& f, bool body) {
    if (!path) { set_error("oeva: null path"); return SSLA_ERR_ARG; }
    std::FILE* fp = std::fopen(path, "rb");
    if (!fp) { set_error(std::string("oeva: cannot open ") + path); return SSLA_ERR_IO; }
    uint32_t hdr[5];
    if (std::fread(hdr, 4, 5, fp) != 5) {
        std::fclose(fp);
        set_error(std::string("oeva: header read failed: ") + path);
        return SSLA_ERR_FORMAT;
    }
    if (hdr[0] != SSLA_OEVA_MAGIC || hdr[1] != SSLA_OEVA_VERSION) {
        std::fclose(fp);
        set_error(std::string("oeva: bad magic/version: ") + path);
        return SSLA_ERR_FORMAT;
    }
    f.na = hdr[2];
    f.cols = hdr[3];
    f.ncp = hdr[4];
    const size_t per = size_t(f.na) * f.cols;
    // a corrupt header must not turn into a huge allocation (here or in a
    // caller sizing its buffers from the header): a dump's checkpoints stay
    // far below 4 Gi floats
    if (per > (size_t(1) << 28) || size_t(f.ncp) * per > (size_t(1) << 32)) {
        std::fclose(fp);
        set_error(std::string("oeva: implausible header sizes: ") + path);
        return SSLA_ERR_FORMAT;
    }
    if (body) {
        try {
            f.idx.assign(f.ncp, 0);
            f.preds.assign(size_t(f.ncp) * per, 0.0f);
        } catch (const std::exception&) {
            std::fclose(fp);
            set_error(std::string("oeva: out of memory reading ") + path);
            return SSLA_ERR_IO;
        }
        for (uint32_t i = 0; i < f.ncp; ++i) {
            if (std::fread(&f.idx[i], 8, 1, fp) != 1) break;
            if (std::fread(f.preds.data() + i * per, sizeof(float), per, fp) != per) break;
        }
    }
    std::fclose(fp);
    return SSLA_OK;
}

}  // namespace

extern "C" {

int ssla_hip_preds_snapshot(const float* preds, const unsigned* version, int n_cells, int cols,
                            float* preds_out, unsigned* version_out, int max_tries) {
    if (!preds || !version || !preds_out || !version_out || n_cells < 0 || cols <= 0) {
        set_error("preds_snapshot: bad argument");
        return SSLA_ERR_ARG;
    }
    if (max_tries < 1) max_tries = 1;
    int torn = 0;
    for (int c = 0; c < n_cells; ++c) {
        const float* src = preds + size_t(c) * cols;
        float* dst = preds_out + size_t(c) * cols;
        bool ok = false;
        for (int t = 0; t < max_tries && !ok; ++t) {
            if (t) backoff();
            ok = read_cell(src, version + c, cols, dst, version_out + c);
        }
        if (!ok) {
            version_out[c] |= kBusy;
            ++torn;
        }
    }
    return torn;
}

int ssla_hip_decode_cells(const float* raw, int n_cells, int cols, int grid_w, int gx0, int gy0,
                          int stride_w, int stride_h, float* out) {
    if (!raw || !out || n_cells < 0 || cols < 5 || grid_w <= 0) {
        set_error("decode_cells: bad argument");
        return SSLA_ERR_ARG;
    }
    for (int c = 0; c < n_cells; ++c)
        decode_row(raw + size_t(c) * cols, gx0 + c % grid_w, gy0 + c / grid_w, stride_w, stride_h, cols,
                   out + size_t(c) * cols);
    return SSLA_OK;
}

int ssla_hip_grid_decode(const HybridS2S3Config* cfg, const float* zero_row, int stride_w,
                         int stride_h, int max_tries, float* out) {
    if (!cfg || !zero_row || !out || cfg->n_blocks < 0 || cfg->n_blocks > SSLA_MAX_BLOCKS ||
        cfg->H3 <= 0 || cfg->W3 <= 0) {
        set_error("grid_decode: bad argument");
        return SSLA_ERR_ARG;
    }
    const int cols = SSLA_HEAD_OUT;
    const int W3 = cfg->W3, H3 = cfg->H3;
    // Untouched cells hold the head's output for an all-zero feature, as a
    // freshly built CPU pipeline does (src/ssla_kernels.cpp:966-987).
    std::vector<float> raw;
    try {
        raw.resize(size_t(H3) * W3 * cols);
    } catch (const std::exception&) {
        set_error("grid_decode: cannot hold the s3 grid");
        return SSLA_ERR_ARG;
    }
    for (size_t c = 0; c < size_t(H3) * W3; ++c) std::memcpy(&raw[c * cols], zero_row, sizeof(float) * cols);
    int torn = 0;
    std::vector<float> cell(cols);
    for (int b = 0; b < cfg->n_blocks; ++b) {
        const HybridStrip& s = cfg->strip[b];
        const float* p = cfg->preds[b];
        const unsigned* v = cfg->version[b];
        if (!p || !v) continue;
        const int w = s.s3_owned_hi - s.s3_owned_lo, h = s.s3_owned_y_hi - s.s3_owned_y_lo;
        if (w <= 0 || h <= 0 || s.s3_owned_lo < 0 || s.s3_owned_hi > W3 || s.s3_owned_y_lo < 0 ||
            s.s3_owned_y_hi > H3) {
            if (w > 0 && h > 0) {
                set_error("grid_decode: block " + std::to_string(b) + " owned box outside the s3 grid");
                return SSLA_ERR_ARG;
            }
            continue;
        }
        for (int i = 0; i < w * h; ++i) {
            unsigned ver = 0;
            bool ok = false;
            for (int t = 0; t < (max_tries < 1 ? 1 : max_tries) && !ok; ++t) {
                if (t) backoff();
                ok = read_cell(p + size_t(i) * cols, v + i, cols, cell.data(), &ver);
            }
            if (!ok) ++torn;
            if (!ok || ver == 0) continue;
            const int gx = s.s3_owned_lo + i % w, gy = s.s3_owned_y_lo + i / w;
            std::memcpy(&raw[(size_t(gy) * W3 + gx) * cols], cell.data(), sizeof(float) * cols);
        }
    }
    for (int gy = 0; gy < H3; ++gy)
        for (int gx = 0; gx < W3; ++gx) {
            const size_t c = size_t(gy) * W3 + gx;
            decode_row(&raw[c * cols], gx, gy, stride_w, stride_h, cols, out + c * cols);
        }
    return torn;
}

int ssla_hip_collect_boxes(const float* raw, int s3w, int s3h, int s3x_lo, int s3y_lo, float scale,
                           float obj_thresh, int W_full, int H_full, float* boxes_xywh,
                           float* scores, int max_boxes, float* max_seen) {
    if (!max_seen || s3w < 0 || s3h < 0 || (s3w > 0 && s3h > 0 && !raw) ||
        (max_boxes > 0 && (!boxes_xywh || !scores))) {
        set_error("collect_boxes: bad argument");
        return SSLA_ERR_ARG;
    }
    if (s3w == 0 || s3h == 0) return 0;
    const int cols = SSLA_HEAD_OUT;
    int kept = 0;
    for (int k = 0; k < s3w * s3h; ++k) {
        const float* r = raw + size_t(k) * cols;
        const float obj = 1.0f / (1.0f + std::exp(-r[4]));
        if (obj > *max_seen) *max_seen = obj;
        if (!(obj >= obj_thresh)) continue;
        const float s3y = float(s3y_lo) + float(k / s3w);
        const float s3x = float(s3x_lo) + float(k % s3w);
        const float cx_in = s3x * 8.0f + 4.0f + r[0] * 8.0f;
        const float cy_in = s3y * 8.0f + 4.0f + r[1] * 8.0f;
        const float w_in = std::fmin(std::fmax(std::exp(r[2]) * 8.0f, 2.0f), float(W_full));
        const float h_in = std::fmin(std::fmax(std::exp(r[3]) * 8.0f, 2.0f), float(H_full));
        if (kept < max_boxes) {
            float* bx = boxes_xywh + size_t(kept) * 4;
            bx[0] = (cx_in - w_in / 2.0f) * scale;
            bx[1] = (cy_in - h_in / 2.0f) * scale;
            bx[2] = w_in * scale;
            bx[3] = h_in * scale;
            scores[kept] = obj;
        }
        ++kept;
    }
    return kept;
}

int ssla_hip_oeva_write(const char* path, unsigned num_anchors, unsigned cols, unsigned n_cp,
                        const unsigned long long* event_idx, const float* preds) {
    if (!path || num_anchors == 0 || cols == 0 || (n_cp > 0 && (!event_idx || !preds))) {
        set_error("oeva_write: bad argument");
        return SSLA_ERR_ARG;
    }
    std::FILE* fp = std::fopen(path, "wb");
    if (!fp) { set_error(std::string("oeva: cannot open ") + path); return SSLA_ERR_IO; }
    const uint32_t hdr[5] = {SSLA_OEVA_MAGIC, SSLA_OEVA_VERSION, num_anchors, cols, n_cp};
    bool ok = std::fwrite(hdr, 4, 5, fp) == 5;
    const size_t per = size_t(num_anchors) * cols;
    for (unsigned i = 0; ok && i < n_cp; ++i) {
        const uint64_t e = event_idx[i];
        ok = std::fwrite(&e, 8, 1, fp) == 1 && std::fwrite(preds + i * per, sizeof(float), per, fp) == per;
    }
    ok = (std::fclose(fp) == 0) && ok;
    if (!ok) { set_error(std::string("oeva: write failed: ") + path); return SSLA_ERR_IO; }
    return SSLA_OK;
}

int ssla_hip_oeva_header(const char* path, unsigned* out3) {
    if (!out3) { set_error("oeva_header: null out"); return SSLA_ERR_ARG; }
    OevaFile f;
    const int rc = oeva_load(path, f, false);
    if (rc != SSLA_OK) return rc;
    out3[0] = f.na;
    out3[1] = f.cols;
    out3[2] = f.ncp;
    return SSLA_OK;
}

int ssla_hip_oeva_read(const char* path, unsigned long long* event_idx, float* preds,
                       unsigned cap_cp) {
    OevaFile f;
    const int rc = oeva_load(path, f, true);
    if (rc != SSLA_OK) return rc;
    if (f.ncp > cap_cp || (f.ncp > 0 && (!event_idx || !preds))) {
        set_error("oeva_read: output holds fewer checkpoints than the file");
        return SSLA_ERR_ARG;
    }
    for (uint32_t i = 0; i < f.ncp; ++i) event_idx[i] = f.idx[i];
    if (!f.preds.empty()) std::memcpy(preds, f.preds.data(), f.preds.size() * sizeof(float));
    return SSLA_OK;
}

int ssla_hip_oeva_diff(const char* path_a, const char* path_b, double tol_abs,
                       SslaHipOevaDiff* out) {
    if (!out) { set_error("oeva_diff: null out"); return SSLA_ERR_ARG; }
    std::memset(out, 0, sizeof(*out));
    OevaFile a, b;
    int rc = oeva_load(path_a, a, true);
    if (rc != SSLA_OK) return rc;
    rc = oeva_load(path_b, b, true);
    if (rc != SSLA_OK) return rc;
    out->ok = (a.na == b.na && a.cols == b.cols && a.ncp == b.ncp) ? 1 : 0;
    out->n_cp = a.ncp;
    if (!out->ok) return SSLA_OK;
    const size_t per = size_t(a.na) * a.cols;
    for (uint32_t i = 0; i < a.ncp; ++i) {
        if (a.idx[i] != b.idx[i]) {
            out->ok = 0;
            break;
        }
        double cp_max = 0.0;
        for (size_t j = 0; j < per; ++j) {
            const double d = std::fabs(double(a.preds[i * per + j]) - double(b.preds[i * per + j]));
            if (d > cp_max) cp_max = d;   // NaN compares false and is passed over
        }
        if (cp_max > out->max_abs_delta) out->max_abs_delta = cp_max;
        if (cp_max > tol_abs) ++out->n_mismatched_cp;
    }
    return SSLA_OK;
}

}  // extern "C"
