// api.cpp -- the C ABI of libssla_hip.so (include/ssla_hip.h): memory
// helpers, weight-directory loading and packing, configuration binding,
// per-block state, and the drain entry points.
#include <hip/hip_runtime.h>

#include <algorithm>
#include <cmath>
#include <cstdio>
#include <cstring>
#include <exception>
#include <map>
#include <mutex>
#include <set>
#include <string>
#include <vector>

#include "drain_live.h"
#include "drain_scan.h"
#include "pack.h"
#include "ssla_hip.h"
#include "weights_dir.h"

namespace ssla {

namespace {
thread_local std::string t_err;

std::mutex g_alloc_mu;
std::set<void*> g_state_bases;   // blocks allocated by ssla_hip_state_alloc
std::map<void*, size_t> g_state_bytes;   // their sizes: one allocation holds a block's state
std::set<void*> g_pred_bases;    // preds allocated by ssla_hip_preds_alloc
std::set<void*> g_clock_blocks;  // clock anchor blocks of ssla_hip_timing_alloc (4 words)
}  // namespace

void set_error(const std::string& msg) { t_err = msg; }

unsigned long long* timing_clock_sync(const HybridS2S3Config* cfg, int blk) {
    unsigned long long* c = cfg->kernel_start_clk[blk];
    std::lock_guard<std::mutex> lk(g_alloc_mu);
    return (c && cfg->kernel_end_clk[blk] == c + 1 && g_clock_blocks.count(c)) ? c + 2 : nullptr;
}

namespace {

#define API_HIP(call)                                                         \
    do {                                                                      \
        hipError_t e_ = (call);                                               \
        if (e_ != hipSuccess) {                                               \
            set_error(std::string(#call) + ": " + hipGetErrorString(e_));    \
            return SSLA_ERR_HIP;                                              \
        }                                                                     \
    } while (0)

// GPU layer li (0..3 = L4..L7): input / output widths.
constexpr int kIn[4] = {24, 48, 48, 96};
constexpr int kOut[4] = {48, 48, 96, 96};

// ---- device layouts of the fused layer weights ---------------------------
// qvgIn (A, 3*OUT, IN) -> (9, IN, 3*OUT); goW (A, D, D) -> (9, OUT_in, OUT_out);
// input_proj (OUT, IN) -> (IN, OUT).
struct PackedLayer {
    std::vector<float> qvg_dev;   // (9, IN, 3*OUT)
    std::vector<float> gow_dev;   // (9, OUT, OUT)
    std::vector<float> ip_dev;    // (IN, OUT) or empty
    std::vector<float> gamma, beta;
};

const NpzTensor& need(const std::map<std::string, NpzTensor>& W, const std::string& k,
                      std::vector<int64_t> shape) {
    const auto it = W.find(k);
    if (it == W.end()) throw std::runtime_error("weights.npz: missing " + k);
    const NpzTensor& t = it->second;
    std::vector<int64_t> s = t.shape;
    // 1x1 conv weights may carry trailing unit dims (C_out, C_in, 1, 1).
    while (s.size() > shape.size() && s.back() == 1) s.pop_back();
    if (s != shape) {
        std::string got, want;
        for (auto d : t.shape) got += std::to_string(d) + ",";
        for (auto d : shape) want += std::to_string(d) + ",";
        throw std::runtime_error("weights.npz: " + k + " has shape (" + got + ") expected (" + want + ")");
    }
    return t;
}

PackedLayer pack_layer(const std::map<std::string, NpzTensor>& W, const std::string& pre,
                       int IN, int D) {
    const FusedLayer F = fuse_layer(W, pre, IN, D);
    if (F.A != 9) throw std::runtime_error(pre + ": expected 9 patch positions (K=3)");
    PackedLayer L;
    L.gamma = F.gamma;
    L.beta = F.beta;
    if (!F.input_proj.empty()) {
        L.ip_dev.resize((size_t)IN * D);
        for (int o = 0; o < D; ++o)
            for (int i = 0; i < IN; ++i) L.ip_dev[(size_t)i * D + o] = F.input_proj[(size_t)o * IN + i];
    }
    L.qvg_dev.assign((size_t)9 * IN * 3 * D, 0.f);
    L.gow_dev.assign((size_t)9 * D * D, 0.f);
    for (int p = 0; p < 9; ++p) {
        for (int r = 0; r < 3 * D; ++r)
            for (int i = 0; i < IN; ++i)
                L.qvg_dev[((size_t)p * IN + i) * 3 * D + r] = F.qvgIn[((size_t)p * 3 * D + r) * IN + i];
        for (int o = 0; o < D; ++o)
            for (int i = 0; i < D; ++i)
                L.gow_dev[((size_t)p * D + i) * D + o] = F.goW[((size_t)p * D + o) * D + i];
    }
    return L;
}

// Head level 0, BatchNorm folded (hybrid_common.py:327-409):
// scale = bn_w / sqrt(bn_var + 1e-5); shift = bn_b - scale*mu;
// W' = W*scale[:,None]; b' = b_conv*scale + shift.  Stored (IN, OUT).
struct PackedHead {
    std::vector<float> cls_conv_W, cls_conv_b, cls_pred_W, cls_pred_b;
    std::vector<float> reg_conv_W, reg_conv_b, reg_pred_W, reg_pred_b;
    std::vector<float> obj_pred_W, obj_pred_b;
};

void fold_conv_bn(const std::map<std::string, NpzTensor>& W, const std::string& branch,
                  std::vector<float>& Wd, std::vector<float>& bd) {
    const int C = 96;
    const NpzTensor& cw = need(W, "head/" + branch + "/0/0/weight", {C, C});
    const NpzTensor& g = need(W, "head/" + branch + "/0/1/weight", {C});
    const NpzTensor& b = need(W, "head/" + branch + "/0/1/bias", {C});
    const NpzTensor& mu = need(W, "head/" + branch + "/0/1/running_mean", {C});
    const NpzTensor& var = need(W, "head/" + branch + "/0/1/running_var", {C});
    const auto cb = W.find("head/" + branch + "/0/0/bias");
    Wd.assign((size_t)C * C, 0.f);
    bd.assign(C, 0.f);
    for (int o = 0; o < C; ++o) {
        const float scale = g.data[o] / std::sqrt(var.data[o] + 1e-5f);
        const float shift = b.data[o] - scale * mu.data[o];
        for (int i = 0; i < C; ++i) Wd[(size_t)i * C + o] = cw.data[(size_t)o * C + i] * scale;
        const float bc = cb != W.end() ? cb->second.data.at(o) : 0.0f;
        bd[o] = bc * scale + shift;
    }
}

void transpose_pred(const NpzTensor& t, int rows, std::vector<float>& out) {
    const int C = 96;
    out.assign((size_t)C * rows, 0.f);
    for (int k = 0; k < rows; ++k)
        for (int i = 0; i < C; ++i) out[(size_t)i * rows + k] = t.data[(size_t)k * C + i];
}

PackedHead pack_head(const std::map<std::string, NpzTensor>& W, int n_cls) {
    PackedHead h;
    fold_conv_bn(W, "cls_convs", h.cls_conv_W, h.cls_conv_b);
    fold_conv_bn(W, "reg_convs", h.reg_conv_W, h.reg_conv_b);
    transpose_pred(need(W, "head/cls_preds/0/weight", {n_cls, 96}), n_cls, h.cls_pred_W);
    h.cls_pred_b = need(W, "head/cls_preds/0/bias", {n_cls}).data;
    transpose_pred(need(W, "head/reg_preds/0/weight", {4, 96}), 4, h.reg_pred_W);
    h.reg_pred_b = need(W, "head/reg_preds/0/bias", {4}).data;
    transpose_pred(need(W, "head/obj_preds/0/weight", {1, 96}), 1, h.obj_pred_W);
    h.obj_pred_b = need(W, "head/obj_preds/0/bias", {1}).data;
    return h;
}

// Raw head row [reg4, obj, cls2] of one 96-channel feature in fp32, the
// device head's arithmetic (1x1 convs with BN folded, SiLU, three preds).
void head_row_host(const PackedHead& h, const float* x, float* out) {
    const int C = 96;
    float cf[C], rf[C];
    for (int o = 0; o < C; ++o) {
        float a = h.cls_conv_b[o], r = h.reg_conv_b[o];
        for (int i = 0; i < C; ++i) {
            a += x[i] * h.cls_conv_W[(size_t)i * C + o];
            r += x[i] * h.reg_conv_W[(size_t)i * C + o];
        }
        cf[o] = a / (1.0f + std::exp(-a));
        rf[o] = r / (1.0f + std::exp(-r));
    }
    auto pred = [&](const float* f, const std::vector<float>& Wt, const std::vector<float>& b,
                    int rows, float* dst) {
        for (int k = 0; k < rows; ++k) {
            float a = b[k];
            for (int i = 0; i < C; ++i) a += f[i] * Wt[(size_t)i * rows + k];
            dst[k] = a;
        }
    };
    pred(rf, h.reg_pred_W, h.reg_pred_b, 4, out);
    pred(rf, h.obj_pred_W, h.obj_pred_b, 1, out + 4);
    pred(cf, h.cls_pred_W, h.cls_pred_b, 2, out + 5);
}

}  // namespace
}  // namespace ssla

using namespace ssla;

struct SslaHipModel {
    void* dev = nullptr;
    LayerWeightsS2S3 layers[4] = {};
    const float* head[10] = {};   // cls_conv W,b, cls_pred W,b, reg_conv W,b, reg_pred W,b, obj W,b
    SslaHipModelInfo info = {};
    PackedHead host_head;         // host copy for ssla_hip_model_head_row
};

extern "C" {

const char* ssla_hip_last_error(void) { return t_err.c_str(); }

int ssla_hip_abi_layout(long long* out, int cap) {
    if (!out || cap < 7) {
        set_error("ssla_hip_abi_layout: need 7 slots");
        return SSLA_ERR_ARG;
    }
    out[0] = sizeof(HybridInputRec);
    out[1] = sizeof(HybridS2S3Config);
    out[2] = offsetof(HybridS2S3Config, preds);
    out[3] = sizeof(HybridS2S3OutputSlot);
    out[4] = sizeof(GpuTimingSlot);
    out[5] = sizeof(HybridStrip);
    out[6] = sizeof(LayerWeightsS2S3);
    return SSLA_OK;
}

int ssla_hip_malloc_device(size_t nbytes, void** out) {
    if (!out) { set_error("null out"); return SSLA_ERR_ARG; }
    *out = nullptr;
    API_HIP(hipMalloc(out, nbytes ? nbytes : 1));
    return SSLA_OK;
}

int ssla_hip_malloc_host(size_t nbytes, void** out) {
    if (!out) { set_error("null out"); return SSLA_ERR_ARG; }
    *out = nullptr;
    API_HIP(hipHostMalloc(out, nbytes ? nbytes : 1, hipHostMallocCoherent | hipHostMallocMapped));
    return SSLA_OK;
}

int ssla_hip_free_device(void* p) {
    if (p) API_HIP(hipFree(p));
    return SSLA_OK;
}

int ssla_hip_free_host(void* p) {
    if (p) API_HIP(hipHostFree(p));
    return SSLA_OK;
}

int ssla_hip_memcpy(void* dst, const void* src, size_t nbytes) {
    if (!nbytes) return SSLA_OK;
    if (!dst || !src) { set_error("null pointer"); return SSLA_ERR_ARG; }
    API_HIP(hipMemcpy(dst, src, nbytes, hipMemcpyDefault));
    return SSLA_OK;
}

int ssla_hip_memset(void* dst, int value, size_t nbytes) {
    if (!nbytes) return SSLA_OK;
    if (!dst) { set_error("null pointer"); return SSLA_ERR_ARG; }
    API_HIP(hipMemsetAsync(dst, value, nbytes, nullptr));
    API_HIP(hipStreamSynchronize(nullptr));
    return SSLA_OK;
}

int ssla_hip_device_synchronize(void) {
    API_HIP(hipDeviceSynchronize());
    return SSLA_OK;
}

int ssla_hip_stream_create(void** out) {
    if (!out) { set_error("null out"); return SSLA_ERR_ARG; }
    *out = nullptr;
    hipStream_t s = nullptr;
    API_HIP(hipStreamCreateWithFlags(&s, hipStreamNonBlocking));
    *out = s;
    return SSLA_OK;
}

int ssla_hip_stream_destroy(void* stream) {
    if (!stream) return SSLA_OK;
    API_HIP(hipStreamDestroy(static_cast<hipStream_t>(stream)));
    return SSLA_OK;
}

int ssla_hip_stream_synchronize(void* stream) {
    API_HIP(hipStreamSynchronize(static_cast<hipStream_t>(stream)));
    return SSLA_OK;
}

long long ssla_hip_npz_read(const char* dir, const char* key, float* out, long long cap,
                            long long* shape, int* ndim) {
    if (!dir || !key) { set_error("null argument"); return SSLA_ERR_ARG; }
    try {
        const auto W = read_npz(dir);
        const auto it = W.find(key);
        if (it == W.end()) { set_error(std::string("no tensor ") + key); return SSLA_ERR_FORMAT; }
        const NpzTensor& t = it->second;
        const long long n = (long long)t.data.size();
        if (out) {
            if (cap < n) { set_error("output buffer too small"); return SSLA_ERR_ARG; }
            std::memcpy(out, t.data.data(), sizeof(float) * (size_t)n);
        }
        if (ndim) *ndim = (int)t.shape.size();
        if (shape)
            for (size_t i = 0; i < t.shape.size() && i < 4; ++i) shape[i] = t.shape[i];
        return n;
    } catch (const std::exception& e) {
        set_error(e.what());
        return SSLA_ERR_IO;
    }
}

int ssla_hip_meta_read(const char* dir, int* out) {
    if (!dir || !out) { set_error("null argument"); return SSLA_ERR_ARG; }
    try {
        const ModelMeta m = read_meta(dir);
        out[0] = m.height;
        out[1] = m.width;
        out[2] = m.num_classes;
        out[3] = m.ssla_tdrop_window;
        return SSLA_OK;
    } catch (const std::exception& e) {
        set_error(e.what());
        return SSLA_ERR_IO;
    }
}

int ssla_hip_model_load(const char* dir, SslaHipModel** out) {
    if (!dir || !out) { set_error("null argument"); return SSLA_ERR_ARG; }
    *out = nullptr;
    ModelMeta meta;
    std::map<std::string, NpzTensor> W;
    try {
        meta = read_meta(dir);
        W = read_npz(dir);
    } catch (const std::exception& e) {
        set_error(e.what());
        return SSLA_ERR_IO;
    }
    SslaHipModelInfo info{};
    std::vector<PackedLayer> layers;
    PackedHead head;
    try {
        if (meta.model != "ssla_s_yolox_det")
            throw std::runtime_error("meta.json: model '" + meta.model + "' is not ssla_s_yolox_det");
        if (meta.height <= 0 || meta.width <= 0 || meta.height % 8 || meta.width % 8)
            throw std::runtime_error("meta.json: height and width must be positive multiples of 8");
        info.height = meta.height;
        info.width = meta.width;
        info.num_classes = meta.num_classes > 0 ? meta.num_classes : 2;
        info.tdrop_window = meta.ssla_tdrop_window > 0 ? meta.ssla_tdrop_window : 4;
        info.H2 = meta.height >> 2;
        info.W2 = meta.width >> 2;
        info.H3 = info.H2 >> 1;
        info.W3 = info.W2 >> 1;
        // SSLA layer indices, sorted (ssla_kernels.cpp:178-198); the GPU
        // path takes the last four (stages 2 and 3).
        const std::vector<int> idx = ssla_layer_indices(W);
        if (idx.size() != 8)
            throw std::runtime_error("weights.npz: expected 8 SSLA layers, found " + std::to_string(idx.size()));
        for (int li = 0; li < 4; ++li)
            layers.push_back(pack_layer(W, "layers/" + std::to_string(idx[4 + li]), kIn[li], kOut[li]));
        info.has_head = W.count("head/cls_convs/0/0/weight") ? 1 : 0;
        if (info.has_head) {
            if (info.num_classes != 2)
                throw std::runtime_error("the device head writes [reg4, obj, cls2]: num_classes must be 2");
            head = pack_head(W, info.num_classes);
        }
    } catch (const std::exception& e) {
        set_error(e.what());
        return SSLA_ERR_FORMAT;
    }
    std::vector<const std::vector<float>*> bufs;
    for (auto& L : layers) {
        bufs.push_back(&L.qvg_dev);
        bufs.push_back(&L.gow_dev);
        bufs.push_back(&L.ip_dev);
        bufs.push_back(&L.gamma);
        bufs.push_back(&L.beta);
    }
    const std::vector<float>* hb[10] = {&head.cls_conv_W, &head.cls_conv_b, &head.cls_pred_W,
                                        &head.cls_pred_b, &head.reg_conv_W, &head.reg_conv_b,
                                        &head.reg_pred_W, &head.reg_pred_b, &head.obj_pred_W,
                                        &head.obj_pred_b};
    for (auto* b : hb) bufs.push_back(b);
    size_t total = 0;
    for (auto* b : bufs) total += (b->size() * sizeof(float) + 255) & ~size_t(255);
    SslaHipModel* m = new SslaHipModel();
    m->info = info;
    if (hipMalloc(&m->dev, total) != hipSuccess) {
        set_error("hipMalloc of model weights failed");
        delete m;
        return SSLA_ERR_HIP;
    }
    char* p = static_cast<char*>(m->dev);
    std::vector<const float*> ptrs;
    for (auto* b : bufs) {
        if (b->empty()) { ptrs.push_back(nullptr); continue; }
        if (hipMemcpy(p, b->data(), b->size() * sizeof(float), hipMemcpyHostToDevice) != hipSuccess) {
            set_error("hipMemcpy of model weights failed");
            (void)hipFree(m->dev);
            delete m;
            return SSLA_ERR_HIP;
        }
        ptrs.push_back(reinterpret_cast<const float*>(p));
        p += (b->size() * sizeof(float) + 255) & ~size_t(255);
    }
    for (int li = 0; li < 4; ++li) {
        m->layers[li].qvgIn = ptrs[li * 5 + 0];
        m->layers[li].goW = ptrs[li * 5 + 1];
        m->layers[li].input_proj = ptrs[li * 5 + 2];
        m->layers[li].ln_gamma = ptrs[li * 5 + 3];
        m->layers[li].ln_beta = ptrs[li * 5 + 4];
    }
    for (int k = 0; k < 10; ++k) m->head[k] = ptrs[20 + k];
    m->host_head = std::move(head);
    *out = m;
    return SSLA_OK;
}

int ssla_hip_model_head_row(const SslaHipModel* m, const float* feat, float* out) {
    if (!m || !feat || !out) { set_error("model_head_row: null argument"); return SSLA_ERR_ARG; }
    if (!m->info.has_head) { set_error("model_head_row: the model has no head"); return SSLA_ERR_STATE; }
    head_row_host(m->host_head, feat, out);
    return SSLA_OK;
}

int ssla_hip_head_row(const char* weights_dir, const float* feat, float* out) {
    if (!weights_dir || !feat || !out) { set_error("head_row: null argument"); return SSLA_ERR_ARG; }
    std::map<std::string, NpzTensor> W;
    try {
        W = read_npz(weights_dir);
    } catch (const std::exception& e) {
        set_error(e.what());
        return SSLA_ERR_IO;
    }
    if (!W.count("head/cls_convs/0/0/weight")) {
        set_error("head_row: weights.npz has no head");
        return SSLA_ERR_STATE;
    }
    try {
        head_row_host(pack_head(W, 2), feat, out);
    } catch (const std::exception& e) {
        set_error(e.what());
        return SSLA_ERR_FORMAT;
    }
    return SSLA_OK;
}

int ssla_hip_model_info(const SslaHipModel* m, SslaHipModelInfo* out) {
    if (!m || !out) { set_error("null argument"); return SSLA_ERR_ARG; }
    *out = m->info;
    return SSLA_OK;
}

void ssla_hip_model_free(SslaHipModel* m) {
    if (!m) return;
    if (m->dev) (void)hipFree(m->dev);
    delete m;
}

int ssla_hip_config_bind(const SslaHipModel* m, int n_blocks, HybridS2S3Config* cfg) {
    if (!m || !cfg) { set_error("null argument"); return SSLA_ERR_ARG; }
    if (n_blocks < 1 || n_blocks > SSLA_MAX_BLOCKS) { set_error("n_blocks must be in [1, 16]"); return SSLA_ERR_ARG; }
    std::memset(cfg, 0, sizeof(*cfg));
    const SslaHipModelInfo& I = m->info;
    cfg->H2 = I.H2; cfg->W2 = I.W2; cfg->H3 = I.H3; cfg->W3 = I.W3;
    cfg->tdrop_window = I.tdrop_window;
    cfg->head_out_dim = SSLA_HEAD_OUT;
    cfg->n_blocks = n_blocks;
    for (int b = 0; b < n_blocks; ++b) {
        HybridStrip& s = cfg->strip[b];
        s.owned_lo = 0; s.owned_hi = I.W2; s.owned_y_lo = 0; s.owned_y_hi = I.H2;
        s.s3_owned_lo = 0; s.s3_owned_hi = I.W3; s.s3_owned_y_lo = 0; s.s3_owned_y_hi = I.H3;
        for (int li = 0; li < 4; ++li) cfg->layers[b][li] = m->layers[li];
    }
    if (I.has_head) {
        cfg->head_cls_conv_W = m->head[0]; cfg->head_cls_conv_b = m->head[1];
        cfg->head_cls_pred_W = m->head[2]; cfg->head_cls_pred_b = m->head[3];
        cfg->head_reg_conv_W = m->head[4]; cfg->head_reg_conv_b = m->head[5];
        cfg->head_reg_pred_W = m->head[6]; cfg->head_reg_pred_b = m->head[7];
        cfg->head_obj_pred_W = m->head[8]; cfg->head_obj_pred_b = m->head[9];
    }
    return SSLA_OK;
}

int ssla_hip_state_alloc(HybridS2S3Config* cfg, int blk) {
    if (!cfg || blk < 0 || blk >= SSLA_MAX_BLOCKS) { set_error("bad block"); return SSLA_ERR_ARG; }
    if (cfg->H2 <= 0 || cfg->W2 <= 0) { set_error("config has no grid"); return SSLA_ERR_STATE; }
    {
        std::lock_guard<std::mutex> lk(g_alloc_mu);
        if (cfg->hidden[blk][0] && g_state_bases.count(cfg->hidden[blk][0])) {
            set_error("state of this block is already allocated (ssla_hip_state_free first)");
            return SSLA_ERR_STATE;
        }
    }
    const size_t c2 = (size_t)cfg->H2 * cfg->W2, c3 = (size_t)cfg->H3 * cfg->W3;
    const size_t sz[6] = {c2 * 48 * 4, c2 * 48 * 4, c3 * 96 * 4, c3 * 96 * 4, c2, c3};
    size_t total = 0;
    for (size_t s : sz) total += (s + 255) & ~size_t(255);
    void* base = nullptr;
    API_HIP(hipMalloc(&base, total));
    hipError_t e = hipMemset(base, 0, total);
    if (e == hipSuccess) e = hipStreamSynchronize(nullptr);
    if (e != hipSuccess) {
        set_error(std::string("state_alloc: clearing the state: ") + hipGetErrorString(e));
        (void)hipFree(base);
        return SSLA_ERR_HIP;
    }
    char* p = static_cast<char*>(base);
    void* parts[6];
    for (int i = 0; i < 6; ++i) {
        parts[i] = p;
        p += (sz[i] + 255) & ~size_t(255);
    }
    for (int li = 0; li < 4; ++li) cfg->hidden[blk][li] = static_cast<float*>(parts[li]);
    cfg->tdrop_s2[blk] = static_cast<unsigned char*>(parts[4]);
    cfg->tdrop_s3[blk] = static_cast<unsigned char*>(parts[5]);
    std::lock_guard<std::mutex> lk(g_alloc_mu);
    g_state_bases.insert(base);
    g_state_bytes[base] = total;
    return SSLA_OK;
}

int ssla_hip_state_reset(const HybridS2S3Config* cfg, int blk) {
    if (!cfg || blk < 0 || blk >= SSLA_MAX_BLOCKS) { set_error("bad block"); return SSLA_ERR_ARG; }
    const size_t c2 = (size_t)cfg->H2 * cfg->W2, c3 = (size_t)cfg->H3 * cfg->W3;
    const size_t sz[4] = {c2 * 48 * 4, c2 * 48 * 4, c3 * 96 * 4, c3 * 96 * 4};
    for (int li = 0; li < 4; ++li) {
        if (!cfg->hidden[blk][li]) { set_error("hidden state not allocated"); return SSLA_ERR_STATE; }
        API_HIP(hipMemset(cfg->hidden[blk][li], 0, sz[li]));
    }
    if (!cfg->tdrop_s2[blk] || !cfg->tdrop_s3[blk]) { set_error("tdrop counters not allocated"); return SSLA_ERR_STATE; }
    API_HIP(hipMemset(cfg->tdrop_s2[blk], 0, c2));
    API_HIP(hipMemset(cfg->tdrop_s3[blk], 0, c3));
    API_HIP(hipStreamSynchronize(nullptr));
    return SSLA_OK;
}

int ssla_hip_state_reset_async(const HybridS2S3Config* cfg, int blk, void* stream) {
    if (!cfg || blk < 0 || blk >= SSLA_MAX_BLOCKS) { set_error("bad block"); return SSLA_ERR_ARG; }
    hipStream_t st = static_cast<hipStream_t>(stream);
    {
        // state from ssla_hip_state_alloc: hidden layers and counters are
        // one allocation, cleared by one fill
        size_t bytes = 0;
        {
            std::lock_guard<std::mutex> lk(g_alloc_mu);
            const auto it = g_state_bytes.find(cfg->hidden[blk][0]);
            if (it != g_state_bytes.end()) bytes = it->second;
        }
        if (bytes) return zero_async(cfg->hidden[blk][0], bytes, st);
    }
    const size_t c2 = (size_t)cfg->H2 * cfg->W2, c3 = (size_t)cfg->H3 * cfg->W3;
    const size_t sz[4] = {c2 * 48 * 4, c2 * 48 * 4, c3 * 96 * 4, c3 * 96 * 4};
    for (int li = 0; li < 4; ++li) {
        if (!cfg->hidden[blk][li]) { set_error("hidden state not allocated"); return SSLA_ERR_STATE; }
        API_HIP(hipMemsetAsync(cfg->hidden[blk][li], 0, sz[li], st));
    }
    if (!cfg->tdrop_s2[blk] || !cfg->tdrop_s3[blk]) { set_error("tdrop counters not allocated"); return SSLA_ERR_STATE; }
    API_HIP(hipMemsetAsync(cfg->tdrop_s2[blk], 0, c2, st));
    API_HIP(hipMemsetAsync(cfg->tdrop_s3[blk], 0, c3, st));
    return SSLA_OK;
}

void ssla_hip_state_free(HybridS2S3Config* cfg, int blk) {
    if (!cfg || blk < 0 || blk >= SSLA_MAX_BLOCKS) return;
    void* base = cfg->hidden[blk][0];
    {
        std::lock_guard<std::mutex> lk(g_alloc_mu);
        if (!base || !g_state_bases.erase(base)) return;
        g_state_bytes.erase(base);
    }
    (void)hipFree(base);
    for (int li = 0; li < 4; ++li) cfg->hidden[blk][li] = nullptr;
    cfg->tdrop_s2[blk] = nullptr;
    cfg->tdrop_s3[blk] = nullptr;
}

int ssla_hip_preds_alloc(HybridS2S3Config* cfg, int blk) {
    if (!cfg || blk < 0 || blk >= SSLA_MAX_BLOCKS) { set_error("bad block"); return SSLA_ERR_ARG; }
    const HybridStrip& s = cfg->strip[blk];
    const int w = s.s3_owned_hi - s.s3_owned_lo, h = s.s3_owned_y_hi - s.s3_owned_y_lo;
    if (w <= 0 || h <= 0) { set_error("block has an empty s3 owned box"); return SSLA_ERR_STATE; }
    {
        std::lock_guard<std::mutex> lk(g_alloc_mu);
        if (cfg->preds[blk] && g_pred_bases.count(cfg->preds[blk])) {
            set_error("predictions of this block are already allocated (ssla_hip_preds_free first)");
            return SSLA_ERR_STATE;
        }
    }
    const size_t cells = (size_t)w * h;
    const size_t pb = (cells * 7 * 4 + 255) & ~size_t(255);
    void* base = nullptr;
    API_HIP(hipHostMalloc(&base, pb + cells * 4, hipHostMallocCoherent | hipHostMallocMapped));
    std::memset(base, 0, pb + cells * 4);
    cfg->preds[blk] = static_cast<float*>(base);
    cfg->version[blk] = reinterpret_cast<unsigned int*>(static_cast<char*>(base) + pb);
    std::lock_guard<std::mutex> lk(g_alloc_mu);
    g_pred_bases.insert(base);
    return SSLA_OK;
}

void ssla_hip_preds_free(HybridS2S3Config* cfg, int blk) {
    if (!cfg || blk < 0 || blk >= SSLA_MAX_BLOCKS) return;
    void* base = cfg->preds[blk];
    {
        std::lock_guard<std::mutex> lk(g_alloc_mu);
        if (!base || !g_pred_bases.erase(base)) return;
    }
    (void)hipHostFree(base);
    cfg->preds[blk] = nullptr;
    cfg->version[blk] = nullptr;
}

int ssla_hip_drain_n_ex(const HybridS2S3Config* cfg, const HybridInputRec* const* rings,
                        const int* ns, HybridS2S3OutputSlot* const* outs,
                        const SslaHipDrainOpts* opts) {
    if (!cfg || !rings || !ns) { set_error("null argument"); return SSLA_ERR_ARG; }
    hipStream_t st = opts ? static_cast<hipStream_t>(opts->stream) : nullptr;
    const bool sync = opts ? opts->sync != 0 : true;
    float* phase_ms = opts ? opts->phase_ms : nullptr;
    const int batch = opts ? opts->batch : 0;
    double* bph = opts ? opts->batch_phase_us : nullptr;
    const int group = opts ? opts->group : 0;
    if (batch != 0) {
        if (phase_ms) { set_error("phase_ms is only measured by the whole-ring drain"); return SSLA_ERR_ARG; }
        if (group > 1)
            return batch_drain_group(cfg, rings, ns, outs, opts->head_outs, batch, group, st, bph);
        return batch_drain(cfg, rings, ns, outs, opts->head_outs, nullptr, batch, st, sync, bph);
    }
    if (group > 1) { set_error("group is a batch-mode option"); return SSLA_ERR_ARG; }
    if (bph) { set_error("batch_phase_us is only measured by the batch-mode drain"); return SSLA_ERR_ARG; }
    return scan_drain(cfg, rings, ns, outs, opts ? opts->head_outs : nullptr, st, sync, phase_ms,
                      opts ? opts->phase_mask : 0ull);
}

int ssla_hip_drain_batch_noalloc(const HybridS2S3Config* cfg, const HybridInputRec* const* rings,
                                 const int* ns, HybridS2S3OutputSlot* const* outs,
                                 float* const* head_outs, int batch, void* stream, int sync) {
    if (!cfg || !rings || !ns) { set_error("null argument"); return SSLA_ERR_ARG; }
    hipStream_t st = static_cast<hipStream_t>(stream);
    const int rc = batch_drain_noalloc(cfg, rings, ns, outs, head_outs, batch, st);
    if (rc) return rc;
    if (sync) API_HIP(hipStreamSynchronize(st));
    return SSLA_OK;
}

int ssla_hip_drain_reserve(const HybridS2S3Config* cfg, int max_records) {
    return drain_reserve(cfg, max_records);
}

int ssla_hip_drain_n(const HybridS2S3Config* cfg, const HybridInputRec* const* rings,
                     const int* ns, HybridS2S3OutputSlot* const* outs,
                     unsigned long long* const* batch_clks) {
    if (!cfg || !rings || !ns) { set_error("null argument"); return SSLA_ERR_ARG; }
    if (batch_clks) {
        // the reference's drain_n batching: 8 records per batch, clock pairs
        return batch_drain(cfg, rings, ns, outs, nullptr, batch_clks, 8, nullptr, true, nullptr);
    }
    SslaHipDrainOpts o{};
    o.sync = 1;
    return ssla_hip_drain_n_ex(cfg, rings, ns, outs, &o);
}

int ssla_hip_wall_clock_khz(int* out) {
    if (!out) { set_error("null argument"); return SSLA_ERR_ARG; }
    API_HIP(hipDeviceGetAttribute(out, hipDeviceAttributeWallClockRate, 0));
    return SSLA_OK;
}

int ssla_hip_timing_alloc(HybridS2S3Config* cfg, int blk, unsigned int capacity) {
    if (!cfg || blk < 0 || blk >= SSLA_MAX_BLOCKS) { set_error("bad block"); return SSLA_ERR_ARG; }
    if (capacity == 0 || (capacity & (capacity - 1))) { set_error("capacity must be a power of two"); return SSLA_ERR_ARG; }
    if (cfg->timing_mask && cfg->timing_mask != capacity - 1) {
        set_error("all blocks share one timing capacity");
        return SSLA_ERR_ARG;
    }
    {
        std::lock_guard<std::mutex> lk(g_alloc_mu);
        if (cfg->timing[blk] && g_state_bases.count(cfg->timing[blk])) {
            set_error("timing of this block is already allocated (ssla_hip_timing_free first)");
            return SSLA_ERR_STATE;
        }
    }
    void* t = nullptr;
    API_HIP(hipMalloc(&t, sizeof(GpuTimingSlot) * (size_t)capacity));
    hipError_t e = hipMemset(t, 0, sizeof(GpuTimingSlot) * (size_t)capacity);
    if (e == hipSuccess) e = hipStreamSynchronize(nullptr);
    if (e != hipSuccess) {
        set_error(std::string("timing_alloc: clearing the ring: ") + hipGetErrorString(e));
        (void)hipFree(t);
        return SSLA_ERR_HIP;
    }
    // [start, end, ping, pong] (the last two: the live kernels' clock handshake)
    void* clk = nullptr;
    if (hipHostMalloc(&clk, 32, hipHostMallocCoherent | hipHostMallocMapped) != hipSuccess) {
        (void)hipFree(t);
        set_error("hipHostMalloc of clock anchors failed");
        return SSLA_ERR_HIP;
    }
    std::memset(clk, 0, 32);
    cfg->timing[blk] = static_cast<GpuTimingSlot*>(t);
    cfg->timing_mask = capacity - 1;
    cfg->kernel_start_clk[blk] = static_cast<unsigned long long*>(clk);
    cfg->kernel_end_clk[blk] = static_cast<unsigned long long*>(clk) + 1;
    std::lock_guard<std::mutex> lk(g_alloc_mu);
    g_state_bases.insert(t);
    g_pred_bases.insert(clk);
    g_clock_blocks.insert(clk);
    return SSLA_OK;
}

void ssla_hip_timing_free(HybridS2S3Config* cfg, int blk) {
    if (!cfg || blk < 0 || blk >= SSLA_MAX_BLOCKS) return;
    void* t = cfg->timing[blk];
    void* clk = cfg->kernel_start_clk[blk];
    std::lock_guard<std::mutex> lk(g_alloc_mu);
    if (t && g_state_bases.erase(t)) {
        (void)hipFree(t);
        cfg->timing[blk] = nullptr;
    }
    g_clock_blocks.erase(clk);
    if (clk && g_pred_bases.erase(clk)) {
        (void)hipHostFree(clk);
        cfg->kernel_start_clk[blk] = nullptr;
        cfg->kernel_end_clk[blk] = nullptr;
    }
}

int ssla_hip_persistent_start(const HybridS2S3Config* cfg, HybridInputRec* const* rings,
                              unsigned long long ring_mask, unsigned long long* const* tails,
                              int* stop_flag, unsigned long long* const* events_done,
                              unsigned int spin_ns, const SslaHipLiveOpts* opts, SslaHipLive** out) {
    if (!cfg || !rings || !tails || !out) { set_error("null argument"); return SSLA_ERR_ARG; }
    const int max_batch = (opts && opts->max_batch) ? opts->max_batch : kLiveBatchMax;
    const unsigned idle = (opts && opts->idle_timeout_ms) ? opts->idle_timeout_ms : 30000u;
    const int group = opts ? opts->group : 0;
    const int stages = (opts && opts->stages) ? opts->stages : 1;
    LiveSession* s = nullptr;
    const int rc = live_start(cfg, rings, ring_mask, tails, stop_flag, events_done, spin_ns,
                              max_batch, idle, opts ? opts->phase_us : nullptr, group, stages, &s);
    *out = reinterpret_cast<SslaHipLive*>(s);
    return rc;
}

int ssla_hip_persistent_start2(const HybridS2S3Config* cfg, HybridInputRec* ring0,
                               HybridInputRec* ring1, unsigned long long ring_mask,
                               unsigned long long* tail0, unsigned long long* tail1,
                               int* stop_flag, unsigned long long* events_done0,
                               unsigned long long* events_done1, unsigned int spin_ns,
                               SslaHipLive** out) {
    if (!cfg || cfg->n_blocks != 2) {
        set_error("the two-ring persistent drain needs cfg->n_blocks == 2");
        return SSLA_ERR_ARG;
    }
    HybridInputRec* rings[2] = {ring0, ring1};
    unsigned long long* tails[2] = {tail0, tail1};
    unsigned long long* dones[2] = {events_done0, events_done1};
    SslaHipLiveOpts opts{};
    opts.max_batch = 8;
    return ssla_hip_persistent_start(cfg, rings, ring_mask, tails, stop_flag, dones, spin_ns,
                                     &opts, out);
}

int ssla_hip_persistent_wait(SslaHipLive* h, int timeout_ms, int* status) {
    return live_wait(reinterpret_cast<LiveSession*>(h), timeout_ms, status);
}

int ssla_hip_drain_n2(const HybridS2S3Config* cfg, const HybridInputRec* ring0,
                      const HybridInputRec* ring1, int n0, int n1,
                      HybridS2S3OutputSlot* out0, HybridS2S3OutputSlot* out1) {
    if (!cfg || cfg->n_blocks != 2) { set_error("the two-ring drain needs cfg->n_blocks == 2"); return SSLA_ERR_ARG; }
    const HybridInputRec* rings[2] = {ring0, ring1};
    const int ns[2] = {n0, n1};
    HybridS2S3OutputSlot* outs[2] = {out0, out1};
    return ssla_hip_drain_n(cfg, rings, ns, outs, nullptr);
}

}  // extern "C"
