// stage01.cpp -- see stage01.h.
#include "stage01.h"

#include <algorithm>
#include <cmath>
#include <cstring>
#include <stdexcept>

namespace ssla {
namespace {

inline float sigmoid(float x) { return 1.0f / (1.0f + std::exp(-x)); }

// One SSLA layer for one event at (x, y) on an (Hl, Wl) grid.  Patch cells
// are visited in the reference's order: the fixed delta 8..0 table for
// interior events, the dy/dx walk on the border (ssla_kernels.cpp:343-369).
// Weights are input-major (T.qvg (A, IN, 3*OUT), T.go (A, OUT, OUT) with
// T.go[p][i][o], T.ip (IN, OUT)) so every inner loop runs over contiguous
// output channels and vectorises.
template <int IN, int OUT>
void layer(const TLayer& T, float* H, int x, int y, int Hl, int Wl, const float* in, float* out,
           bool full) {
    constexpr int NC = 3 * OUT;
    alignas(32) float acc[OUT] = {};
    alignas(32) float res[OUT];
    if (full) {
        if (!T.ip.empty()) {
            for (int o = 0; o < OUT; ++o) res[o] = 0.f;
            for (int i = 0; i < IN; ++i) {
                const float xi = in[i];
                const float* w = T.ip.data() + (size_t)i * OUT;
                for (int o = 0; o < OUT; ++o) res[o] += xi * w[o];
            }
        } else {
            for (int o = 0; o < OUT; ++o) res[o] = in[o];
        }
    }
    auto patch = [&](int cell, int p) {
        const float* Wp = T.qvg.data() + (size_t)p * IN * NC;
        float* h = H + (size_t)cell * OUT;
        alignas(32) float r[NC];
        if (!full) {
            // state only: the v and g columns
            for (int c = OUT; c < NC; ++c) r[c] = 0.f;
            for (int i = 0; i < IN; ++i) {
                const float xi = in[i];
                const float* w = Wp + (size_t)i * NC;
                for (int c = OUT; c < NC; ++c) r[c] += xi * w[c];
            }
            for (int c = 0; c < OUT; ++c) h[c] = sigmoid(r[2 * OUT + c]) * h[c] + r[OUT + c];
            return;
        }
        for (int c = 0; c < NC; ++c) r[c] = 0.f;
        for (int i = 0; i < IN; ++i) {
            const float xi = in[i];
            const float* w = Wp + (size_t)i * NC;
            for (int c = 0; c < NC; ++c) r[c] += xi * w[c];
        }
        alignas(32) float qh[OUT];
        for (int c = 0; c < OUT; ++c) {
            const float hc = sigmoid(r[2 * OUT + c]) * h[c] + r[OUT + c];
            h[c] = hc;
            qh[c] = r[c] * hc;
        }
        const float* G = T.go.data() + (size_t)p * OUT * OUT;
        for (int i = 0; i < OUT; ++i) {
            const float qi = qh[i];
            const float* w = G + (size_t)i * OUT;
            for (int o = 0; o < OUT; ++o) acc[o] += qi * w[o];
        }
    };
    const int base = y * Wl + x;
    if (T.A == 1) {
        patch(base, 0);
    } else if (x > 0 && x + 1 < Wl && y > 0 && y + 1 < Hl) {
        const int offs[9] = {-Wl - 1, -Wl, -Wl + 1, -1, 0, 1, Wl - 1, Wl, Wl + 1};
        for (int k = 0; k < 9; ++k) patch(base + offs[k], 8 - k);
    } else {
        for (int dy = -1; dy <= 1; ++dy) {
            const int py = y + dy;
            if (py < 0 || py >= Hl) continue;
            for (int dx = -1; dx <= 1; ++dx) {
                const int px = x + dx;
                if (px < 0 || px >= Wl) continue;
                patch(py * Wl + px, (1 - dy) * 3 + (1 - dx));
            }
        }
    }
    if (!full) return;
    double sum = 0.0;
    for (int o = 0; o < OUT; ++o) {
        acc[o] += res[o];
        sum += (double)acc[o];
    }
    const double mean = sum / OUT;
    double var = 0.0;
    for (int o = 0; o < OUT; ++o) {
        const double d = (double)acc[o] - mean;
        var += d * d;
    }
    var /= OUT;
    const double inv = 1.0 / std::sqrt(var + 1e-5);
    for (int o = 0; o < OUT; ++o)
        out[o] = (float)(((double)acc[o] - mean) * inv * (double)T.gamma[o] + (double)T.beta[o]);
}

// Input-major copies of a fused layer (see layer()).
TLayer transpose_layer(const FusedLayer& L) {
    TLayer T;
    const int A = L.A, IN = L.in_dim, D = L.out_dim, NC = 3 * D;
    T.A = A;
    T.qvg.resize((size_t)A * IN * NC);
    T.go.resize((size_t)A * D * D);
    for (int p = 0; p < A; ++p) {
        for (int r = 0; r < NC; ++r)
            for (int i = 0; i < IN; ++i)
                T.qvg[((size_t)p * IN + i) * NC + r] = L.qvgIn[((size_t)p * NC + r) * IN + i];
        for (int o = 0; o < D; ++o)
            for (int i = 0; i < D; ++i)
                T.go[((size_t)p * D + i) * D + o] = L.goW[((size_t)p * D + o) * D + i];
    }
    if (!L.input_proj.empty()) {
        T.ip.resize((size_t)IN * D);
        for (int o = 0; o < D; ++o)
            for (int i = 0; i < IN; ++i) T.ip[(size_t)i * D + o] = L.input_proj[(size_t)o * IN + i];
    }
    T.gamma = L.gamma;
    T.beta = L.beta;
    return T;
}

}  // namespace

Stage01::Stage01(const std::string& dir) {
    const ModelMeta meta = read_meta(dir);
    if (meta.model != "ssla_s_yolox_det")
        throw std::runtime_error("meta.json: model '" + meta.model + "' is not ssla_s_yolox_det");
    if (meta.height <= 0 || meta.width <= 0 || meta.height % 8 || meta.width % 8)
        throw std::runtime_error("meta.json: height and width must be positive multiples of 8");
    H_ = meta.height;
    W_ = meta.width;
    if (meta.ssla_tdrop_window > 0) window_ = meta.ssla_tdrop_window;
    const auto Wt = read_npz(dir);
    const std::vector<int> idx = ssla_layer_indices(Wt);
    if (idx.size() != 8) throw std::runtime_error("weights.npz: expected 8 SSLA layers");
    const int io[4][2] = {{2, 12}, {12, 12}, {12, 24}, {24, 24}};
    for (int l = 0; l < 4; ++l) {
        const FusedLayer F = fuse_layer(Wt, "layers/" + std::to_string(idx[l]), io[l][0], io[l][1]);
        if ((l == 0) != (F.A == 1))
            throw std::runtime_error("weights.npz: layer 0 must have K = 1 and layers 1-3 K = 3");
        L_[l] = transpose_layer(F);
    }
    reset();
}

void Stage01::reset() {
    const size_t c0 = (size_t)H_ * W_, c1 = c0 / 4;
    hidden_[0].assign(c0 * 12, 0.f);
    hidden_[1].assign(c0 * 12, 0.f);
    hidden_[2].assign(c1 * 24, 0.f);
    hidden_[3].assign(c1 * 24, 0.f);
    td_[0].assign(c1, 0);
    td_[1].assign(c1 / 4, 0);
    last_t_.assign(c0, -1.0);
}

void Stage01::preprocess(float t_us, int x, int y, float p, float feat[2]) {
    if (x < 0 || x >= W_ || y < 0 || y >= H_) {
        feat[0] = feat[1] = 0.f;
        return;
    }
    const size_t k = (size_t)y * W_ + x;
    const double prev = last_t_[k];
    float dt = 1.0f;
    if (prev >= 0.0) dt = (float)std::min(1.0, std::max(0.0, ((double)t_us - prev) / 1e5));
    last_t_[k] = (double)t_us;
    feat[0] = dt;
    feat[1] = p;
}

void Stage01::stage0(int x, int y, const float in[2], float out[12], bool full) {
    float mid[12];
    layer<2, 12>(L_[0], hidden_[0].data(), x, y, H_, W_, in, mid, true);
    layer<12, 12>(L_[1], hidden_[1].data(), x, y, H_, W_, mid, out, full);
}

void Stage01::stage1(int x1, int y1, const float in[12], float out[24], bool full) {
    float mid[24];
    layer<12, 24>(L_[2], hidden_[2].data(), x1, y1, H_ / 2, W_ / 2, in, mid, true);
    layer<24, 24>(L_[3], hidden_[3].data(), x1, y1, H_ / 2, W_ / 2, mid, out, full);
}

bool Stage01::tdrop_at(int level, int px, int py) {
    const int Wp = level == 0 ? W_ / 2 : W_ / 4;
    std::uint8_t& c = td_[level][(size_t)py * Wp + px];
    const unsigned pre = c;
    c = (std::uint8_t)(pre + 1u);
    return window_ <= 1 || pre % (unsigned)window_ == 0u;
}

}  // namespace ssla
