// stage01.h -- SSLA-S stages 0 and 1 on the host CPU (the producer side of
// the drain): per-pixel preprocessing, layers L0..L3, and the two tdrop
// gates, for one shard.  Same arithmetic as the reference's generic fp32
// path (src/ssla_kernels.cpp:288-385, 738-921): fp32 matvecs and LRU,
// sigmoid = 1/(1+exp(-x)), fp64 LayerNorm.
#pragma once

#include <cstdint>
#include <string>
#include <vector>

#include "pack.h"

namespace ssla {

// One layer with input-major weights: qvg (A, IN, 3*OUT), go (A, OUT, OUT)
// indexed [p][i][o], ip (IN, OUT) or empty.
struct TLayer {
    int A = 0;
    std::vector<float> qvg, go, ip, gamma, beta;
};

class Stage01 {
public:
    // Loads meta.json + weights.npz; throws std::runtime_error on errors.
    explicit Stage01(const std::string& weights_dir);

    void reset();
    int H() const { return H_; }
    int W() const { return W_; }
    int tdrop_window() const { return window_; }

    // feat = [dt_norm, p]; dt_norm = clamp((t - last_t[pixel]) / 1e5, 0, 1),
    // 1 for the first event of a pixel (ssla_kernels.cpp:288-309).
    void preprocess(float t_us, int x, int y, float p, float feat[2]);

    // Stage forward at the stage's resolution.  full = false runs the
    // second layer state-only (v, g and the hidden update; no output).
    void stage0(int x, int y, const float in[2], float out[12], bool full);
    void stage1(int x1, int y1, const float in[12], float out[24], bool full);

    // Counter of the pooled cell (px, py) after stage `level` (0 or 1):
    // pre = c; c = pre + 1 (mod 256); pass = window <= 1 || pre % window == 0.
    bool tdrop_at(int level, int px, int py);

private:
    int H_ = 0, W_ = 0, window_ = 4;
    TLayer L_[4];
    std::vector<float> hidden_[4];
    std::vector<std::uint8_t> td_[2];
    std::vector<double> last_t_;
};

}  // namespace ssla
