// stage01.h -- SSLA-S stages 0 and 1 on the host CPU (the producer side of
// the drain): per-pixel preprocessing, layers L0..L3, and the two tdrop
// gates, for one shard.  Same arithmetic as the reference's generic fp32
// path (src/ssla_kernels.cpp:288-385, 738-921): fp32 matvecs and LRU,
// sigmoid = 1/(1+exp(-x)), fp64 LayerNorm.
#pragma once

#include <cstddef>
#include <cstdint>
#include <new>
#include <string>
#include <vector>

#include "pack.h"

namespace ssla {

// 32-byte aligned storage for the AVX2 weight rows.
template <class T>
struct AlignedAlloc {
    using value_type = T;
    AlignedAlloc() = default;
    template <class U>
    AlignedAlloc(const AlignedAlloc<U>&) {}
    T* allocate(std::size_t n) {
        void* p = ::operator new(n * sizeof(T), std::align_val_t(32));
        return static_cast<T*>(p);
    }
    void deallocate(T* p, std::size_t) { ::operator delete(p, std::align_val_t(32)); }
    template <class U>
    bool operator==(const AlignedAlloc<U>&) const { return true; }
    template <class U>
    bool operator!=(const AlignedAlloc<U>&) const { return false; }
};

// One layer with input-major weights, every output run padded with zeros
// to OP = OUT rounded up to 8 lanes: qvg (A, IN, 3*OP) holding the q, v
// and g columns at offsets 0, OP, 2*OP; go (A, OUT, OP) indexed [p][i][o];
// ip (IN, OP) or empty.  Rows start on 32-byte boundaries.
struct TLayer {
    int A = 0;
    int OP = 0;
    std::vector<float, AlignedAlloc<float>> qvg, go, ip;
    std::vector<float> gamma, beta;
};

// Per-batch work space of the layer-major batch path.
struct BatchScratch {
    std::vector<int> cell;                              // (n, A) patch cell or -1
    std::vector<float, AlignedAlloc<float>> P, QH, ACC; // projections, q*h, gather-o sums
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

    // The same over n events in order (in / out: n rows of 2 / 12 / 24
    // floats; full[e] as above), layer by layer: each layer's hidden state
    // sees the events in order, so the results equal n single calls.  Rows
    // of out for events with full[e] == 0 are left untouched.
    void stage0_batch(int n, const int* x, const int* y, const float* in,
                      const std::uint8_t* full, float* out);
    void stage1_batch(int n, const int* x1, const int* y1, const float* in,
                      const std::uint8_t* full, float* out);

    // Counter of the pooled cell (px, py) after stage `level` (0 or 1):
    // pre = c; c = pre + 1 (mod 256); pass = window <= 1 || pre % window == 0.
    bool tdrop_at(int level, int px, int py);

private:
    int H_ = 0, W_ = 0, window_ = 4;
    TLayer L_[4];
    std::vector<float> hidden_[4];
    std::vector<std::uint8_t> td_[2];
    std::vector<double> last_t_;
    BatchScratch sc_;
    std::vector<float> mid_;
    std::vector<std::uint8_t> ones_;
};

}  // namespace ssla
