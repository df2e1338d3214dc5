// stage01.cpp -- see stage01.h.
#include "stage01.h"

#include <immintrin.h>

#include <algorithm>
#include <cmath>
#include <cstring>
#include <stdexcept>

namespace ssla {
namespace {

// exp on 8 / 4 lanes (AVX2 + FMA): Cody-Waite range reduction
// x = k ln2 + r with ln2 split into a short high part and a low part
// (0.693359375 and -2.12194440e-4, as in the Cephes library's expf) so
// k * high is exact, |r| <= ln2 / 2; e^r by its degree-6 Taylor polynomial
// (truncation error below 1.3e-7 relative); 2^k from the exponent bits.
// Inputs are clamped to [-87, 88], where 2^k stays a normal float.  All
// steps are FMA/round builtins so -ffast-math cannot reassociate them.
inline __m256 exp8(__m256 x) {
    x = _mm256_min_ps(_mm256_max_ps(x, _mm256_set1_ps(-87.0f)), _mm256_set1_ps(88.0f));
    const __m256 k = _mm256_round_ps(_mm256_mul_ps(x, _mm256_set1_ps(1.44269504088896341f)),
                                     _MM_FROUND_TO_NEAREST_INT | _MM_FROUND_NO_EXC);
    __m256 r = _mm256_fnmadd_ps(k, _mm256_set1_ps(0.693359375f), x);
    r = _mm256_fnmadd_ps(k, _mm256_set1_ps(-2.12194440e-4f), r);
    __m256 p = _mm256_set1_ps(1.0f / 720.0f);
    p = _mm256_fmadd_ps(p, r, _mm256_set1_ps(1.0f / 120.0f));
    p = _mm256_fmadd_ps(p, r, _mm256_set1_ps(1.0f / 24.0f));
    p = _mm256_fmadd_ps(p, r, _mm256_set1_ps(1.0f / 6.0f));
    p = _mm256_fmadd_ps(p, r, _mm256_set1_ps(0.5f));
    p = _mm256_fmadd_ps(p, r, _mm256_set1_ps(1.0f));
    p = _mm256_fmadd_ps(p, r, _mm256_set1_ps(1.0f));
    const __m256i e = _mm256_slli_epi32(_mm256_add_epi32(_mm256_cvtps_epi32(k), _mm256_set1_epi32(127)), 23);
    return _mm256_mul_ps(p, _mm256_castsi256_ps(e));
}

inline __m128 exp4(__m128 x) {
    x = _mm_min_ps(_mm_max_ps(x, _mm_set1_ps(-87.0f)), _mm_set1_ps(88.0f));
    const __m128 k = _mm_round_ps(_mm_mul_ps(x, _mm_set1_ps(1.44269504088896341f)),
                                  _MM_FROUND_TO_NEAREST_INT | _MM_FROUND_NO_EXC);
    __m128 r = _mm_fnmadd_ps(k, _mm_set1_ps(0.693359375f), x);
    r = _mm_fnmadd_ps(k, _mm_set1_ps(-2.12194440e-4f), r);
    __m128 p = _mm_set1_ps(1.0f / 720.0f);
    p = _mm_fmadd_ps(p, r, _mm_set1_ps(1.0f / 120.0f));
    p = _mm_fmadd_ps(p, r, _mm_set1_ps(1.0f / 24.0f));
    p = _mm_fmadd_ps(p, r, _mm_set1_ps(1.0f / 6.0f));
    p = _mm_fmadd_ps(p, r, _mm_set1_ps(0.5f));
    p = _mm_fmadd_ps(p, r, _mm_set1_ps(1.0f));
    p = _mm_fmadd_ps(p, r, _mm_set1_ps(1.0f));
    const __m128i e = _mm_slli_epi32(_mm_add_epi32(_mm_cvtps_epi32(k), _mm_set1_epi32(127)), 23);
    return _mm_mul_ps(p, _mm_castsi128_ps(e));
}

// The gated state update of one patch cell over N channels (N % 4 == 0):
// h = sigmoid(g) * h + v, and qh = q * h when q is given.
template <int N>
inline void gate_update(float* h, const float* g, const float* v, const float* q, float* qh) {
    static_assert(N % 4 == 0, "channel count must be a multiple of 4");
    int c = 0;
    for (; c + 8 <= N; c += 8) {
        const __m256 one = _mm256_set1_ps(1.0f);
        const __m256 s = _mm256_div_ps(one, _mm256_add_ps(one, exp8(_mm256_sub_ps(_mm256_setzero_ps(),
                                                                              _mm256_loadu_ps(g + c)))));
        const __m256 hn = _mm256_fmadd_ps(s, _mm256_loadu_ps(h + c), _mm256_loadu_ps(v + c));
        _mm256_storeu_ps(h + c, hn);
        if (q) _mm256_storeu_ps(qh + c, _mm256_mul_ps(_mm256_loadu_ps(q + c), hn));
    }
    for (; c < N; c += 4) {
        const __m128 one = _mm_set1_ps(1.0f);
        const __m128 s = _mm_div_ps(one, _mm_add_ps(one, exp4(_mm_sub_ps(_mm_setzero_ps(),
                                                                          _mm_loadu_ps(g + c)))));
        const __m128 hn = _mm_fmadd_ps(s, _mm_loadu_ps(h + c), _mm_loadu_ps(v + c));
        _mm_storeu_ps(h + c, hn);
        if (q) _mm_storeu_ps(qh + c, _mm_mul_ps(_mm_loadu_ps(q + c), hn));
    }
}

// Up to kTile events share each weight load in the projection and
// gather-o products.
constexpr int kTile = 4;

// acc[t][v] += sum_i x_t[i] * W[i][8v .. 8v+8) for NT <= kTile events
// (inputs xs[t], IN floats each) and V 8-lane vectors; W rows are `ld`
// floats apart.  One FMA chain per (event, vector), i ascending, so every
// event's sums come out the same whatever events share its tile.
template <int IN, int V, int NT>
inline void tile_matvec_n(const float* const* xs, const float* W, int ld, __m256 (*acc)[V]) {
    __m256 a[NT][V];
#pragma GCC unroll 4
    for (int t = 0; t < NT; ++t)
#pragma GCC unroll 9
        for (int v = 0; v < V; ++v) a[t][v] = acc[t][v];
#pragma GCC unroll 2
    for (int i = 0; i < IN; ++i) {
        __m256 xi[NT];
#pragma GCC unroll 4
        for (int t = 0; t < NT; ++t) xi[t] = _mm256_broadcast_ss(xs[t] + i);
        const float* w = W + (size_t)i * ld;
#pragma GCC unroll 9
        for (int v = 0; v < V; ++v) {
            const __m256 wv = _mm256_load_ps(w + 8 * v);
#pragma GCC unroll 4
            for (int t = 0; t < NT; ++t) a[t][v] = _mm256_fmadd_ps(xi[t], wv, a[t][v]);
        }
    }
#pragma GCC unroll 4
    for (int t = 0; t < NT; ++t)
#pragma GCC unroll 9
        for (int v = 0; v < V; ++v) acc[t][v] = a[t][v];
}

// Events per tile for V vectors: at most 10 accumulators, so they, the
// broadcast inputs and one weight vector fit the 16 vector registers.
template <int V>
constexpr int tile_events() {
    return std::max(1, std::min(kTile, 10 / V));
}

template <int IN, int V>
inline void tile_matvec(int nt, const float* const* xs, const float* W, int ld, __m256 (*acc)[V]) {
    constexpr int MAXNT = tile_events<V>();
    if (MAXNT >= 4 && nt >= 4) {
        tile_matvec_n<IN, V, (MAXNT >= 4 ? 4 : 1)>(xs, W, ld, acc);
    } else if (MAXNT >= 3 && nt == 3) {
        tile_matvec_n<IN, V, (MAXNT >= 3 ? 3 : 1)>(xs, W, ld, acc);
    } else if (MAXNT >= 2 && nt == 2) {
        tile_matvec_n<IN, V, (MAXNT >= 2 ? 2 : 1)>(xs, W, ld, acc);
    } else {
        tile_matvec_n<IN, V, 1>(xs, W, ld, acc);
    }
}

// One SSLA layer over a batch of n events, layer-major: the layer's hidden
// state sees the events in batch order, exactly as if each event ran its
// layer alone, because the projections do not read the state and the
// state updates run in event order.
//   A  projections: for every patch position p and every event whose patch
//      cell at p is inside the grid, [q v g] = qvg[p]^T x (q only for
//      events with full set); the weights of p are reused across the batch.
//   B  state scan, event order, patch cells in the reference's order
//      (p = 8..0; ssla_kernels.cpp:343-369): h = sigmoid(g) h + v,
//      qh = q * h.
//   C  for full events: acc = sum over p = 8..0 of go[p]^T qh, plus the
//      input projection (or the input itself), then fp64 LayerNorm.
// in: n rows of `ldi` floats; out: n rows of `ldo` floats (full events).
template <int IN, int OUT>
void layer_batch(const TLayer& T, float* H, int Hl, int Wl, int n, const int* xs, const int* ys,
                 const float* in, int ldi, const std::uint8_t* full, float* out, int ldo,
                 BatchScratch& sc) {
    constexpr int OP = (OUT + 7) / 8 * 8;
    constexpr int VO = OP / 8;            // vectors per q / v / g run
    constexpr int NCP = 3 * OP;
    const int A = T.A;
    sc.cell.resize((size_t)n * A);
    sc.P.resize((size_t)n * A * NCP);
    sc.QH.resize((size_t)n * A * OP);
    sc.ACC.resize((size_t)n * OP);
    int* cell = sc.cell.data();
    float* P = sc.P.data();
    float* QH = sc.QH.data();
    float* ACC = sc.ACC.data();
    for (int e = 0; e < n; ++e) {
        const int x = xs[e], y = ys[e];
        for (int p = 0; p < A; ++p) {
            const int dy = A == 1 ? 0 : 1 - p / 3, dx = A == 1 ? 0 : 1 - p % 3;
            const int px = x + dx, py = y + dy;
            cell[(size_t)e * A + p] = (px >= 0 && px < Wl && py >= 0 && py < Hl) ? py * Wl + px : -1;
        }
    }
    // A: projections, weights of one patch position at a time (they stay
    // in L1 across the batch).  Full events need [q v g], the others [v g];
    // each class runs in tiles sized to keep every accumulator in a register.
    constexpr int NTF = tile_events<3 * VO>();
    constexpr int NTS = tile_events<2 * VO>();
    int idx[kTile];
    const float* xp[kTile];
    for (int p = 0; p < A; ++p) {
        const float* Wp = T.qvg.data() + (size_t)p * IN * NCP;
        for (int cls = 0; cls < 2; ++cls) {          // 0: full, 1: state only
            const int cap = cls == 0 ? NTF : NTS;
            int e = 0;
            while (e < n) {
                int nt = 0;
                for (; e < n && nt < cap; ++e) {
                    if (cell[(size_t)e * A + p] < 0 || (full[e] != 0) != (cls == 0)) continue;
                    idx[nt] = e;
                    xp[nt] = in + (size_t)e * ldi;
                    ++nt;
                }
                if (!nt) break;
                if (cls == 0) {
                    __m256 acc[kTile][3 * VO];
                    for (int t = 0; t < kTile; ++t)
                        for (int v = 0; v < 3 * VO; ++v) acc[t][v] = _mm256_setzero_ps();
                    tile_matvec<IN, 3 * VO>(nt, xp, Wp, NCP, acc);
                    for (int t = 0; t < nt; ++t)
                        for (int v = 0; v < 3 * VO; ++v)
                            _mm256_store_ps(P + ((size_t)idx[t] * A + p) * NCP + 8 * v, acc[t][v]);
                } else {
                    __m256 acc[kTile][2 * VO];
                    for (int t = 0; t < kTile; ++t)
                        for (int v = 0; v < 2 * VO; ++v) acc[t][v] = _mm256_setzero_ps();
                    tile_matvec<IN, 2 * VO>(nt, xp, Wp + OP, NCP, acc);
                    for (int t = 0; t < nt; ++t)
                        for (int v = 0; v < 2 * VO; ++v)
                            _mm256_store_ps(P + ((size_t)idx[t] * A + p) * NCP + OP + 8 * v, acc[t][v]);
                }
            }
        }
    }
    // B: state scan in event order
    for (int e = 0; e < n; ++e) {
        for (int p = A - 1; p >= 0; --p) {
            const int c = cell[(size_t)e * A + p];
            if (c < 0) continue;
            float* r = P + ((size_t)e * A + p) * NCP;
            gate_update<OUT>(H + (size_t)c * OUT, r + 2 * OP, r + OP, full[e] ? r : nullptr,
                             QH + ((size_t)e * A + p) * OP);
        }
    }
    // C: gather-o for full events, patch positions 8..0, then LayerNorm
    for (int e = 0; e < n; ++e)
        if (full[e]) std::memset(ACC + (size_t)e * OP, 0, sizeof(float) * OP);
    constexpr int NTG = tile_events<VO>();
    for (int p = A - 1; p >= 0; --p) {
        const float* G = T.go.data() + (size_t)p * OUT * OP;
        int e = 0;
        while (e < n) {
            int nt = 0;
            for (; e < n && nt < NTG; ++e) {
                if (!full[e] || cell[(size_t)e * A + p] < 0) continue;
                idx[nt] = e;
                xp[nt] = QH + ((size_t)e * A + p) * OP;
                ++nt;
            }
            if (!nt) break;
            __m256 acc[kTile][VO];
            for (int t = 0; t < nt; ++t)
                for (int v = 0; v < VO; ++v) acc[t][v] = _mm256_load_ps(ACC + (size_t)idx[t] * OP + 8 * v);
            tile_matvec<OUT, VO>(nt, xp, G, OP, acc);
            for (int t = 0; t < nt; ++t)
                for (int v = 0; v < VO; ++v) _mm256_store_ps(ACC + (size_t)idx[t] * OP + 8 * v, acc[t][v]);
        }
    }
    for (int e = 0; e < n; ++e) {
        if (!full[e]) continue;
        const float* x = in + (size_t)e * ldi;
        alignas(32) float res[OP];
        if (!T.ip.empty()) {
            __m256 r[1][VO];
            for (int v = 0; v < VO; ++v) r[0][v] = _mm256_setzero_ps();
            const float* xt[1] = {x};
            tile_matvec<IN, VO>(1, xt, T.ip.data(), OP, r);
            for (int v = 0; v < VO; ++v) _mm256_store_ps(res + 8 * v, r[0][v]);
        } else {
            for (int o = 0; o < OUT; ++o) res[o] = x[o];
        }
        float* a = ACC + (size_t)e * OP;
        double sum = 0.0;
        for (int o = 0; o < OUT; ++o) {
            a[o] += res[o];
            sum += (double)a[o];
        }
        const double mean = sum / OUT;
        double var = 0.0;
        for (int o = 0; o < OUT; ++o) {
            const double d = (double)a[o] - mean;
            var += d * d;
        }
        var /= OUT;
        const double inv = 1.0 / std::sqrt(var + 1e-5);
        float* y = out + (size_t)e * ldo;
        for (int o = 0; o < OUT; ++o)
            y[o] = (float)(((double)a[o] - mean) * inv * (double)T.gamma[o] + (double)T.beta[o]);
    }
}

// Input-major, lane-padded copies of a fused layer (see TLayer).
TLayer transpose_layer(const FusedLayer& L) {
    TLayer T;
    const int A = L.A, IN = L.in_dim, D = L.out_dim;
    const int OP = (D + 7) / 8 * 8, NCP = 3 * OP;
    T.A = A;
    T.OP = OP;
    T.qvg.assign((size_t)A * IN * NCP, 0.f);
    T.go.assign((size_t)A * D * OP, 0.f);
    for (int p = 0; p < A; ++p) {
        for (int part = 0; part < 3; ++part)
            for (int o = 0; o < D; ++o)
                for (int i = 0; i < IN; ++i)
                    T.qvg[((size_t)p * IN + i) * NCP + part * OP + o] =
                        L.qvgIn[((size_t)p * 3 * D + part * D + o) * IN + i];
        for (int o = 0; o < D; ++o)
            for (int i = 0; i < D; ++i)
                T.go[((size_t)p * D + i) * OP + o] = L.goW[((size_t)p * D + o) * D + i];
    }
    if (!L.input_proj.empty()) {
        T.ip.assign((size_t)IN * OP, 0.f);
        for (int o = 0; o < D; ++o)
            for (int i = 0; i < IN; ++i) T.ip[(size_t)i * OP + o] = L.input_proj[(size_t)o * IN + i];
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
    const std::uint8_t f = full;
    stage0_batch(1, &x, &y, in, &f, out);
}

void Stage01::stage1(int x1, int y1, const float in[12], float out[24], bool full) {
    const std::uint8_t f = full;
    stage1_batch(1, &x1, &y1, in, &f, out);
}

void Stage01::stage0_batch(int n, const int* x, const int* y, const float* in,
                           const std::uint8_t* full, float* out) {
    if (n <= 0) return;
    mid_.resize((size_t)n * 12);
    ones_.assign((size_t)n, 1);
    layer_batch<2, 12>(L_[0], hidden_[0].data(), H_, W_, n, x, y, in, 2, ones_.data(), mid_.data(), 12,
                       sc_);
    layer_batch<12, 12>(L_[1], hidden_[1].data(), H_, W_, n, x, y, mid_.data(), 12, full, out, 12, sc_);
}

void Stage01::stage1_batch(int n, const int* x1, const int* y1, const float* in,
                           const std::uint8_t* full, float* out) {
    if (n <= 0) return;
    mid_.resize((size_t)n * 24);
    ones_.assign((size_t)n, 1);
    layer_batch<12, 24>(L_[2], hidden_[2].data(), H_ / 2, W_ / 2, n, x1, y1, in, 12, ones_.data(),
                        mid_.data(), 24, sc_);
    layer_batch<24, 24>(L_[3], hidden_[3].data(), H_ / 2, W_ / 2, n, x1, y1, mid_.data(), 24, full,
                        out, 24, sc_);
}

bool Stage01::tdrop_at(int level, int px, int py) {
    const int Wp = level == 0 ? W_ / 2 : W_ / 4;
    std::uint8_t& c = td_[level][(size_t)py * Wp + px];
    const unsigned pre = c;
    c = (std::uint8_t)(pre + 1u);
    return window_ <= 1 || pre % (unsigned)window_ == 0u;
}

}  // namespace ssla
