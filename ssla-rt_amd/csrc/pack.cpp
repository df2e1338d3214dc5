// pack.cpp -- see pack.h.
#include "pack.h"

#include <algorithm>
#include <stdexcept>

namespace ssla {
namespace {

const NpzTensor& get(const std::map<std::string, NpzTensor>& W, const std::string& k,
                     const std::vector<int64_t>& shape) {
    const auto it = W.find(k);
    if (it == W.end()) throw std::runtime_error("weights.npz: missing " + k);
    if (!shape.empty() && it->second.shape != shape) {
        std::string got;
        for (auto d : it->second.shape) got += std::to_string(d) + ",";
        throw std::runtime_error("weights.npz: " + k + " has shape (" + got + ")");
    }
    return it->second;
}

// C = B @ A, B (bo, bi), A (bi, ai), k-outer fp32 accumulation.
void mm(const float* B, int bo, int bi, const float* A, int ai, float* C) {
    for (int o = 0; o < bo; ++o) {
        float* cr = C + (size_t)o * ai;
        std::fill(cr, cr + ai, 0.0f);
        for (int k = 0; k < bi; ++k) {
            const float bv = B[(size_t)o * bi + k];
            const float* ar = A + (size_t)k * ai;
            for (int i = 0; i < ai; ++i) cr[i] += bv * ar[i];
        }
    }
}

}  // namespace

FusedLayer fuse_layer(const std::map<std::string, NpzTensor>& W, const std::string& pre,
                      int IN, int D) {
    const NpzTensor& Win = get(W, pre + "/W_in_cat", {});
    const NpzTensor& Wout = get(W, pre + "/W_out_cat", {});
    if (Win.shape.size() != 2 || Win.shape[0] != IN || Wout.shape.size() != 2 || Wout.shape[1] != D)
        throw std::runtime_error(pre + ": W_in_cat must be (in_dim, n*out_dim) and W_out_cat (n*out_dim, out_dim)");
    const int win_cols = (int)Win.shape[1], wout_rows = (int)Wout.shape[0];
    if (win_cols % D || wout_rows % D) throw std::runtime_error(pre + ": W_*_cat not a multiple of out_dim");
    const int n_in = win_cols / D, n_out = wout_rows / D;
    const int A = std::max(n_in, n_out);
    if ((n_in != 1 && n_in != A) || (n_out != 1 && n_out != A) || (A != 1 && A != 9))
        throw std::runtime_error(pre + ": position counts must be 1 or 9");
    const NpzTensor& qW = get(W, pre + "/q_proj/weight", {D, D});
    const NpzTensor& vW = get(W, pre + "/v_proj/weight", {D, D});
    const NpzTensor& gW = get(W, pre + "/g_proj/weight", {D, D});
    const NpzTensor& oW = get(W, pre + "/o_proj/weight", {D, D});
    FusedLayer L;
    L.in_dim = IN;
    L.out_dim = D;
    L.A = A;
    L.gamma = get(W, pre + "/norm/weight", {D}).data;
    L.beta = get(W, pre + "/norm/bias", {D}).data;
    const auto ip = W.find(pre + "/input_proj/weight");
    if (IN != D) {
        if (ip == W.end()) throw std::runtime_error(pre + ": in_dim != out_dim but no input_proj");
        L.input_proj = get(W, pre + "/input_proj/weight", {D, IN}).data;
    } else if (ip != W.end()) {
        throw std::runtime_error(pre + ": unexpected input_proj for in_dim == out_dim");
    }
    std::vector<float> scatter((size_t)D * IN), gather((size_t)D * D);
    L.qvgIn.assign((size_t)A * 3 * D * IN, 0.f);
    L.goW.assign((size_t)A * D * D, 0.f);
    for (int p = 0; p < A; ++p) {
        const int pin = n_in == 1 ? 0 : p, pout = n_out == 1 ? 0 : p;
        for (int d = 0; d < D; ++d)
            for (int c = 0; c < IN; ++c)
                scatter[(size_t)d * IN + c] = Win.data[(size_t)c * win_cols + (size_t)pin * D + d];
        for (int i = 0; i < D; ++i)
            for (int j = 0; j < D; ++j)
                gather[(size_t)i * D + j] = Wout.data[((size_t)pout * D + j) * D + i];
        float* q = L.qvgIn.data() + (size_t)p * 3 * D * IN;
        mm(qW.data.data(), D, D, scatter.data(), IN, q);
        mm(vW.data.data(), D, D, scatter.data(), IN, q + (size_t)D * IN);
        mm(gW.data.data(), D, D, scatter.data(), IN, q + (size_t)2 * D * IN);
        mm(gather.data(), D, D, oW.data.data(), D, L.goW.data() + (size_t)p * D * D);
    }
    return L;
}

std::vector<int> ssla_layer_indices(const std::map<std::string, NpzTensor>& W) {
    std::vector<int> idx;
    for (const auto& kv : W) {
        const std::string& k = kv.first;
        if (k.rfind("layers/", 0) != 0) continue;
        const size_t sl = k.find('/', 7);
        if (sl == std::string::npos || k.substr(sl + 1) != "W_in_cat") continue;
        idx.push_back(std::stoi(k.substr(7, sl - 7)));
    }
    std::sort(idx.begin(), idx.end());
    return idx;
}

}  // namespace ssla
