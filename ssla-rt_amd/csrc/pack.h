// pack.h -- fused per-position weights of one SSLA layer (host code).
//
// qvgIn[p] = [qW; vW; gW] @ scatter_p  (A, 3*D, IN), goW[p] = gather_p @ oW
// (A, D, D), with scatter_p[d, c] = W_in_cat[c, p*D + d] and gather_p[i, j] =
// W_out_cat[p*D + j, i] (src/ssla_kernels.cpp:73-153, weights_ssla.py:24-88).
// Products accumulate in fp32 over the inner index in ascending order.
#pragma once

#include <map>
#include <string>
#include <vector>

#include "weights_dir.h"

namespace ssla {

struct FusedLayer {
    int in_dim = 0, out_dim = 0, A = 0;   // A = 1 (K = 1) or 9 (K = 3)
    std::vector<float> qvgIn;             // (A, 3*D, IN)
    std::vector<float> goW;               // (A, D, D)
    std::vector<float> input_proj;        // (D, IN) or empty (IN == D)
    std::vector<float> gamma, beta;       // (D,)
};

// Reads and fuses layers/<index>; throws std::runtime_error on schema errors.
FusedLayer fuse_layer(const std::map<std::string, NpzTensor>& W, const std::string& prefix,
                      int in_dim, int out_dim);

// The sorted SSLA layer indices of a weights.npz (ssla_kernels.cpp:178-198).
std::vector<int> ssla_layer_indices(const std::map<std::string, NpzTensor>& W);

}  // namespace ssla
