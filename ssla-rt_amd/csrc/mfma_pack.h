// mfma_pack.h -- fragment-order weight copies for the 16 x 16 x 4 fp32 MFMA
// contractions of the drains (v_mfma_f32_16x16x4_f32).
//
// Operand layout of v_mfma_f32_16x16x4_f32 for lane l, i = l % 16, k = l / 16:
//   A: row i, column k;  B: row k, column i;  D (4 values): rows 4k..4k+3,
//   column i.
// A contraction over K runs K / 4 such steps; step s covers K rows 4s..4s+3.
// The packed copies store, per work item, the B values of each lane for
// four consecutive steps as one float4, so one wave-wide 16-byte load
// (1 KB contiguous) feeds four MFMAs.
//
//   projection  (ProjPack): per layer, items (delta, 16-column tile of
//               [q | v | g]); B[k][c] = qvgIn[delta][k][c], k < IN
//   contraction (OutPack):  items (16-column tile, K part of kKSplit);
//               B = [goW as (9*OUT) x OUT, delta-major; input_proj (IN x OUT)
//               when IN != OUT]
#pragma once

#include <hip/hip_runtime.h>

#include "ssla_abi.h"

namespace ssla {

constexpr int kMT = 16;       // MFMA tile rows / columns
constexpr int kKSplit = 8;    // K parts of the contraction

typedef float f32x4 __attribute__((ext_vector_type(4)));

// Global-memory accesses through address-space-1 pointers: pointers that
// reach device code as generic values (loaded from descriptor tables) would
// otherwise compile to flat instructions that also wait on the LDS counter.
#define SSLA_GLOBAL __attribute__((address_space(1)))
__device__ __forceinline__ float gload(const float* p) {
    return *(const SSLA_GLOBAL float*)p;
}
__device__ __forceinline__ void gstore(float* p, float v) {
    *(SSLA_GLOBAL float*)p = v;
}

template <int IN, int OUT>
struct ProjPack {
    static constexpr int NC = 3 * OUT, T = NC / kMT, TQ = OUT / kMT, KS = IN / 4;
    static constexpr int KS4 = (KS + 3) / 4;     // float4 groups of steps
    static constexpr int N = 9 * T;              // (delta, column tile) items
    static constexpr size_t PACKED = (size_t)N * KS4 * 256;   // floats
    static_assert(OUT % kMT == 0 && IN % 4 == 0, "tile shapes");
    // b[s], s < 4 * KS4: this lane's B value of step s of item `it`
    static __device__ __forceinline__ void load(const float* __restrict__ pp, int it, int lane,
                                                float* b) {
        const SSLA_GLOBAL f32x4* src = (const SSLA_GLOBAL f32x4*)pp + (size_t)it * KS4 * 64 + lane;
        #pragma unroll
        for (int g = 0; g < KS4; ++g) {
            const f32x4 v = src[g * 64];
            #pragma unroll
            for (int j = 0; j < 4; ++j) b[4 * g + j] = v[j];
        }
    }
};

template <int IN, int OUT>
struct OutPack {
    static constexpr bool IP = IN != OUT;          // residual through input_proj
    static constexpr int KQ = 9 * OUT, KT = KQ + (IP ? IN : 0);
    static constexpr int NT = OUT / kMT, STEPS = KT / 4;
    static constexpr int SPER = (STEPS + kKSplit - 1) / kKSplit;   // steps per K part
    static constexpr int SP4 = (SPER + 3) / 4;
    static constexpr int N = NT * kKSplit;         // (column tile, K part) items
    static constexpr size_t PACKED = (size_t)N * SP4 * 256;   // floats
    static __device__ __forceinline__ void load(const float* __restrict__ po, int it, int lane,
                                                float* b) {
        const SSLA_GLOBAL f32x4* src = (const SSLA_GLOBAL f32x4*)po + (size_t)it * SP4 * 64 + lane;
        #pragma unroll
        for (int g = 0; g < SP4; ++g) {
            const f32x4 v = src[g * 64];
            #pragma unroll
            for (int j = 0; j < 4; ++j) b[4 * g + j] = v[j];
        }
    }
};

// The contraction split at delta boundaries (whole-ring drain): items
// (16-column tile nt, part), parts 0..8 the rows of goW[delta] (OUT / 4
// steps), part 9 (when IN != OUT) input_proj (IN / 4 steps, zero padded).
template <int IN, int OUT>
struct OutPackD {
    static constexpr bool IP = IN != OUT;
    static constexpr int NT = OUT / kMT, PARTS = 9 + (IP ? 1 : 0);
    static constexpr int SD = OUT / 4, SD4 = SD / 4;   // steps and float4 groups per part
    static constexpr int N = NT * PARTS;
    static constexpr size_t PACKED = (size_t)N * SD4 * 256;   // floats
    static_assert(OUT % 16 == 0 && IN <= OUT, "part shapes");
    static __device__ __forceinline__ void load(const float* __restrict__ po, int nt, int part,
                                                int lane, float* b) {
        const SSLA_GLOBAL f32x4* src =
            (const SSLA_GLOBAL f32x4*)po + (size_t)(nt * PARTS + part) * SD4 * 64 + lane;
        #pragma unroll
        for (int g = 0; g < SD4; ++g) {
            const f32x4 v = src[g * 64];
            #pragma unroll
            for (int j = 0; j < 4; ++j) b[4 * g + j] = v[j];
        }
    }
};

// element (item, group g, lane, j) = qvgIn[delta][(4g + j) * 4 + lane / 16][t * 16 + lane % 16]
template <int IN, int OUT>
__device__ __forceinline__ float proj_elem(const float* __restrict__ qvgIn, size_t q) {
    using P = ProjPack<IN, OUT>;
    const int j = (int)(q & 3), lane = (int)((q >> 2) & 63);
    const size_t r = q >> 8;
    const int g = (int)(r % P::KS4), it = (int)(r / P::KS4);
    const int d = it / P::T, t = it - d * P::T;
    const int k = (4 * g + j) * 4 + lane / 16, c = t * kMT + lane % 16;
    return k < IN ? qvgIn[((size_t)d * IN + k) * P::NC + c] : 0.f;
}

// element (item (nt, ks), group g, lane, j) = B[k][nt * 16 + lane % 16] with
// k = (ks * SPER + 4g + j) * 4 + lane / 16; zero past the part or past K
template <int IN, int OUT>
__device__ __forceinline__ float out_elem(const float* __restrict__ goW,
                                          const float* __restrict__ ip, size_t q) {
    using O = OutPack<IN, OUT>;
    const int j = (int)(q & 3), lane = (int)((q >> 2) & 63);
    const size_t r = q >> 8;
    const int g = (int)(r % O::SP4), it = (int)(r / O::SP4);
    const int nt = it / kKSplit, ks = it - nt * kKSplit;
    const int step = 4 * g + j, s = ks * O::SPER + step;
    const int k = s * 4 + lane / 16, c = nt * kMT + lane % 16;
    float v = 0.f;
    if (step < O::SPER && s < O::STEPS)
        v = k < O::KQ ? goW[(size_t)k * OUT + c] : ip[(size_t)(k - O::KQ) * OUT + c];
    return v;
}

// element ((nt, part), group g, lane, j): local row kl = (4g + j) * 4 + lane / 16,
// column c = nt * 16 + lane % 16; goW[part * OUT + kl][c] or input_proj[kl][c]
template <int IN, int OUT>
__device__ __forceinline__ float out_d_elem(const float* __restrict__ goW,
                                            const float* __restrict__ ip, size_t q) {
    using O = OutPackD<IN, OUT>;
    const int j = (int)(q & 3), lane = (int)((q >> 2) & 63);
    const size_t r = q >> 8;
    const int g = (int)(r % O::SD4), it = (int)(r / O::SD4);
    const int nt = it / O::PARTS, part = it - nt * O::PARTS;
    const int kl = (4 * g + j) * 4 + lane / 16, c = nt * kMT + lane % 16;
    float v = 0.f;
    if (part < 9) v = goW[((size_t)part * OUT + kl) * OUT + c];
    else if (kl < IN) v = ip[(size_t)kl * OUT + c];
    return v;
}

// Packed copies of the four layers L4..L7.
struct PackedWeights {
    const float* pp[4];
    const float* po[4];
};

// Source weights of the four layers, by value for the packing kernel.
struct PackSrc {
    const float* qvgIn[4];
    const float* goW[4];
    const float* ip[4];
};

// Floats of one layer's projection copy and contraction copy.
template <int IN, int OUT, bool D>
struct LayerPack {
    static constexpr size_t NP = ProjPack<IN, OUT>::PACKED;
    static constexpr size_t NO = D ? OutPackD<IN, OUT>::PACKED : OutPack<IN, OUT>::PACKED;
};

// Buffer order: L4 projection, L4 contraction, L5 ..., L7 contraction.
// D selects the contraction split at delta boundaries (whole-ring drain)
// instead of the K split of the batch kernels.
template <bool D>
struct PackLayout {
    using A = LayerPack<SSLA_C1, SSLA_C2, D>;
    using B = LayerPack<SSLA_C2, SSLA_C2, D>;
    using C = LayerPack<SSLA_C2, SSLA_C3, D>;
    using E = LayerPack<SSLA_C3, SSLA_C3, D>;
    static constexpr size_t off[9] = {0,
                                      A::NP, A::NP + A::NO,
                                      A::NP + A::NO + B::NP, A::NP + A::NO + B::NP + B::NO,
                                      A::NP + A::NO + B::NP + B::NO + C::NP,
                                      A::NP + A::NO + B::NP + B::NO + C::NP + C::NO,
                                      A::NP + A::NO + B::NP + B::NO + C::NP + C::NO + E::NP,
                                      A::NP + A::NO + B::NP + B::NO + C::NP + C::NO + E::NP +
                                          E::NO};
};

template <int IN, int OUT, bool D>
__device__ __forceinline__ float out_any(const float* goW, const float* ip, size_t q) {
    if constexpr (D) return out_d_elem<IN, OUT>(goW, ip, q);
    else return out_elem<IN, OUT>(goW, ip, q);
}

// All eight copies in one launch, one thread per packed float.
template <bool D>
__global__ void k_pack_all(PackSrc s, float* __restrict__ buf) {
    using L = PackLayout<D>;
    const size_t q = (size_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (q >= L::off[8]) return;
    float v;
    if (q < L::off[1]) v = proj_elem<SSLA_C1, SSLA_C2>(s.qvgIn[0], q);
    else if (q < L::off[2]) v = out_any<SSLA_C1, SSLA_C2, D>(s.goW[0], s.ip[0], q - L::off[1]);
    else if (q < L::off[3]) v = proj_elem<SSLA_C2, SSLA_C2>(s.qvgIn[1], q - L::off[2]);
    else if (q < L::off[4]) v = out_any<SSLA_C2, SSLA_C2, D>(s.goW[1], s.ip[1], q - L::off[3]);
    else if (q < L::off[5]) v = proj_elem<SSLA_C2, SSLA_C3>(s.qvgIn[2], q - L::off[4]);
    else if (q < L::off[6]) v = out_any<SSLA_C2, SSLA_C3, D>(s.goW[2], s.ip[2], q - L::off[5]);
    else if (q < L::off[7]) v = proj_elem<SSLA_C3, SSLA_C3>(s.qvgIn[3], q - L::off[6]);
    else v = out_any<SSLA_C3, SSLA_C3, D>(s.goW[3], s.ip[3], q - L::off[7]);
    buf[q] = v;
}

template <bool D>
inline size_t packed_floats() { return PackLayout<D>::off[8]; }

inline size_t packed_weight_floats() { return packed_floats<false>(); }
inline size_t packed_weight_floats_d() { return packed_floats<true>(); }

template <bool D>
inline hipError_t pack_all(const LayerWeightsS2S3* L, float* buf, PackedWeights* out,
                           hipStream_t st) {
    using PL = PackLayout<D>;
    PackSrc s{};
    for (int i = 0; i < 4; ++i) {
        s.qvgIn[i] = L[i].qvgIn;
        s.goW[i] = L[i].goW;
        s.ip[i] = L[i].input_proj;
        out->pp[i] = buf + PL::off[2 * i];
        out->po[i] = buf + PL::off[2 * i + 1];
    }
    constexpr int TB = 256;
    hipLaunchKernelGGL((k_pack_all<D>), dim3((unsigned)((PL::off[8] + TB - 1) / TB)), dim3(TB), 0,
                       st, s, buf);
    return hipGetLastError();
}

// Fills `out` from layers L[0..3] (L4..L7) into buf (packed_weight_floats_d()
// floats), on stream st; returns the launch status.
inline hipError_t pack_weights_d(const LayerWeightsS2S3* L, float* buf, PackedWeights* out,
                                 hipStream_t st) {
    return pack_all<true>(L, buf, out, st);
}

// Same for the batch kernels (packed_weight_floats() floats).
inline hipError_t pack_weights(const LayerWeightsS2S3* L, float* buf, PackedWeights* out,
                               hipStream_t st) {
    return pack_all<false>(L, buf, out, st);
}

}  // namespace ssla
