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
__global__ void k_pack_proj(const float* __restrict__ qvgIn, float* __restrict__ pp) {
    using P = ProjPack<IN, OUT>;
    const size_t q = (size_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (q >= P::PACKED) return;
    const int j = (int)(q & 3), lane = (int)((q >> 2) & 63);
    const size_t r = q >> 8;
    const int g = (int)(r % P::KS4), it = (int)(r / P::KS4);
    const int d = it / P::T, t = it - d * P::T;
    const int k = (4 * g + j) * 4 + lane / 16, c = t * kMT + lane % 16;
    pp[q] = k < IN ? qvgIn[((size_t)d * IN + k) * P::NC + c] : 0.f;
}

// element (item (nt, ks), group g, lane, j) = B[k][nt * 16 + lane % 16] with
// k = (ks * SPER + 4g + j) * 4 + lane / 16; zero past the part or past K
template <int IN, int OUT>
__global__ void k_pack_out(const float* __restrict__ goW, const float* __restrict__ ip,
                           float* __restrict__ po) {
    using O = OutPack<IN, OUT>;
    const size_t q = (size_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (q >= O::PACKED) return;
    const int j = (int)(q & 3), lane = (int)((q >> 2) & 63);
    const size_t r = q >> 8;
    const int g = (int)(r % O::SP4), it = (int)(r / O::SP4);
    const int nt = it / kKSplit, ks = it - nt * kKSplit;
    const int step = 4 * g + j, s = ks * O::SPER + step;
    const int k = s * 4 + lane / 16, c = nt * kMT + lane % 16;
    float v = 0.f;
    if (step < O::SPER && s < O::STEPS)
        v = k < O::KQ ? goW[(size_t)k * OUT + c] : ip[(size_t)(k - O::KQ) * OUT + c];
    po[q] = v;
}

// element ((nt, part), group g, lane, j): local row kl = (4g + j) * 4 + lane / 16,
// column c = nt * 16 + lane % 16; goW[part * OUT + kl][c] or input_proj[kl][c]
template <int IN, int OUT>
__global__ void k_pack_out_d(const float* __restrict__ goW, const float* __restrict__ ip,
                             float* __restrict__ po) {
    using O = OutPackD<IN, OUT>;
    const size_t q = (size_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (q >= O::PACKED) return;
    const int j = (int)(q & 3), lane = (int)((q >> 2) & 63);
    const size_t r = q >> 8;
    const int g = (int)(r % O::SD4), it = (int)(r / O::SD4);
    const int nt = it / O::PARTS, part = it - nt * O::PARTS;
    const int kl = (4 * g + j) * 4 + lane / 16, c = nt * kMT + lane % 16;
    float v = 0.f;
    if (part < 9) v = goW[((size_t)part * OUT + kl) * OUT + c];
    else if (kl < IN) v = ip[(size_t)kl * OUT + c];
    po[q] = v;
}

// Packed copies of the four layers L4..L7.
struct PackedWeights {
    const float* pp[4];
    const float* po[4];
};

inline size_t packed_weight_floats() {
    return ProjPack<SSLA_C1, SSLA_C2>::PACKED + ProjPack<SSLA_C2, SSLA_C2>::PACKED +
           ProjPack<SSLA_C2, SSLA_C3>::PACKED + ProjPack<SSLA_C3, SSLA_C3>::PACKED +
           OutPack<SSLA_C1, SSLA_C2>::PACKED + OutPack<SSLA_C2, SSLA_C2>::PACKED +
           OutPack<SSLA_C2, SSLA_C3>::PACKED + OutPack<SSLA_C3, SSLA_C3>::PACKED;
}

template <int IN, int OUT>
inline float* pack_layer(const LayerWeightsS2S3& L, float* dst, const float** pp, const float** po,
                         hipStream_t st) {
    constexpr int TB = 256;
    const size_t np = ProjPack<IN, OUT>::PACKED, no = OutPack<IN, OUT>::PACKED;
    hipLaunchKernelGGL((k_pack_proj<IN, OUT>), dim3((unsigned)((np + TB - 1) / TB)), dim3(TB), 0,
                       st, L.qvgIn, dst);
    *pp = dst;
    dst += np;
    hipLaunchKernelGGL((k_pack_out<IN, OUT>), dim3((unsigned)((no + TB - 1) / TB)), dim3(TB), 0,
                       st, L.goW, L.input_proj, dst);
    *po = dst;
    return dst + no;
}

// Copies for the whole-ring drain: projection as above, contraction split
// at delta boundaries.
inline size_t packed_weight_floats_d() {
    return ProjPack<SSLA_C1, SSLA_C2>::PACKED + ProjPack<SSLA_C2, SSLA_C2>::PACKED +
           ProjPack<SSLA_C2, SSLA_C3>::PACKED + ProjPack<SSLA_C3, SSLA_C3>::PACKED +
           OutPackD<SSLA_C1, SSLA_C2>::PACKED + OutPackD<SSLA_C2, SSLA_C2>::PACKED +
           OutPackD<SSLA_C2, SSLA_C3>::PACKED + OutPackD<SSLA_C3, SSLA_C3>::PACKED;
}

template <int IN, int OUT>
inline float* pack_layer_d(const LayerWeightsS2S3& L, float* dst, const float** pp,
                           const float** po, hipStream_t st) {
    constexpr int TB = 256;
    const size_t np = ProjPack<IN, OUT>::PACKED, no = OutPackD<IN, OUT>::PACKED;
    hipLaunchKernelGGL((k_pack_proj<IN, OUT>), dim3((unsigned)((np + TB - 1) / TB)), dim3(TB), 0,
                       st, L.qvgIn, dst);
    *pp = dst;
    dst += np;
    hipLaunchKernelGGL((k_pack_out_d<IN, OUT>), dim3((unsigned)((no + TB - 1) / TB)), dim3(TB),
                       0, st, L.goW, L.input_proj, dst);
    *po = dst;
    return dst + no;
}

inline hipError_t pack_weights_d(const LayerWeightsS2S3* L, float* buf, PackedWeights* out,
                                 hipStream_t st) {
    float* p = buf;
    p = pack_layer_d<SSLA_C1, SSLA_C2>(L[0], p, &out->pp[0], &out->po[0], st);
    p = pack_layer_d<SSLA_C2, SSLA_C2>(L[1], p, &out->pp[1], &out->po[1], st);
    p = pack_layer_d<SSLA_C2, SSLA_C3>(L[2], p, &out->pp[2], &out->po[2], st);
    p = pack_layer_d<SSLA_C3, SSLA_C3>(L[3], p, &out->pp[3], &out->po[3], st);
    return hipGetLastError();
}

// Fills `out` from layers L[0..3] (L4..L7) into buf (packed_weight_floats()
// floats), on stream st; returns the launch status.
inline hipError_t pack_weights(const LayerWeightsS2S3* L, float* buf, PackedWeights* out,
                               hipStream_t st) {
    float* p = buf;
    p = pack_layer<SSLA_C1, SSLA_C2>(L[0], p, &out->pp[0], &out->po[0], st);
    p = pack_layer<SSLA_C2, SSLA_C2>(L[1], p, &out->pp[1], &out->po[1], st);
    p = pack_layer<SSLA_C2, SSLA_C3>(L[2], p, &out->pp[2], &out->po[2], st);
    p = pack_layer<SSLA_C3, SSLA_C3>(L[3], p, &out->pp[3], &out->po[3], st);
    return hipGetLastError();
}

}  // namespace ssla
