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
//               when IN != OUT]  (batch and live kernels)
//   transposed contraction (OutPackT): the whole-ring drain's A operands,
//               with q recomputed from the record inputs (below)
#pragma once

#include <hip/hip_runtime.h>

#include "drain_common.h"
#include "ssla_abi.h"

namespace ssla {

constexpr int kMT = 16;       // MFMA tile rows / columns
constexpr int kKSplit = 8;    // K parts of the contraction

typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef float f32x2 __attribute__((ext_vector_type(2)));

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

// The transposed contraction of the whole-ring drain (k_outt):
//   q^T = Wq[delta]^T X^T,  Y^T = sum_delta goW[delta]^T (q^T * h^T) + input_proj^T X^T,
// with the weights as the A operands and record tiles as the columns.  Per
// layer one region holds three A-operand copies (g = lane / 16, j = lane % 16):
//   q:   items (delta, channel tile ct), groups t < KG, lane, i < 4:
//          qvgIn[delta][16 t + 4 g + i][16 ct + j]        (0 at or past IN)
//   goW: items (delta, ct, output tile ot), lane, i < 4:
//          goW[delta][16 ct + 4 g + i][16 ot + j]
//   ip:  items ot, groups t < KG, lane, i < 4 (IN != OUT only):
//          input_proj[16 t + 4 g + i][16 ot + j]          (0 at or past IN)
// Step 4 t + i of a chain pairs lane group g with input channel
// 16 t + 4 g + i instead of 4 (4 t + i) + g.  The sum over K does not depend
// on its order, and with this order a lane's B values are one float4 of a
// record's input row (q, input_proj), or the four q*h values it already holds
// in the MFMA output layout (rows 4 g .. 4 g + 3 of the q tile) for goW.
// An input of 16 t + 8 channels (IN = 24) ends in a half group: its two steps
// pair lane group g with channels 16 t + 2 g + i (i < 2), one float2 of the
// row, so no step multiplies padding (steps(t) = 2 there, else 4).
template <int IN, int OUT>
struct OutPackT {
    static constexpr bool IP = IN != OUT;
    static constexpr int NT = OUT / kMT, KG = (IN + 15) / 16;
    static constexpr bool TAIL8 = IN % 16 == 8;
    static_assert(IN % 16 == 0 || TAIL8, "input widths: multiples of 16, or of 16 plus 8");
    static __host__ __device__ constexpr int steps(int t) { return TAIL8 && t == KG - 1 ? 2 : 4; }
    // the input channel of step i of group t for lane group g
    static __host__ __device__ constexpr int kidx(int t, int g, int i) {
        return TAIL8 && t == KG - 1 ? 16 * t + 2 * g + i : 16 * t + 4 * g + i;
    }
    static constexpr size_t Q = (size_t)9 * NT * KG * 256;    // floats
    static constexpr size_t GO = (size_t)9 * NT * NT * 256;
    static constexpr size_t IPF = IP ? (size_t)NT * KG * 256 : 0;
    static constexpr size_t PACKED = Q + GO + IPF;
    static_assert(OUT % kMT == 0 && IN % 4 == 0 && (IP || IN == OUT), "tile shapes");
};

// element q of a layer's OutPackT region
template <int IN, int OUT>
__device__ __forceinline__ float outt_elem(const float* __restrict__ qvgIn,
                                           const float* __restrict__ goW,
                                           const float* __restrict__ ip, size_t q) {
    using O = OutPackT<IN, OUT>;
    const int i = (int)(q & 3), lane = (int)((q >> 2) & 63), g = lane >> 4, j = lane & 15;
    if (q < O::Q) {
        size_t r = q >> 8;
        const int t = (int)(r % O::KG);
        r /= O::KG;
        const int ct = (int)(r % O::NT), d = (int)(r / O::NT);
        const int k = O::kidx(t, g, i);
        return i < O::steps(t) && k < IN ? qvgIn[((size_t)d * IN + k) * (3 * OUT) + 16 * ct + j]
                                         : 0.f;
    }
    q -= O::Q;
    if (q < O::GO) {
        size_t r = q >> 8;
        const int ot = (int)(r % O::NT);
        r /= O::NT;
        const int ct = (int)(r % O::NT), d = (int)(r / O::NT);
        return goW[((size_t)d * OUT + 16 * ct + 4 * g + i) * OUT + 16 * ot + j];
    }
    q -= O::GO;
    const size_t r = q >> 8;
    const int t = (int)(r % O::KG), ot = (int)(r / O::KG);
    const int k = O::kidx(t, g, i);
    return i < O::steps(t) && k < IN ? ip[(size_t)k * OUT + 16 * ot + j] : 0.f;
}

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
    static constexpr size_t NO = D ? OutPackT<IN, OUT>::PACKED : OutPack<IN, OUT>::PACKED;
};

// Buffer order: L4 projection, L4 contraction, L5 ..., L7 contraction.
// D selects the transposed contraction of the whole-ring drain (OutPackT)
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
__device__ __forceinline__ float out_any(const float* qvgIn, const float* goW, const float* ip,
                                         size_t q) {
    if constexpr (D) return outt_elem<IN, OUT>(qvgIn, goW, ip, q);
    else return out_elem<IN, OUT>(goW, ip, q);
}

// Packed float q of all eight copies (q < PackLayout<D>::off[8]).
template <bool D>
__device__ __forceinline__ void pack_elem(const PackSrc& s, float* __restrict__ buf, size_t q) {
    using L = PackLayout<D>;
    float v;
    if (q < L::off[1]) v = proj_elem<SSLA_C1, SSLA_C2>(s.qvgIn[0], q);
    else if (q < L::off[2]) v = out_any<SSLA_C1, SSLA_C2, D>(s.qvgIn[0], s.goW[0], s.ip[0], q - L::off[1]);
    else if (q < L::off[3]) v = proj_elem<SSLA_C2, SSLA_C2>(s.qvgIn[1], q - L::off[2]);
    else if (q < L::off[4]) v = out_any<SSLA_C2, SSLA_C2, D>(s.qvgIn[1], s.goW[1], s.ip[1], q - L::off[3]);
    else if (q < L::off[5]) v = proj_elem<SSLA_C2, SSLA_C3>(s.qvgIn[2], q - L::off[4]);
    else if (q < L::off[6]) v = out_any<SSLA_C2, SSLA_C3, D>(s.qvgIn[2], s.goW[2], s.ip[2], q - L::off[5]);
    else if (q < L::off[7]) v = proj_elem<SSLA_C3, SSLA_C3>(s.qvgIn[3], q - L::off[6]);
    else v = out_any<SSLA_C3, SSLA_C3, D>(s.qvgIn[3], s.goW[3], s.ip[3], q - L::off[7]);
    buf[q] = v;
}

// All eight copies in one launch, one thread per packed float.
template <bool D>
__global__ void k_pack_all(PackSrc s, float* __restrict__ buf) {
    const size_t q = (size_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (q < PackLayout<D>::off[8]) pack_elem<D>(s, buf, q);
}

template <bool D>
inline size_t packed_floats() { return PackLayout<D>::off[8]; }

inline size_t packed_weight_floats() { return packed_floats<false>(); }
inline size_t packed_weight_floats_d() { return packed_floats<true>(); }

// The sources of the eight copies, and where each lands in buf.
template <bool D>
inline PackSrc pack_setup(const LayerWeightsS2S3* L, float* buf, PackedWeights* out) {
    using PL = PackLayout<D>;
    PackSrc s{};
    for (int i = 0; i < 4; ++i) {
        s.qvgIn[i] = L[i].qvgIn;
        s.goW[i] = L[i].goW;
        s.ip[i] = L[i].input_proj;
        out->pp[i] = buf + PL::off[2 * i];
        out->po[i] = buf + PL::off[2 * i + 1];
    }
    return s;
}

template <bool D>
inline hipError_t pack_all(const LayerWeightsS2S3* L, float* buf, PackedWeights* out,
                           hipStream_t st) {
    using PL = PackLayout<D>;
    const PackSrc s = pack_setup<D>(L, buf, out);
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
