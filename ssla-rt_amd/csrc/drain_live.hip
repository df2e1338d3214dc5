// drain_live.hip -- in-kernel batches of SSLA-S s2 + s3 + YOLOX head on
// gfx950: the persistent live drain and the batch-mode drain.
//
// One 512-thread workgroup owns one stream (block): its hidden state, tdrop
// counters, ring and outputs.  Records are taken in batches of up to 32 in
// ring order; each batch runs the reference's per-event schedule as a few
// workgroup-wide phases per layer:
//   tdrop   one wave, one lane per record: arrival rank among the batch's
//           records at the same cell (ssla_ref.py:190-195)
//   pairs   pair (record e, delta d) has the fixed index 9 e + d; one wave
//           sets up each record's pairs and the per-delta record lists, then
//           one thread per pair finds the next pair at its cell among the
//           later records' patches
//   P       q, v, g as 16 x 16 MFMA tiles: per delta, the records with a
//           pair there times the delta's weight columns; v and g for every
//           pair, q only for the pairs of the layer's output records
//   S       one lane per (cell, channel) walks the cell's pairs in record
//           order, loading eight pairs' g, v (and q) before the eight
//           dependent steps h = sigmoid(g) h + v; q*h where it is consumed
//   O       16 output records at a time: their nine q*h rows (and input,
//           for the residual projection) staged in LDS as one row each and
//           contracted with [goW; input_proj] by MFMA, K split four ways
//           and added in order; then fp64 LayerNorm, one wave per record
// The masks are the reference's (...celled.cuh:1027-1064): L4 all, L5 state
// for all / output for pass2, L6 pass2, L7 state for pass2 / output for
// pass3, head for owned pass3 records.  L4/L5 share one pair set, L6/L7
// another.
//
// The live kernel polls a ring in fine-grained host memory: one wave loads
// up to max_batch consecutive seq_done tags and takes the ready prefix
// (groups: member 0 decides; the other members probe a few slots
// themselves and load what they see ready before the batch word comes).
// It stops on the
// host's stop flag, on a ring overrun, or after an idle timeout on the
// constant-rate wall clock, so every wave always reaches an exit.
//
// With a profile buffer attached, thread 0 adds the wall-clock time of each
// phase (after its closing barrier) to one of SSLA_BATCH_PHASES slots.
#include <hip/hip_runtime.h>

#include <chrono>
#include <cstdint>
#include <cstring>
#include <map>
#include <mutex>
#include <thread>
#include <string>
#include <vector>

#include "drain_common.h"
#include "drain_live.h"
#include "mfma_pack.h"

namespace ssla {

struct LiveWeights {
    LayerWeightsS2S3 L[4];
    PackedWeights pk;       // MFMA fragment-order copies of the layer weights
    HeadPtrs head;
    int have_head;          // HeadKind
};

// Per-block view of the state, ring and outputs (device memory).
struct LiveDesc {
    const HybridInputRec* ring;
    unsigned long long ring_mask;       // live: capacity - 1; batch mode: ~0
    unsigned long long* tail;           // live: consumer position (host memory)
    unsigned long long* events_done;    // live: mirror of tail for monitors
    int n;                              // batch mode: records to drain
    int pad0;
    float* hidden[4];
    unsigned char* td2;
    unsigned char* td3;
    float* scratch;                     // LP rows of 3*96 floats
    HybridS2S3OutputSlot* out;          // batch mode
    float* head_out;                    // batch mode
    unsigned long long* batch_clk;      // batch mode
    float* preds;
    unsigned int* version;
    GpuTimingSlot* timing;
    unsigned int timing_mask;
    unsigned int pad1;
    unsigned long long* kstart;
    unsigned long long* kend;
    unsigned long long* clk_sync;       // live: [ping, pong] after kend, or null
    unsigned long long* prof;           // SSLA_BATCH_PHASES sums, or null
    HybridStrip strip;
    unsigned long long t0;              // live, groups: the tail at launch
};

namespace {

constexpr int LB = kLiveBatchMax;   // records per batch, at most
constexpr int kSpecTags = 8;        // ring slots a group member probes ahead of the batch word
constexpr int LT = 512;             // threads per workgroup
constexpr int NW = LT / 64;         // waves per workgroup
constexpr int LP = kPatch * LB;     // pairs per layer, at most
constexpr int NCMAX = 3 * SSLA_C3;  // widest pair row
constexpr int XS = 100;             // LDS row stride of record features (4 mod 32 banks)
constexpr int MT = kMT;             // MFMA tile rows / columns (v_mfma_f32_16x16x4_f32)
constexpr int QS = kPatch * SSLA_C3 + SSLA_C3 / 2 + 4;   // contraction row: 9*OUT q*h + IN residual
constexpr int KSPL = kKSplit;       // split of the contraction's K among waves
constexpr int NPROF = SSLA_BATCH_PHASES;

// profile slots (order of SSLA_BATCH_PHASES)
enum {
    PF_LOAD = 0, PF_TD2, PF_PAIRS2, PF_L4, PF_L5 = PF_L4 + 4, PF_TD3 = PF_L5 + 4, PF_PAIRS3,
    PF_L6, PF_L7 = PF_L6 + 4, PF_HEADH = PF_L7 + 4, PF_HEADO, PF_PREDS, PF_PUBLISH,
    PF_BATCHES, PF_RECORDS,
    PF_XWAIT                            // groups: exchange waits of L4..L7 (4 slots)
};
static_assert(PF_XWAIT + 4 <= NPROF, "profile slots");

struct alignas(16) Lds {
    float X[LB][XS];                     // layer input (becomes the layer output)
    float Y[LB][XS];                     // pre-LayerNorm sums / head cls hidden
    union {
        float QH[MT][QS];                // contraction rows of one 16-record chunk
        float R[LB][XS];                 // head reg hidden (after the last layer)
    };
    float PK[KSPL][MT][SSLA_C3];         // split-K partial sums
    float H7[LB][8];
    unsigned long long tpush[LB], temit[LB];
    int ex[LB], ey[LB];                  // coordinates at the current level
    int c2[LB], c3[LB];                  // s2 / s3 centre cell, -1 when absent
    unsigned char vld[LB], own[LB], p2[LB], p3[LB];
    int pidx[LB][kPatch];                // pair of (record, delta), or -1
    int pe[LP], pc[LP], pnext[LP], lead[LP];
    unsigned pk[LB];                     // x | y << 16 of records in the pair set, else ~0
    unsigned pbits[LB];                  // deltas of each record's pairs (bit d)
    unsigned dmask;                      // deltas of any record's pairs
    int dcnt[kPatch], dcnto[kPatch];
    int dev[kPatch][LB];                 // records with a pair at delta
    int devo[kPatch][LB];                // ... that are output records of the layer
    int ol[LB];                          // output records of the current layer
    int nlead, nout, bsize, flag, prof_on;
    unsigned long long t_pop, tprev;
    unsigned long long prof[NPROF];
};

// The workgroup's working set.  A namespace-scope LDS variable (rather than
// a parameter) keeps its address space and 16-byte alignment visible inside
// the per-batch function that both kernels call, so row reads compile to
// ds_read_b128.
__shared__ Lds g_lds;

template <class SL>
__device__ __forceinline__ void mark(SL& S, int slot) {
    if (S.prof_on && threadIdx.x == 0) {
        const unsigned long long t = (unsigned long long)wall_clock64();
        S.prof[slot] += t - S.tprev;
        S.tprev = t;
    }
}

// Wave-wide sums (all 64 lanes active) from DPP moves inside each 16-lane
// row (quad_perm xor 1, xor 2, row_half_mirror, row_mirror), a ds_swizzle
// swap of the 16-lane halves of each 32-lane group, and the two 32-lane
// group sums read from lanes 0 and 32 (wave-uniform result).
namespace dppc {
constexpr int kXor1 = 0xB1;        // quad_perm [1, 0, 3, 2]
constexpr int kXor2 = 0x4E;        // quad_perm [2, 3, 0, 1]
constexpr int kHalfMirror = 0x141; // row_half_mirror: lane i <- 7 - i in each 8
constexpr int kMirror = 0x140;     // row_mirror: lane i <- 15 - i in each 16
constexpr int kSwap16 = 0x401F;    // ds_swizzle bit mode, xor 16 within 32
}  // namespace dppc

template <int CTRL>
__device__ __forceinline__ int dpp_i(int v) {
    return __builtin_amdgcn_mov_dpp(v, CTRL, 0xF, 0xF, false);
}

template <int CTRL>
__device__ __forceinline__ float dpp_f(float v) {
    return __builtin_bit_cast(float, dpp_i<CTRL>(__builtin_bit_cast(int, v)));
}

template <int CTRL>
__device__ __forceinline__ double dpp_d(double v) {
    const unsigned long long b = __builtin_bit_cast(unsigned long long, v);
    const unsigned lo = (unsigned)dpp_i<CTRL>((int)(unsigned)b);
    const unsigned hi = (unsigned)dpp_i<CTRL>((int)(unsigned)(b >> 32));
    return __builtin_bit_cast(double, ((unsigned long long)hi << 32) | lo);
}

__device__ __forceinline__ double swap16_d(double v) {
    const unsigned long long b = __builtin_bit_cast(unsigned long long, v);
    const unsigned lo = (unsigned)__builtin_amdgcn_ds_swizzle((int)(unsigned)b, dppc::kSwap16);
    const unsigned hi = (unsigned)__builtin_amdgcn_ds_swizzle((int)(unsigned)(b >> 32), dppc::kSwap16);
    return __builtin_bit_cast(double, ((unsigned long long)hi << 32) | lo);
}

__device__ __forceinline__ double lane_d(double v, int l) {
    const unsigned long long b = __builtin_bit_cast(unsigned long long, v);
    const unsigned lo = (unsigned)__builtin_amdgcn_readlane((int)(unsigned)b, l);
    const unsigned hi = (unsigned)__builtin_amdgcn_readlane((int)(unsigned)(b >> 32), l);
    return __builtin_bit_cast(double, ((unsigned long long)hi << 32) | lo);
}

__device__ __forceinline__ double wave_sum(double v) {
    v += dpp_d<dppc::kXor1>(v);
    v += dpp_d<dppc::kXor2>(v);
    v += dpp_d<dppc::kHalfMirror>(v);
    v += dpp_d<dppc::kMirror>(v);
    v += swap16_d(v);
    return lane_d(v, 0) + lane_d(v, 32);
}

__device__ __forceinline__ float wave_sumf(float v) {
    v += dpp_f<dppc::kXor1>(v);
    v += dpp_f<dppc::kXor2>(v);
    v += dpp_f<dppc::kHalfMirror>(v);
    v += dpp_f<dppc::kMirror>(v);
    v += __builtin_bit_cast(float, __builtin_amdgcn_ds_swizzle(__builtin_bit_cast(int, v), dppc::kSwap16));
    return __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, v), 0)) +
           __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, v), 32));
}

// A float4 of an LDS row: x is 16-byte aligned and `at` a multiple of 4.
// Arrival-rank tdrop for one batch (wave 0; lane = record).  All lanes read
// the counter in one load before the last record of each cell stores the
// advanced value.
// In two parts, so that other wave-0 work can run while the counters load:
// tdrop_begin (every lane of wave 0) ranks the records and issues the
// counter loads, tdrop_end sets the pass flags and stores the counters.
struct TdropLane {
    int c;
    unsigned rank, cnt;
    bool live, last;
};

__device__ __forceinline__ TdropLane tdrop_begin(int B, const unsigned char* td, const int* cell,
                                                 const unsigned char* mask) {
    const int e = threadIdx.x;
    TdropLane r;
    // lane j's cell when record j is live, else -1; the other lanes' keys
    // are read from registers (the whole wave runs the loop)
    r.c = e < B ? cell[e] : -1;
    r.live = r.c >= 0 && (mask == nullptr || mask[e]);
    const int key = r.live ? r.c : -1;
    r.rank = 0;
    r.last = true;
    for (int j = 0; j < B; ++j) {
        const bool lj = __builtin_amdgcn_readlane(key, j) == key;
        if (lj && j < e) ++r.rank;
        if (lj && j > e) r.last = false;
    }
    r.cnt = r.live ? (unsigned)gmem(td)[r.c] : 0u;
    return r;
}

__device__ __forceinline__ void tdrop_end(int B, unsigned char* td, unsigned char* pass, int window,
                                          const TdropLane& r) {
    const int e = threadIdx.x;
    if (e >= B) return;
    if (!r.live) {
        pass[e] = 0;
        return;
    }
    const unsigned pre = (r.cnt + r.rank) & 255u;
    pass[e] = (window <= 1 || pre % (unsigned)window == 0u) ? 1 : 0;
    if (r.last) gmem(td)[r.c] = (unsigned char)((r.cnt + r.rank + 1u) & 255u);
}

template <class SL>
__device__ __forceinline__ void batch_tdrop(SL& S, int B, unsigned char* td, const int* cell,
                            const unsigned char* mask, unsigned char* pass, int window) {
    if (threadIdx.x >= 64) return;
    const TdropLane r = tdrop_begin(B, td, cell, mask);
    tdrop_end(B, td, pass, window, r);
}

// (record, delta) pairs of the records in `set` on an Hl x Wl grid.  Pair
// (e, d) -- record e and the cell (ey + 1 - d / 3, ex + 1 - d % 3) of its
// 3x3 patch -- has the fixed index e * 9 + d; pidx[e][d] is that index, or
// -1 when e is not in the set or the cell is off the grid, and pbits[e] the
// mask of e's pairs (dmask: of every record's).  LISTS: per-delta lists of
// the records with a pair there (dev, dcnt).  Then one thread per pair: its
// record and cell, its successor at the cell (the pair of the first later
// record of the set whose patch holds the cell) and whether it leads the
// cell (no earlier record's patch holds it).  pairs_wave0: the per-record
// part (wave 0, every lane).
template <class SL, bool LISTS>
__device__ __forceinline__ void pairs_wave0(SL& S, int B, const unsigned char* set, int Hl, int Wl) {
    const int e = threadIdx.x;
    const bool in = e < B && set[e];
    const int ex = in ? S.ex[e] : 0, ey = in ? S.ey[e] : 0;
    unsigned bits = 0;
    if (in) {
        #pragma unroll
        for (int d = 0; d < kPatch; ++d) {
            const int ty = ey + 1 - d / 3, tx = ex + 1 - d % 3;
            if (ty >= 0 && ty < Hl && tx >= 0 && tx < Wl) bits |= 1u << d;
        }
    }
    if (e == 0) {
        S.dmask = 0u;
        S.nlead = 0;
    }
    if (e < LB) {
        S.pbits[e] = bits;
        S.pk[e] = in ? ((unsigned)ex | ((unsigned)ey << 16)) : 0xffffffffu;
        #pragma unroll
        for (int d = 0; d < kPatch; ++d) S.pidx[e][d] = ((bits >> d) & 1u) ? e * kPatch + d : -1;
    }
    if (bits) atomicOr(&S.dmask, bits);   // after lane 0's store: one wave, LDS order
    if constexpr (LISTS) {
        const unsigned long long lt = (1ull << e) - 1ull;
        #pragma unroll
        for (int d = 0; d < kPatch; ++d) {
            const bool has = (bits >> d) & 1u;
            const unsigned long long bal = __ballot(has);
            if (has) S.dev[d][__popcll(bal & lt)] = e;
            if (e == 0) S.dcnt[d] = __popcll(bal);
        }
    }
}

// The pairs' records, cells, successors and leads (after pairs_wave0 and a
// barrier); O(B) per pair.  Ends with a barrier.
template <class SL>
__device__ __forceinline__ void pairs_links(SL& S, int B, int Wl) {
    const int tid = threadIdx.x;
    for (int p = tid; p < kPatch * B; p += LT) {
        const int e = p / kPatch, d = p - e * kPatch;
        if (!((S.pbits[e] >> d) & 1u)) continue;
        const unsigned ke = S.pk[e];
        const int tx = (int)(ke & 0xffffu) + 1 - d % 3, ty = (int)(ke >> 16) + 1 - d / 3;
        S.pe[p] = e;
        S.pc[p] = ty * Wl + tx;
        int nx = -1;
        bool lead = true;
        for (int j = 0; j < B; ++j) {
            const unsigned k = S.pk[j];
            const int dx = tx - (int)(k & 0xffffu), dy = ty - (int)(k >> 16);
            if (k == 0xffffffffu || dx < -1 || dx > 1 || dy < -1 || dy > 1) continue;
            if (j < e) lead = false;
            else if (j > e && nx < 0) nx = j * kPatch + (1 - dy) * 3 + (1 - dx);
        }
        S.pnext[p] = nx;
        if (lead) S.lead[atomicAdd(&S.nlead, 1)] = p;
    }
    __syncthreads();
}

template <class SL, bool LISTS = true>
__device__ __forceinline__ void build_pairs(SL& S, int B, const unsigned char* set, int Hl, int Wl) {
    if (threadIdx.x < 64) pairs_wave0<SL, LISTS>(S, B, set, Hl, Wl);
    __syncthreads();
    pairs_links(S, B, Wl);
}

// P: scratch[pair][0, 3*OUT) = [q | v | g] of the pair's (record, delta),
// as 16 x 16 MFMA tiles (v_mfma_f32_16x16x4_f32): per delta, the records
// with a pair there (rows) times the delta's weight columns.  v and g
// columns take every pair at delta; q columns only the pairs of output
// records (S.devo), the only ones whose q is consumed.  Each wave owns
// whole (delta, column tile) items and keeps the tile's IN x 16 weights in
// registers across its row tiles, and loads its next item's weights while
// the current item runs.
//   A operand: lane (i, k) = (lane % 16, lane / 16) holds row i, k
//   B operand: lane holds column i, k;  D: lane holds rows 4k..4k+3, column i
template <int IN, int OUT>
struct ProjTile : ProjPack<IN, OUT> {
    using ProjPack<IN, OUT>::T;
    using ProjPack<IN, OUT>::TQ;
    using ProjPack<IN, OUT>::KS;
    using ProjPack<IN, OUT>::NC;
    static __device__ __forceinline__ void run(Lds& S, int it, int li, int lk, const float* b,
                                               float* __restrict__ scratch) {
        const int d = it / T, t = it - d * T;
        const bool qt = t < TQ;
        const int n = qt ? S.dcnto[d] : S.dcnt[d];
        const int* list = qt ? S.devo[d] : S.dev[d];
        const int col = t * MT + li;
        const float* X = &S.X[0][0];
        for (int m0 = 0; m0 < n; m0 += MT) {
            const int xr = list[min(m0 + li, n - 1)] * XS + lk;
            f32x4 acc = {0.f, 0.f, 0.f, 0.f};
            #pragma unroll
            for (int s = 0; s < KS; ++s)
                acc = __builtin_amdgcn_mfma_f32_16x16x4f32(X[xr + s * 4], b[s], acc, 0, 0, 0);
            #pragma unroll
            for (int r = 0; r < 4; ++r) {
                const int rr = m0 + 4 * lk + r;
                if (rr < n) gstore(scratch + (size_t)S.pidx[list[rr]][d] * NC + col, acc[r]);
            }
        }
    }
};

template <int IN, int OUT>
__device__ __forceinline__ void phase_proj(Lds& S, const float* __restrict__ pp,
                                           float* __restrict__ scratch) {
    using P = ProjTile<IN, OUT>;
    static_assert(OUT % MT == 0 && IN % 4 == 0, "tile shapes");
    const int lane = threadIdx.x & 63, wv = threadIdx.x >> 6;
    const int li = lane & 15, lk = lane >> 4;
    // two items in flight per wave: the next item's weights load while the
    // current item's tiles run
    float b0[P::KS4 * 4], b1[P::KS4 * 4];
    int it = wv;
    if (it < P::N) P::load(pp, it, lane, b0);
    while (it < P::N) {
        const int i1 = it + NW, i2 = i1 + NW;
        if (i1 < P::N) P::load(pp, i1, lane, b1);
        P::run(S, it, li, lk, b0, scratch);
        if (i1 >= P::N) break;
        if (i2 < P::N) P::load(pp, i2, lane, b0);
        P::run(S, i1, li, lk, b1, scratch);
        it = i2;
    }
}

// S: the per-cell recurrence in record order; q*h replaces q for pairs of
// output records (outm == nullptr: every record of the set).
template <int OUT>
__device__ __forceinline__ void phase_recur(Lds& S, float* __restrict__ hidden,
                                            float* __restrict__ scratch, const unsigned char* outm) {
    constexpr int NC = 3 * OUT;
    constexpr int CH = 8;
    const int nl = S.nlead;
    for (int t = threadIdx.x; t < nl * OUT; t += LT) {
        const int k = t / OUT, ch = t - k * OUT;
        int q = S.lead[k];
        float* hp = hidden + (size_t)S.pc[q] * OUT + ch;
        float h = gload(hp);
        while (q >= 0) {
            int qs[CH];
            #pragma unroll
            for (int j = 0; j < CH; ++j) {
                qs[j] = q;
                if (q >= 0) q = S.pnext[q];
            }
            float gv[CH], vv[CH], qv[CH];
            bool ov[CH];
            #pragma unroll
            for (int j = 0; j < CH; ++j) {
                const int p = qs[j] < 0 ? 0 : qs[j];      // pair 0 exists: loads stay in bounds
                const float* row = scratch + (size_t)p * NC;
                ov[j] = qs[j] >= 0 && (outm == nullptr || outm[S.pe[p]]);
                gv[j] = gload(row + 2 * OUT + ch);
                vv[j] = gload(row + OUT + ch);
                qv[j] = gload(row + ch);
            }
            #pragma unroll
            for (int j = 0; j < CH; ++j) {
                if (qs[j] >= 0) {
                    h = fmaf(sigmoid_fast(gv[j]), h, vv[j]);
                    if (ov[j]) gstore(scratch + (size_t)qs[j] * NC + ch, qv[j] * h);
                }
            }
        }
        gstore(hp, h);
    }
}

// One (column tile, K part) item of the contraction below: B operand loads
// (the part's weights, one register per 4-row step) and the MFMA chain over
// the staged rows, leaving the partial tile in S.PK[part].
template <int IN, int OUT>
struct OutTile : OutPack<IN, OUT> {
    using OutPack<IN, OUT>::SPER;
    using OutPack<IN, OUT>::STEPS;
    static __device__ __forceinline__ void run(Lds& S, int it, int li, int lk, const float* b) {
        const int nt = it / KSPL, ks = it - nt * KSPL;
        const int col = nt * MT + li;
        f32x4 acc = {0.f, 0.f, 0.f, 0.f};
        #pragma unroll
        for (int j = 0; j < SPER; ++j) {
            const int s = min(ks * SPER + j, STEPS - 1);  // past the end b is 0
            acc = __builtin_amdgcn_mfma_f32_16x16x4f32(S.QH[li][s * 4 + lk], b[j], acc, 0, 0, 0);
        }
        #pragma unroll
        for (int r = 0; r < 4; ++r) S.PK[ks][4 * lk + r][col] = acc[r];
    }
};

// O: Y[e] = sum_delta goW[delta]^T qh(e, delta) + residual for the output
// records S.ol[0, S.nout), 16 records at a time, as one MFMA contraction
// over K = 9*OUT (+ IN): each record's row holds its nine q*h rows (zeros
// where the patch cell is out of bounds) and, with input_proj, its input;
// B is goW (9*OUT x OUT, delta-major) followed by input_proj.  Waves own
// (column tile, K part) items with the part's weights in registers; the
// parts are added in order.
template <int IN, int OUT>
__device__ __forceinline__ void phase_out(Lds& S, const float* __restrict__ po,
                                          const float* __restrict__ scratch) {
    using O = OutTile<IN, OUT>;
    constexpr int NC = 3 * OUT;
    static_assert(O::KT <= QS, "contraction row");
    const int tid = threadIdx.x, lane = tid & 63, wv = tid >> 6;
    const int li = lane & 15, lk = lane >> 4;
    const int no = S.nout;
    for (int c0 = 0; c0 < no; c0 += MT) {
        const int m = min(MT, no - c0);
        for (int t = tid; t < MT * O::KT; t += LT) {
            const int r = t / O::KT, k = t - r * O::KT;
            float v = 0.f;
            if (r < m) {
                const int e = S.ol[c0 + r];
                if (k < O::KQ) {
                    const int d = k / OUT, i = k - d * OUT;
                    const int p = S.pidx[e][d];
                    if (p >= 0) v = gload(scratch + (size_t)p * NC + i);
                } else {
                    v = S.X[e][k - O::KQ];
                }
            }
            S.QH[r][k] = v;
        }
        __syncthreads();
        float b0[O::SP4 * 4], b1[O::SP4 * 4];
        int it = wv;
        if (it < O::N) O::load(po, it, lane, b0);
        while (it < O::N) {
            const int i1 = it + NW, i2 = i1 + NW;
            if (i1 < O::N) O::load(po, i1, lane, b1);
            O::run(S, it, li, lk, b0);
            if (i1 >= O::N) break;
            if (i2 < O::N) O::load(po, i2, lane, b0);
            O::run(S, i1, li, lk, b1);
            it = i2;
        }
        __syncthreads();
        for (int t = tid; t < m * OUT; t += LT) {
            const int r = t / OUT, jj = t - r * OUT;
            const int e = S.ol[c0 + r];
            float a = 0.f;
            #pragma unroll
            for (int ks = 0; ks < KSPL; ++ks) a += S.PK[ks][r][jj];
            S.Y[e][jj] = O::IP ? a : a + S.X[e][jj];
        }
        __syncthreads();
    }
}

// One layer over the pairs built for `set`; output (LayerNormed, in S.X) for
// the records of set and outm (outm == nullptr: all of set).
template <int IN, int OUT>
__device__ __forceinline__ void batch_layer(Lds& S, int B, const unsigned char* set, const unsigned char* outm,
                            const LayerWeightsS2S3& L, const float* pp, const float* po,
                            float* __restrict__ hidden, float* __restrict__ scratch, int slot) {
    const int tid = threadIdx.x;
    if (tid < 64) {
        const bool o = tid < B && set[tid] && (outm == nullptr || outm[tid]);
        const unsigned long long lt = (1ull << tid) - 1ull;
        const unsigned long long bal = __ballot(o);
        if (o) S.ol[__popcll(bal & lt)] = tid;
        if (tid == 0) S.nout = __popcll(bal);
        #pragma unroll
        for (int d = 0; d < kPatch; ++d) {
            const bool has = o && S.pidx[tid][d] >= 0;
            const unsigned long long bd = __ballot(has);
            if (has) S.devo[d][__popcll(bd & lt)] = tid;
            if (tid == 0) S.dcnto[d] = __popcll(bd);
        }
    }
    __syncthreads();
    phase_proj<IN, OUT>(S, pp, scratch);
    __syncthreads();
    mark(S, slot + 0);
    phase_recur<OUT>(S, hidden, scratch, outm);
    __syncthreads();
    mark(S, slot + 1);
    phase_out<IN, OUT>(S, po, scratch);
    mark(S, slot + 2);
    // fp64 LayerNorm, one wave per output record
    const int wv = tid >> 6, lane = tid & 63, no = S.nout;
    for (int r = wv; r < no; r += NW) {
        const int e = S.ol[r];
        const float a = lane < OUT ? S.Y[e][lane] : 0.f;
        const float b = lane + 64 < OUT ? S.Y[e][lane + 64] : 0.f;
        const double mean = wave_sum((double)a + (double)b) / (double)OUT;
        const double da = lane < OUT ? (double)a - mean : 0.0;
        const double db = lane + 64 < OUT ? (double)b - mean : 0.0;
        const double var = wave_sum(da * da + db * db) / (double)OUT;
        const double inv = 1.0 / sqrt(var + 1e-5);
        if (lane < OUT)
            S.X[e][lane] = (float)(da * inv * (double)L.ln_gamma[lane] + (double)L.ln_beta[lane]);
        if (lane + 64 < OUT)
            S.X[e][lane + 64] = (float)(db * inv * (double)L.ln_gamma[lane + 64] + (double)L.ln_beta[lane + 64]);
    }
    __syncthreads();
    mark(S, slot + 3);
}

// Two-branch YOLOX head of the nh records listed in S.ol: hidden layers
// y = SiLU(W x + b) of both branches (one thread per weight column), then
// the seven outputs [reg0..3, obj, cls0, cls1] (one wave per record).
// The two-branch head of the batch's nh output records (indices in S.ol).
// Hidden layers y = SiLU(W x + b) of both branches as 16 x 16 x 4 MFMA tiles
// over all waves: items (row tile of 16 records, branch, 32 output
// channels as two 16-column tiles), A = the records' features (LDS), B =
// the (IN, OUT) row-major weights read straight from memory (lane (li, lk)
// takes row 4 s + lk, column li of step s).  Six items per row tile, so a
// wave's weights arrive in one load round.  Then the seven outputs, one
// wave per record, with the output weights of the lane's channels loaded
// before the hidden layers.
template <class SL>
__device__ __forceinline__ void batch_head_yolox(SL& S, int nh, const LiveWeights& W) {
    constexpr int C = SSLA_C3, KS = C / 4, NT = C / (2 * MT);
    const int tid = threadIdx.x, wv = tid >> 6, lane = tid & 63, li = lane & 15, lk = lane >> 4;
    float wo[2][7];
    #pragma unroll
    for (int h = 0; h < 2; ++h) {
        const int i = lane + 64 * h;
        const bool in = i < C;
        #pragma unroll
        for (int k = 0; k < 4; ++k) wo[h][k] = in ? W.head.reg_pred_W[(size_t)i * 4 + k] : 0.f;
        wo[h][4] = in ? W.head.obj_pred_W[i] : 0.f;
        wo[h][5] = in ? W.head.cls_pred_W[(size_t)i * 2 + 0] : 0.f;
        wo[h][6] = in ? W.head.cls_pred_W[(size_t)i * 2 + 1] : 0.f;
    }
    const int nit = ((nh + MT - 1) / MT) * 2 * NT;
    for (int it = wv; it < nit; it += NW) {
        const int mt = it / (2 * NT), rem = it - mt * 2 * NT, br = rem / NT, ot = rem - br * NT;
        const float* Wb = (br == 0 ? W.head.cls_conv_W : W.head.reg_conv_W) + 2 * ot * MT + li;
        const float* bb = (br == 0 ? W.head.cls_conv_b : W.head.reg_conv_b) + 2 * ot * MT + li;
        float b0[KS], b1[KS];
        #pragma unroll
        for (int s = 0; s < KS; ++s) {
            b0[s] = Wb[(size_t)(4 * s + lk) * C];
            b1[s] = Wb[(size_t)(4 * s + lk) * C + MT];
        }
        const float bias0 = bb[0], bias1 = bb[MT];
        const float* xa = &S.X[S.ol[min(mt * MT + li, nh - 1)]][lk];
        f32x4 a0 = {0.f, 0.f, 0.f, 0.f}, a1 = a0;
        #pragma unroll
        for (int s = 0; s < KS; ++s) {
            const float x = xa[4 * s];
            a0 = __builtin_amdgcn_mfma_f32_16x16x4f32(x, b0[s], a0, 0, 0, 0);
            a1 = __builtin_amdgcn_mfma_f32_16x16x4f32(x, b1[s], a1, 0, 0, 0);
        }
        // D: lane (li, lk) holds records 4 lk .. 4 lk + 3 of the tile, channel li
        const int c0 = 2 * ot * MT + li, c1 = c0 + MT;
        #pragma unroll
        for (int q = 0; q < 4; ++q) {
            const int r = mt * MT + 4 * lk + q;
            if (r < nh) {
                const int e = S.ol[r];
                const float y0 = a0[q] + bias0, y1 = a1[q] + bias1;
                const float v0 = y0 * sigmoid_fast(y0), v1 = y1 * sigmoid_fast(y1);
                if (br == 0) {
                    S.Y[e][c0] = v0;
                    S.Y[e][c1] = v1;
                } else {
                    S.R[e][c0] = v0;
                    S.R[e][c1] = v1;
                }
            }
        }
    }
    __syncthreads();
    mark(S, PF_HEADH);
    for (int r = wv; r < nh; r += NW) {
        const int e = S.ol[r];
        float part[7] = {0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f};
        #pragma unroll
        for (int h = 0; h < 2; ++h) {
            const int i = lane + 64 * h;
            if (i < C) {
                const float yr = S.R[e][i], yc = S.Y[e][i];
                #pragma unroll
                for (int k = 0; k < 5; ++k) part[k] = fmaf(wo[h][k], yr, part[k]);
                part[5] = fmaf(wo[h][5], yc, part[5]);
                part[6] = fmaf(wo[h][6], yc, part[6]);
            }
        }
        #pragma unroll
        for (int k = 0; k < 7; ++k) part[k] = wave_sumf(part[k]);
        if (lane == 0) {
            #pragma unroll
            for (int k = 0; k < 4; ++k) S.H7[e][k] = part[k] + W.head.reg_pred_b[k];
            S.H7[e][4] = part[4] + W.head.obj_pred_b[0];
            S.H7[e][5] = part[5] + W.head.cls_pred_b[0];
            S.H7[e][6] = part[6] + W.head.cls_pred_b[1];
        }
    }
    __syncthreads();
    mark(S, PF_HEADO);
}

// Head of the owned pass-3 records and the prediction grid.  Two-branch
// YOLOX head: hidden layers y = SiLU(W x + b) of both branches (one thread
// per weight column), then the seven outputs [reg0..3, obj, cls0, cls1]
// (one wave per record).  Single-linear head (...celled.cuh:1476-1481):
// raw7 = head_W^T x + head_b, one wave per record.
// Prediction-grid write of thread tid's record: the last owned pass-3
// record of each s3 cell writes its cell (version += the cell's owned
// pass-3 records of the batch).  The cell's current version comes from
// `vsh`, a device-memory copy of the block's version words that only this
// workgroup reads and writes (the device is the words' only writer), or,
// without one, from the version word itself (host memory) -- read here,
// ahead of the head.
struct PredPlan {
    int cell = -1;
    unsigned count = 0, old = 0;
};

template <class SL>
__device__ __forceinline__ PredPlan pred_plan(SL& S, int B, const LiveDesc& d,
                                              unsigned* vsh = nullptr) {
    PredPlan p;
    const int tid = threadIdx.x;
    if (tid >= 64) return p;
    // lane j's s3 cell when record j is an owned pass-3 record, else -1
    // (the whole wave runs the loop; other lanes' keys come from registers)
    const bool mine = tid < B && S.own[tid] && S.p3[tid];
    const int key = mine ? S.c3[tid] : -1;
    int count = 0;
    bool last = true;
    for (int j = 0; j < B; ++j) {
        const bool same = __builtin_amdgcn_readlane(key, j) == key;
        count += same ? 1 : 0;
        if (same && j > tid) last = false;
    }
    if (mine) {
        const int e = tid;
        const HybridStrip& s = d.strip;
        const int hx = S.ex[e] - s.s3_owned_lo, hy = S.ey[e] - s.s3_owned_y_lo;
        const int w = s.s3_owned_hi - s.s3_owned_lo, h = s.s3_owned_y_hi - s.s3_owned_y_lo;
        if (last && hx >= 0 && hx < w && hy >= 0 && hy < h) {
            p.cell = hy * w + hx;
            p.count = (unsigned)count;
            if (vsh) {
                p.old = gmem(vsh)[p.cell];
                gmem(vsh)[p.cell] = (p.old + p.count) & ~kPredBusy;
            } else {
                p.old = pred_version(d.version ? d.version + p.cell : nullptr);
            }
        }
    }
    return p;
}

template <class SL>
__device__ __forceinline__ void batch_head(SL& S, int B, const LiveDesc& d, const LiveWeights& W,
                                           const PredPlan* plan = nullptr) {
    constexpr int C = SSLA_C3;
    const int tid = threadIdx.x;
    if (tid < 64) {
        const bool o = tid < B && S.own[tid] && S.p3[tid];
        const unsigned long long bal = __ballot(o);
        if (o) S.ol[__popcll(bal & ((1ull << tid) - 1ull))] = tid;
        if (tid == 0) S.nout = __popcll(bal);
    }
    const PredPlan pp = plan ? *plan : pred_plan(S, B, d);
    __syncthreads();
    const int nh = S.nout;
    if (nh == 0) return;                // no head rows and no prediction cell
    if (W.have_head == kHeadLinear) {
        const int wv = tid >> 6, lane = tid & 63;
        for (int r = wv; r < nh; r += NW) {
            const int e = S.ol[r];
            float part[7] = {0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f};
            for (int i = lane; i < C; i += 64) {
                const float x = S.X[e][i];
                #pragma unroll
                for (int k = 0; k < 7; ++k) part[k] = fmaf(W.head.lin_W[(size_t)i * 7 + k], x, part[k]);
            }
            #pragma unroll
            for (int k = 0; k < 7; ++k) part[k] = wave_sumf(part[k]);
            if (lane == 0) {
                #pragma unroll
                for (int k = 0; k < 7; ++k) S.H7[e][k] = part[k] + W.head.lin_b[k];
            }
        }
        __syncthreads();
        mark(S, PF_HEADO);
    } else {
        batch_head_yolox(S, nh, W);
    }

    if (pp.cell >= 0)
        publish_pred_at(d.preds ? d.preds + (size_t)pp.cell * 7 : nullptr,
                        d.version ? d.version + pp.cell : nullptr, S.H7[tid], pp.count, pp.old);
    __syncthreads();
    mark(S, PF_PREDS);
}

// Records [0, B) are in S (X rows, coordinates, ownership).  Runs both
// stages, the tdrop gates and the head; leaves L7 outputs in S.X and head
// rows in S.H7.
__device__ __noinline__ void process_batch(int B, const LiveDesc& d, const LiveWeights& W,
                                          const Geometry& G) {
    Lds& S = g_lds;
    const int tid = threadIdx.x;
    batch_tdrop(S, B, d.td2, S.c2, nullptr, S.p2, G.window);
    __syncthreads();
    mark(S, PF_TD2);
    build_pairs(S, B, S.vld, G.H2, G.W2);
    mark(S, PF_PAIRS2);
    batch_layer<SSLA_C1, SSLA_C2>(S, B, S.vld, nullptr, W.L[0], W.pk.pp[0], W.pk.po[0], d.hidden[0], d.scratch, PF_L4);
    batch_layer<SSLA_C2, SSLA_C2>(S, B, S.vld, S.p2, W.L[1], W.pk.pp[1], W.pk.po[1], d.hidden[1], d.scratch, PF_L5);
    if (tid < B) {                      // pool to s3
        S.ex[tid] >>= 1;
        S.ey[tid] >>= 1;
        S.c3[tid] = S.vld[tid] ? S.ey[tid] * G.W3 + S.ex[tid] : -1;
    }
    __syncthreads();
    batch_tdrop(S, B, d.td3, S.c3, S.p2, S.p3, G.window);
    __syncthreads();
    mark(S, PF_TD3);
    build_pairs(S, B, S.p2, G.H3, G.W3);
    mark(S, PF_PAIRS3);
    batch_layer<SSLA_C2, SSLA_C3>(S, B, S.p2, nullptr, W.L[2], W.pk.pp[2], W.pk.po[2], d.hidden[2], d.scratch, PF_L6);
    batch_layer<SSLA_C3, SSLA_C3>(S, B, S.p2, S.p3, W.L[3], W.pk.pp[3], W.pk.po[3], d.hidden[3], d.scratch, PF_L7);
    if (W.have_head) batch_head(S, B, d, W);
}

template <class SL>
__device__ __forceinline__ void prof_begin(SL& S, const LiveDesc& d) {
    if (threadIdx.x == 0) {
        S.prof_on = d.prof != nullptr;
        for (int k = 0; k < NPROF; ++k) S.prof[k] = 0;
    }
}

// The profile slots stage B of a two-stage group fills (its member 0 writes
// them; stage A's member 0 writes the others).
__device__ __forceinline__ bool prof_stage_b(int k) {
    return (k >= PF_TD3 && k <= PF_PUBLISH) || k == PF_XWAIT + 2 || k == PF_XWAIT + 3;
}

// stage: -1 every slot, 0 / 1 the slots of stage A / B of a two-stage group
template <class SL>
__device__ __forceinline__ void prof_end(SL& S, const LiveDesc& d, int stage = -1) {
    if (threadIdx.x == 0 && d.prof)
        for (int k = 0; k < NPROF; ++k)
            if (stage < 0 || (stage == 1) == prof_stage_b(k)) gmem(d.prof)[k] = S.prof[k];
}

// Clock handshake with the host (live kernels, poll wave lane 0): when the
// host's ping word (a sequence number) changes, answer in the pong word
// with (wall clock << 8) | (sequence & 0xff), one 64-bit store, so the host
// can bracket a GPU clock reading between its own clock readings.
__device__ __forceinline__ void clock_sync(unsigned long long* cs, unsigned long long& last) {
    if (!cs) return;
    const unsigned long long ping = __hip_atomic_load(gmem(cs), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_SYSTEM);
    if (ping != last) {
        const unsigned long long now = (unsigned long long)wall_clock64();
        __hip_atomic_store(gmem(cs + 1), (now << 8) | (ping & 0xffull), __ATOMIC_RELAXED,
                           __HIP_MEMORY_SCOPE_SYSTEM);
        last = ping;
    }
}


// Loads records e0..B-1 of the batch at ring slot `first` (slots wrap with
// `mask`):
// eight threads per record, each reading one 16-byte piece of it (the ring
// is fine-grained host memory, where every load is a PCIe read request:
// 8 per record instead of 30 separate 4- and 8-byte ones).  Piece 0 holds
// the tag, t and the s2 coordinates, pieces 1..6 feat1, piece 7 the two
// timestamps.
template <class SL>
__device__ __forceinline__ void load_batch(SL& S, int B, const HybridInputRec* ring, unsigned long long first,
                           unsigned long long mask, const HybridStrip& s, const Geometry& G,
                           int e0 = 0) {
    static_assert(sizeof(HybridInputRec) == 128, "eight 16-byte pieces per record");
    const int tid = threadIdx.x;
    if (tid < (B - e0) * 8) {
        const int e = e0 + (tid >> 3), q = tid & 7;
        typedef unsigned u32x4 __attribute__((ext_vector_type(4)));
        const u32x4 v = gmem(reinterpret_cast<const u32x4*>(&ring[(first + e) & mask]))[q];
        if (q >= 1 && q <= 6) {
            *reinterpret_cast<float4*>(&S.X[e][4 * (q - 1)]) =
                make_float4(__uint_as_float(v.x), __uint_as_float(v.y), __uint_as_float(v.z),
                            __uint_as_float(v.w));
        } else if (q == 0) {
            const int x = (int)(v.w & 0xffffu), y = (int)(v.w >> 16);    // bytes 12..15
            const bool ok = x < G.W2 && y < G.H2;
            S.vld[e] = ok ? 1 : 0;
            S.ex[e] = x;
            S.ey[e] = y;
            S.c2[e] = ok ? y * G.W2 + x : -1;
            S.own[e] = (ok && x >= s.owned_lo && x < s.owned_hi && y >= s.owned_y_lo &&
                        y < s.owned_y_hi) ? 1 : 0;
            S.p2[e] = 0;
            S.p3[e] = 0;
        } else {
            S.tpush[e] = (unsigned long long)v.x | ((unsigned long long)v.y << 32);
            S.temit[e] = (unsigned long long)v.z | ((unsigned long long)v.w << 32);
        }
    }
}


// ---------------------------------------------------------------------------
// batch-mode drain of pre-filled rings (one workgroup per block)
// ---------------------------------------------------------------------------
__global__ void __launch_bounds__(LT)
k_batch_drain(const LiveDesc* __restrict__ ld, LiveWeights W, Geometry G, int batch) {
    Lds& S = g_lds;
    const LiveDesc& d = ld[blockIdx.x];
    const int tid = threadIdx.x;
    prof_begin(S, d);
    int bi = 0;
    for (int base = 0; base < d.n; base += batch, ++bi) {
        const int B = min(batch, d.n - base);
        if (tid == 0) {
            S.t_pop = (unsigned long long)wall_clock64();
            S.tprev = S.t_pop;
        }
        load_batch(S, B, d.ring, (unsigned long long)base, ~0ull, d.strip, G);
        __syncthreads();
        mark(S, PF_LOAD);
        process_batch(B, d, W, G);
        // output slots and head rows
        for (int t = tid; t < B * SSLA_C3; t += LT) {
            const int e = t / SSLA_C3, i = t % SSLA_C3;
            if (d.out) gmem(d.out)[base + e].s3_feat[i] = (S.vld[e] && S.p3[e]) ? S.X[e][i] : 0.f;
        }
        if (tid < B) {
            const int e = tid;
            const bool v = S.vld[e], own = S.own[e];
            if (d.out) {
                gmem(d.out)[base + e].pass2 = !v ? -2 : (own ? (int)S.p2[e] : -1);
                gmem(d.out)[base + e].pass3 = !v ? -2 : (own ? (int)S.p3[e] : -1);
            }
            if (d.head_out) {
                const bool hv = W.have_head && own && S.p3[e];
                #pragma unroll
                for (int k = 0; k < 7; ++k) gmem(d.head_out)[(size_t)(base + e) * 7 + k] = hv ? S.H7[e][k] : 0.f;
            }
        }
        if (tid == 0 && d.batch_clk) {
            gmem(d.batch_clk)[(size_t)bi * 2 + 0] = S.t_pop;
            gmem(d.batch_clk)[(size_t)bi * 2 + 1] = (unsigned long long)wall_clock64();
        }
        __syncthreads();
        mark(S, PF_PUBLISH);
        if (tid == 0) {
            S.prof[PF_BATCHES] += 1;
            S.prof[PF_RECORDS] += (unsigned long long)B;
        }
    }
    prof_end(S, d);
}

// ---------------------------------------------------------------------------
// persistent live drain
// ---------------------------------------------------------------------------
__global__ void __launch_bounds__(LT)
k_live(const LiveDesc* __restrict__ ld, LiveWeights W, Geometry G, const int* stop_flag,
       unsigned int spin_ns, unsigned long long idle_ticks, int max_batch,
       int* __restrict__ status) {
    Lds& S = g_lds;
    const LiveDesc& d = ld[blockIdx.x];
    const int tid = threadIdx.x;
    prof_begin(S, d);
    const unsigned long long mask = d.ring_mask;
    unsigned long long t = __hip_atomic_load(gmem(d.tail), __ATOMIC_ACQUIRE, __HIP_MEMORY_SCOPE_SYSTEM);
    unsigned long long last_work = (unsigned long long)wall_clock64();
    // The host pairs the kernel's start and end clocks with its own clock at
    // the moment it sees them, so they are stored relaxed: a release would
    // first write back the L2, and the host would see the value late by as
    // much as that takes (tens of microseconds at the end of a run).
    if (tid == 0 && d.kstart)
        __hip_atomic_store(gmem(d.kstart), last_work, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_SYSTEM);
    const int sleep_iters = (int)(spin_ns / 40u) + 1;
    unsigned long long ping_seen = 0;
    while (true) {
        // every wave has read the previous round's flag / batch size
        __syncthreads();
        // ---- poll: wave 0 probes 64 consecutive tags ------------------------------
        if (tid < 64) {
            SSLA_GLOBAL unsigned long long* tag = gmem(const_cast<unsigned long long*>(&d.ring[(t + tid) & mask].seq_done));
            const unsigned long long s = __hip_atomic_load(tag, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_SYSTEM);
            const bool ready = s == t + (unsigned long long)tid + 1ull;
            const unsigned long long bal = __ballot(ready);
            const int lead = (int)__ffsll((long long)~bal) - 1;   // first not-ready lane, -1 if all
            int n = lead < 0 ? 64 : lead;
            if (n > max_batch) n = max_batch;
            // a tag beyond this round's sequence means the producer lapped the ring
            const bool lapped = (tid == 0) && s > t + 1ull;
            if (tid == 0) {
                clock_sync(d.clk_sync, ping_seen);
                const int stop = __hip_atomic_load(stop_flag, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_SYSTEM);
                const unsigned long long now = (unsigned long long)wall_clock64();
                int f = 0;
                if (stop) f = 1;
                else if (lapped) f = 2;
                else if (n == 0 && now - last_work > idle_ticks) f = 3;
                S.flag = f;
                S.bsize = n;
            }
        }
        __syncthreads();
        const int flag = S.flag, B = S.bsize;
        if (flag) {
            if (tid == 0) {
                if (flag > 1) atomicMax(status, flag);
                if (d.kend)
                    __hip_atomic_store(gmem(d.kend), (unsigned long long)wall_clock64(), __ATOMIC_RELAXED,
                                       __HIP_MEMORY_SCOPE_SYSTEM);
            }
            prof_end(S, d);
            return;
        }
        if (B == 0) {
            for (int i = 0; i < sleep_iters; ++i) __builtin_amdgcn_s_sleep(1);
            continue;
        }
        // pairs with the producer's release store of the tags seen above:
        // the records' fields are visible to the loads that follow
        __atomic_thread_fence(__ATOMIC_ACQUIRE);
        if (tid == 0) {
            S.t_pop = (unsigned long long)wall_clock64();
            S.tprev = S.t_pop;
        }
        load_batch(S, B, d.ring, t, mask, d.strip, G);
        __syncthreads();
        mark(S, PF_LOAD);
        process_batch(B, d, W, G);
        const unsigned long long t_done = (unsigned long long)wall_clock64();
        if (tid < B && d.timing) {
            const unsigned long long seq = t + (unsigned long long)tid;
            SSLA_GLOBAL GpuTimingSlot* ts = gmem(d.timing) + (seq & d.timing_mask);
            ts->t_pop_clk = S.t_pop;
            ts->t_done_clk = t_done;
            ts->seq = (unsigned int)seq;
            ts->owner = (S.own[tid] && S.p2[tid] && S.p3[tid]) ? 1u : 0u;
            ts->t_push_ns = S.tpush[tid];
            ts->t_emit_ns = S.temit[tid];
        }
        t += (unsigned long long)B;
        last_work = t_done;
        // predictions and timing of this batch (written by the record
        // threads, all in wave 0) become visible before the tail
        if (tid < 64) __threadfence_system();
        __syncthreads();
        if (tid == 0) {
            // one release for both stores (a second release store would
            // wait for the first to reach host memory)
            __atomic_thread_fence(__ATOMIC_RELEASE);
            __hip_atomic_store(gmem(d.tail), t, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_SYSTEM);
            if (d.events_done)
                __hip_atomic_store(gmem(d.events_done), t, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_SYSTEM);
        }
        mark(S, PF_PUBLISH);
        if (tid == 0) {
            S.prof[PF_BATCHES] += 1;
            S.prof[PF_RECORDS] += (unsigned long long)B;
        }
    }
}

// ---------------------------------------------------------------------------
// Channel-sliced groups: G workgroups (kGroupMin..kGroupMax) drain one block.
//
// A layer's OUT channels form OUT / 16 slices; member k of the group owns
// slices k, k + G, ...  Every member repeats the per-batch bookkeeping (ring
// load, tdrop, pair lists, LayerNorm) on the whole batch, with its own copy
// of the tdrop counters, so all members take the same decisions.  Per layer
// a member
//   P  projects q, v, g of its slices for the batch's pairs (16 x 16 MFMA
//      tiles, ProjPack weights) into pair rows in LDS;
//   S  runs the recurrence of its slices' channels over the pairs, on its
//      own channels of the block's hidden state (members write disjoint
//      state);
//   O  contracts its slices' q*h with the matching rows of goW (OutPackT's
//      goW fragments as the A operand, the q*h of 16 output records as B):
//      a partial pre-LayerNorm sum over its K slice for every output
//      channel.
// The members then exchange the partial sums.  Each value travels with the
// exchange's sequence number in the high half of one 64-bit word (relaxed
// agent-scope atomics: a reader that sees the tag sees the value), and
// every member adds the partials in member order and then the residual, so
// all members hold the same pre-LayerNorm rows and the same layer output.
// Two word sets alternate by sequence parity.  A member writes exchange
// n + 2 only after reading exchange n + 1 from every member, each of which
// wrote it after reading exchange n, so no word is overwritten before every
// member has read it.  Every exchange carries a header word per member; the
// L4 exchange of each batch is thus a group barrier, and member 0 broadcasts
// the next batch only after every member has loaded this one.  L5's and
// L7's exchanges are left out, by every member alike, when the batch has no
// output record for them.  Every wait is
// bounded on the wall clock: a member whose wait runs out sets status 4
// and leaves, and the others' waits then run out in turn.
// ---------------------------------------------------------------------------
constexpr int GSL = 2;                       // slices per member, at most (96 / 16 / kGroupMin)
constexpr int PRS = 3 * GSL * MT + 4;        // LDS pair row: [q | v | g] x GSL slices (+4: banks)
constexpr int XW = SSLA_C3;                  // words per record in an exchange set
constexpr size_t kXSet = (size_t)kGroupMax * LB * XW;        // one set, all members
constexpr size_t kXHdr = 2 * kXSet;                          // headers: [parity][member]
constexpr size_t kXBc = kXHdr + 2 * kGroupMax;               // member 0's batch word
constexpr size_t kXStride = (kXBc + 1 + 31) & ~(size_t)31;   // words per block
static_assert(kGroupMin * GSL * MT >= SSLA_C3, "slices per member");

struct alignas(16) LdsG {
    union {
        float PR[LP][PRS];               // pair rows of the member's slices
        float R[LB][XS];                 // head reg hidden (after the last layer)
    };
    float X[LB][XS];                     // layer input (becomes the layer output)
    float Y[LB][XS];                     // pre-LayerNorm sums / head cls hidden
    float H7[LB][8];
    unsigned long long tpush[LB], temit[LB];
    int ex[LB], ey[LB];
    int c2[LB], c3[LB];
    unsigned char vld[LB], own[LB], p2[LB], p3[LB];
    int pidx[LB][kPatch];
    int pe[LP], pc[LP], pnext[LP], lead[LP];
    unsigned pk[LB];
    unsigned pbits[LB];
    unsigned dmask;
    int ol[LB];
    int nlead, nout, bsize, flag, prof_on, abort_, nspec;
    unsigned xseq;                       // exchanges done by the group
    unsigned hack;                       // stage A: hand-offs acknowledged by B, last read
    unsigned long long t_pop, tprev;
    unsigned long long prof[NPROF];
};

__shared__ LdsG g_ldsg;

struct GroupCtx {
    unsigned long long* xb;              // the block's exchange words
    unsigned long long wait_ticks;       // limit of one wait inside a batch
    int k, G;
};

__device__ __forceinline__ unsigned long long xword(unsigned payload, unsigned tag) {
    return (unsigned long long)payload | ((unsigned long long)tag << 32);
}

__device__ __forceinline__ void xput(unsigned long long* w, unsigned long long v) {
    __hip_atomic_store(w, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

// The word at w once it carries `tag`; sets `late` (and returns what it
// read) when the wall clock passes `deadline` first.
__device__ __forceinline__ unsigned long long xwait(unsigned long long* w, unsigned tag,
                                                    unsigned long long deadline, bool& late) {
    unsigned long long v = __hip_atomic_load(w, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    while ((unsigned)(v >> 32) != tag) {
        if ((unsigned long long)wall_clock64() > deadline) {
            late = true;
            break;
        }
        __builtin_amdgcn_s_sleep(1);
        v = __hip_atomic_load(w, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    }
    return v;
}

// NCH projection chains of one wave over the batch's records (A: 16-record
// tiles of S.X): chain c multiplies by ProjPack item it[c] (16 weight
// columns) and its outputs go to columns cl[c] .. cl[c] + 15 of the pair
// rows (record, dl[c]) of the records that have that pair.
template <int IN, int OUT, int NCH>
__device__ __forceinline__ void group_proj(LdsG& S, int B, const float* __restrict__ pp,
                                           const int* it, const int* dl, const int* cl, int lane) {
    using P = ProjPack<IN, OUT>;
    const int li = lane & 15, lk = lane >> 4;
    // the weight addresses are formed here, per call: kept out of the
    // persistent loop's registers
    const float* w = pp;
    asm volatile("" : "+s"(w));
    float b[NCH][P::KS4 * 4];
    #pragma unroll
    for (int c = 0; c < NCH; ++c) P::load(w, it[c], lane, b[c]);
    const float* X = &S.X[0][0];
    for (int m0 = 0; m0 < B; m0 += MT) {
        const int xr = min(m0 + li, B - 1) * XS + lk;
        f32x4 a[NCH];
        #pragma unroll
        for (int c = 0; c < NCH; ++c) a[c] = f32x4{0.f, 0.f, 0.f, 0.f};
        #pragma unroll
        for (int s = 0; s < P::KS; ++s) {
            const float x = X[xr + s * 4];
            #pragma unroll
            for (int c = 0; c < NCH; ++c) a[c] = __builtin_amdgcn_mfma_f32_16x16x4f32(x, b[c][s], a[c], 0, 0, 0);
        }
        #pragma unroll
        for (int r = 0; r < 4; ++r) {
            const int rr = m0 + 4 * lk + r;
            if (rr < B) {
                const unsigned pb = S.pbits[rr];
                #pragma unroll
                for (int c = 0; c < NCH; ++c)
                    if ((pb >> dl[c]) & 1u) S.PR[rr * kPatch + dl[c]][cl[c] + li] = a[c][r];
            }
        }
    }
}

// One layer for one member; false when a wait of the exchange ran out.
template <int IN, int OUT>
__device__ __forceinline__ bool group_layer(LdsG& S, int B, const unsigned char* set,
                                            const unsigned char* outm, const LayerWeightsS2S3& L,
                                            const float* __restrict__ pp,
                                            const float* __restrict__ goT,
                                            const float* __restrict__ ipT,
                                            float* __restrict__ hidden, const GroupCtx& gc,
                                            int slot, bool may_skip = false,
                                            unsigned long long* ack = nullptr) {
    using P = ProjPack<IN, OUT>;
    constexpr int NSL = OUT / MT;
    const int tid = threadIdx.x, lane = tid & 63, wv = tid >> 6;
    const int li = lane & 15, lk = lane >> 4;
    if (tid < 64) {
        const bool o = tid < B && set[tid] && (outm == nullptr || outm[tid]);
        const unsigned long long bal = __ballot(o);
        if (o) S.ol[__popcll(bal & ((1ull << tid) - 1ull))] = tid;
        if (tid == 0) S.nout = __popcll(bal);
    }
    const int k = gc.k, G = gc.G;
    const int ns = k < NSL ? (NSL - 1 - k) / G + 1 : 0;      // own slices k, k + G, ...
    // P: the batch's records (A, 16-record tiles) times weight columns of
    // the member's slices, one MFMA chain per (delta, q / v / g, slice);
    // rows of the records with a pair at the delta are kept.  q is written
    // for every pair; the recurrence reads it only for output pairs.  With
    // one slice, wave w takes delta w's three chains and waves 1..3 one of
    // delta 8's each, so each wave loads its weights in one round; else
    // waves take (delta, slice) units of three chains in turn.
    static_assert(NW == 8, "one wave per delta 0..7");
    const unsigned dmask = S.dmask;
    if (ns == 1 && dmask) {
        const int d = wv, xo = wv - 1;
        const bool x4 = xo >= 0 && xo < 3;
        const int it[4] = {d * P::T + k, d * P::T + NSL + k, d * P::T + 2 * NSL + k,
                           8 * P::T + xo * NSL + k};
        const int dl[4] = {d, d, d, 8};
        const int cl[4] = {0, GSL * MT, 2 * GSL * MT, xo * GSL * MT};
        if constexpr (P::KS4 * 4 <= 16) {
            if (x4 && ((dmask >> 8) & 1u)) group_proj<IN, OUT, 4>(S, B, pp, it, dl, cl, lane);
            else if ((dmask >> d) & 1u) group_proj<IN, OUT, 3>(S, B, pp, it, dl, cl, lane);
        } else {
            // 96 inputs: the fourth chain's weights after the first three's
            // MFMAs (four chains' weights at once would not fit the registers)
            if ((dmask >> d) & 1u) group_proj<IN, OUT, 3>(S, B, pp, it, dl, cl, lane);
            if (x4 && ((dmask >> 8) & 1u)) group_proj<IN, OUT, 1>(S, B, pp, it + 3, dl + 3, cl + 3, lane);
        }
    } else if (dmask) {
        for (int u = wv; u < kPatch * ns; u += NW) {
            const int d = u / ns, js = u - d * ns;
            if (!((dmask >> d) & 1u)) continue;
            const int j = k + js * G;
            const int it[3] = {d * P::T + j, d * P::T + NSL + j, d * P::T + 2 * NSL + j};
            const int dl[3] = {d, d, d};
            const int cl[3] = {js * MT, (GSL + js) * MT, (2 * GSL + js) * MT};
            group_proj<IN, OUT, 3>(S, B, pp, it, dl, cl, lane);
        }
    }
    __syncthreads();
    mark(S, slot + 0);
    // ack (stage A's L5): a lane of wave 7, idle from here at live batch
    // sizes, reads the hand-off acknowledgement count; it lands in S.hack
    // before the layer's last barrier, so the hand-off after it rarely
    // waits on a read of its own
    constexpr int kAckLane = 7 * 64;
    unsigned long long ackv = 0;
    if (ack && tid == kAckLane) ackv = __hip_atomic_load(ack, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    // S: one lane per (cell, own channel); q*h replaces q for output pairs
    {
        constexpr int CH = 8;
        const int w16 = MT * ns, nl = S.nlead;
        for (int t = tid; t < nl * w16; t += LT) {
            const int kq = t / w16, c = t - kq * w16, js = c >> 4, cc = c & 15;
            const int qc = js * MT + cc, vc = (GSL + js) * MT + cc, gcl = (2 * GSL + js) * MT + cc;
            int q = S.lead[kq];
            float* hp = hidden + (size_t)S.pc[q] * OUT + (k + js * G) * MT + cc;
            float h = gload(hp);
            while (q >= 0) {
                int qs[CH];
                #pragma unroll
                for (int j = 0; j < CH; ++j) {
                    qs[j] = q;
                    if (q >= 0) q = S.pnext[q];
                }
                #pragma unroll
                for (int j = 0; j < CH; ++j) {
                    if (qs[j] >= 0) {
                        float* row = S.PR[qs[j]];
                        h = fmaf(sigmoid_fast(row[gcl]), h, row[vc]);
                        if (outm == nullptr || outm[S.pe[qs[j]]]) row[qc] *= h;
                    }
                }
            }
            gstore(hp, h);
        }
    }
    __syncthreads();
    mark(S, slot + 1);
    // O: the member's partial sums, then its header word
    const unsigned tag = S.xseq + 1u;
    const int par = (int)(S.xseq & 1u);
    unsigned long long* xs = gc.xb + (size_t)par * kXSet;
    unsigned long long* xh = gc.xb + kXHdr + (size_t)par * kGroupMax;
    const int no = S.nout;
    // may_skip: with no output record (every member counts the same ones)
    // there are no partial sums to exchange and no LayerNorm; the group's
    // exchanges stay in step, since every member skips the same ones
    if (may_skip && no == 0) {
        if (ack) {
            if (tid == kAckLane && (int)((unsigned)(ackv >> 32) - S.hack) > 0) S.hack = (unsigned)(ackv >> 32);
            __syncthreads();
        }
        mark(S, slot + 2);
        mark(S, PF_XWAIT + (slot == PF_L4 ? 0 : slot == PF_L5 ? 1 : slot == PF_L6 ? 2 : 3));
        mark(S, slot + 3);
        return true;
    }
    // the input_proj residual (IN != OUT) is one member's extra K slice: the
    // first member without a channel slice, else member 0
    constexpr bool IPR = IN != OUT;
    constexpr int KG = (IN + 15) / 16;
    const int mres = NSL < G ? NSL : 0;
    const bool has_res = IPR && k == mres;
    if (ns > 0 || has_res) {
        const int nit = NSL * ((no + MT - 1) / MT);
        for (int it = wv; it < nit; it += NW) {
            const int ot = it % NSL, r = (it / NSL) * MT + li;
            const int e = r < no ? S.ol[r] : -1;
            // per own slice: its nine goW fragments first, then three
            // independent MFMA chains (deltas d mod 3), added at the end
            f32x4 c3[3];
            #pragma unroll
            for (int q = 0; q < 3; ++q) c3[q] = f32x4{0.f, 0.f, 0.f, 0.f};
            // the residual's input_proj fragments load with the goW ones
            using OT = OutPackT<IN, OUT>;
            f32x4 ar[KG];
            if (has_res) {
                #pragma unroll
                for (int t = 0; t < KG; ++t)
                    ar[t] = ((const SSLA_GLOBAL f32x4*)ipT)[((size_t)ot * KG + t) * 64 + lane];
            }
            for (int js = 0; js < ns; ++js) {
                f32x4 a[kPatch];
                #pragma unroll
                for (int d = 0; d < kPatch; ++d)
                    a[d] = ((const SSLA_GLOBAL f32x4*)goT)[((size_t)(d * NSL + k + js * G) * NSL + ot) * 64 + lane];
                #pragma unroll
                for (int d = 0; d < kPatch; ++d) {
                    const int p = e >= 0 ? S.pidx[e][d] : -1;
                    f32x4 v = {0.f, 0.f, 0.f, 0.f};
                    if (p >= 0) v = *reinterpret_cast<const f32x4*>(&S.PR[p][js * MT + 4 * lk]);
                    #pragma unroll
                    for (int i = 0; i < 4; ++i)
                        c3[d % 3] = __builtin_amdgcn_mfma_f32_16x16x4f32(a[d][i], v[i], c3[d % 3], 0, 0, 0);
                }
            }
            f32x4 acc = c3[0] + c3[1] + c3[2];
            if (has_res) {
                // input_proj's fragments (OutPackT order); B: the record's
                // input, channels OutPackT::kidx(t, lk, i)
                #pragma unroll
                for (int t = 0; t < KG; ++t) {
                    f32x4 v = {0.f, 0.f, 0.f, 0.f};
                    if (e >= 0) {
                        const float* xe = &S.X[e][OT::kidx(t, lk, 0)];
                        #pragma unroll
                        for (int i = 0; i < OT::steps(t); ++i) v[i] = xe[i];
                    }
                    #pragma unroll
                    for (int i = 0; i < OT::steps(t); ++i)
                        acc = __builtin_amdgcn_mfma_f32_16x16x4f32(ar[t][i], v[i], acc, 0, 0, 0);
                }
            }
            if (r < no) {
                unsigned long long* w = xs + ((size_t)k * LB + r) * XW + ot * MT + 4 * lk;
                #pragma unroll
                for (int i = 0; i < 4; ++i) xput(w + i, xword(__float_as_uint(acc[i]), tag));
            }
        }
    }
    if (tid == 0) xput(xh + k, xword(0u, tag));
    mark(S, slot + 2);
    // the LayerNorm weights of the lane's channels, loaded ahead of the wait
    float lg[2], lbt[2];
    #pragma unroll
    for (int h = 0; h < 2; ++h) {
        const int ch = lane + 64 * h;
        lg[h] = ch < OUT ? gmem(L.ln_gamma)[ch] : 0.f;
        lbt[h] = ch < OUT ? gmem(L.ln_beta)[ch] : 0.f;
    }
    // sums of the members' partials (member order), then the identity residual
    const int ncon = (G < NSL ? G : NSL) + (IPR && NSL < G ? 1 : 0);
    const unsigned long long deadline = (unsigned long long)wall_clock64() + gc.wait_ticks;
    bool late = false;
    for (int t = tid; t < no * OUT; t += LT) {
        const int r = t / OUT, ch = t - r * OUT, e = S.ol[r];
        const float res = IPR ? 0.f : S.X[e][ch];
        // all contributors' words in flight at once, then the stragglers
        unsigned long long w[kGroupMax];
        #pragma unroll
        for (int kk = 0; kk < kGroupMax; ++kk)
            if (kk < ncon)
                w[kk] = __hip_atomic_load(xs + ((size_t)kk * LB + r) * XW + ch, __ATOMIC_RELAXED,
                                          __HIP_MEMORY_SCOPE_AGENT);
        float sum = 0.f;
        #pragma unroll
        for (int kk = 0; kk < kGroupMax; ++kk)
            if (kk < ncon) {
                if ((unsigned)(w[kk] >> 32) != tag)
                    w[kk] = xwait(xs + ((size_t)kk * LB + r) * XW + ch, tag, deadline, late);
                sum += __uint_as_float((unsigned)w[kk]);
            }
        S.Y[e][ch] = sum + res;
    }
    if (tid < G) (void)xwait(xh + tid, tag, deadline, late);
    if (late) S.abort_ = 1;
    __syncthreads();
    if (S.abort_) return false;
    if (tid == 0) S.xseq = tag;
    mark(S, PF_XWAIT + (slot == PF_L4 ? 0 : slot == PF_L5 ? 1 : slot == PF_L6 ? 2 : 3));
    // fp64 LayerNorm, one wave per output record
    for (int r = wv; r < no; r += NW) {
        const int e = S.ol[r];
        const float a = lane < OUT ? S.Y[e][lane] : 0.f;
        const float b = lane + 64 < OUT ? S.Y[e][lane + 64] : 0.f;
        const double mean = wave_sum((double)a + (double)b) / (double)OUT;
        const double da = lane < OUT ? (double)a - mean : 0.0;
        const double db = lane + 64 < OUT ? (double)b - mean : 0.0;
        const double var = wave_sum(da * da + db * db) / (double)OUT;
        const double inv = 1.0 / sqrt(var + 1e-5);
        if (lane < OUT) S.X[e][lane] = (float)(da * inv * (double)lg[0] + (double)lbt[0]);
        if (lane + 64 < OUT) S.X[e][lane + 64] = (float)(db * inv * (double)lg[1] + (double)lbt[1]);
    }
    if (ack && tid == kAckLane && (int)((unsigned)(ackv >> 32) - S.hack) > 0) S.hack = (unsigned)(ackv >> 32);
    __syncthreads();
    mark(S, slot + 3);
    return true;
}

// One batch for one member (the schedule of process_batch); false when an
// exchange wait ran out.  Member 0 also runs the head.
// Stage A of a group's batch: tdrop_s2, the s2 pairs, L4 and L5 (leaves L5's
// outputs in S.X for the pass-2 records).
__device__ __forceinline__ bool group_stage_a(int B, const LiveDesc& d, const LiveWeights& W,
                                             const Geometry& G, GroupCtx gc,
                                             const float* const* goT, const float* const* ipT,
                                             unsigned char* td2, unsigned long long* ack = nullptr) {
    LdsG& S = g_ldsg;
    // wave 0: tdrop_s2 with the per-record pair setup while its counters load
    if (threadIdx.x < 64) {
        const TdropLane r = tdrop_begin(B, td2, S.c2, nullptr);
        pairs_wave0<LdsG, false>(S, B, S.vld, G.H2, G.W2);
        tdrop_end(B, td2, S.p2, G.window, r);
    }
    __syncthreads();
    mark(S, PF_TD2);
    pairs_links(S, B, G.W2);
    mark(S, PF_PAIRS2);
    if (!group_layer<SSLA_C1, SSLA_C2>(S, B, S.vld, nullptr, W.L[0], W.pk.pp[0], goT[0], ipT[0], d.hidden[0], gc, PF_L4))
        return false;
    return group_layer<SSLA_C2, SSLA_C2>(S, B, S.vld, S.p2, W.L[1], W.pk.pp[1], goT[1], ipT[1], d.hidden[1], gc, PF_L5,
                                         true, ack);
}

// Stage B: pooling to s3, tdrop_s3, the s3 pairs, L6, L7 and (member 0) the
// head.  `l6_done` (may be null) runs once L6's exchange has completed, i.e.
// once every member of the group has read the batch's inputs.
template <class F>
__device__ __forceinline__ bool group_stage_b(int B, const LiveDesc& d, const LiveWeights& W,
                                             const Geometry& G, GroupCtx gc,
                                             const float* const* goT, const float* const* ipT,
                                             unsigned char* td3, unsigned* vsh, F l6_done) {
    LdsG& S = g_ldsg;
    const int tid = threadIdx.x;
    // wave 0 (lane = record): pooling to s3, then tdrop_s3 with the
    // per-record pair setup while its counters load
    if (tid < 64) {
        if (tid < B) {
            S.ex[tid] >>= 1;
            S.ey[tid] >>= 1;
            S.c3[tid] = S.vld[tid] ? S.ey[tid] * G.W3 + S.ex[tid] : -1;
        }
        const TdropLane r = tdrop_begin(B, td3, S.c3, S.p2);
        pairs_wave0<LdsG, false>(S, B, S.p2, G.H3, G.W3);
        tdrop_end(B, td3, S.p3, G.window, r);
    }
    __syncthreads();
    mark(S, PF_TD3);
    pairs_links(S, B, G.W3);
    mark(S, PF_PAIRS3);
    if (!group_layer<SSLA_C2, SSLA_C3>(S, B, S.p2, nullptr, W.L[2], W.pk.pp[2], goT[2], ipT[2], d.hidden[2], gc, PF_L6))
        return false;
    l6_done();
    // member 0's prediction-grid versions, read while L7 runs
    PredPlan pp;
    if (gc.k == 0 && W.have_head) pp = pred_plan(S, B, d, vsh);
    if (!group_layer<SSLA_C3, SSLA_C3>(S, B, S.p2, S.p3, W.L[3], W.pk.pp[3], goT[3], ipT[3], d.hidden[3], gc, PF_L7,
                                       true))
        return false;
    if (gc.k == 0 && W.have_head) batch_head(S, B, d, W, &pp);
    return true;
}

// One group running both stages of a batch.
__device__ __forceinline__ bool process_group(int B, const LiveDesc& d, const LiveWeights& W,
                                           const Geometry& G, GroupCtx gc,
                                           const float* const* goT, const float* const* ipT,
                                           unsigned char* td2,
                                           unsigned char* td3, unsigned* vsh) {
    if (!group_stage_a(B, d, W, G, gc, goT, ipT, td2)) return false;
    return group_stage_b(B, d, W, G, gc, goT, ipT, td3, vsh, [] {});
}

// Two-stage groups (live drain): per block a group A of G workgroups runs
// the batch load, tdrop_s2, the s2 pairs, L4 and L5, then hands the batch
// to a group B of G more workgroups, which runs tdrop_s3, the s3 pairs, L6,
// L7, the head, the predictions and the timing slots -- while A takes the
// next batch.  The hand-off goes through kHSlots slots of tagged words (as
// the exchanges: each 64-bit word carries the hand-off's sequence number,
// so a reader that sees the tag sees the value): a header (batch size and
// exit flag), the batch's pop time, and per record its s2 coordinates and
// flags, both timestamps and its L5 output row.  B's member 0 acknowledges
// hand-off n (one word: the count of hand-offs taken) once L6's exchange
// has completed (every member of B has read it); A's member 0 writes
// hand-off n into slot n mod kHSlots only when hand-off n - kHSlots has been
// acknowledged, re-reading the word only when the count it last read does
// not show that.  Two slots keep A at most two batches ahead of B: where B
// is the slower stage, A then takes bigger batches instead of queueing
// small ones in front of B (16 slots let 16 rings' B stages fall 16 batches
// behind: push -> prediction p50 570 us against 100).  B advances the ring
// tail (A read the batch's slots before handing it over) and the
// events_done counter after its stage.  Waits are bounded as the
// exchanges' are.
constexpr int kHRec = 5 + SSLA_C2;                  // words per record
constexpr unsigned kHSlots = 2;                     // hand-off slots per block
constexpr size_t kHSlot = 3 + (size_t)LB * kHRec;   // header, pop time (2), records
constexpr size_t kHAck = kHSlots * kHSlot;          // the acknowledgement word
constexpr size_t kHStride = (kHAck + 1 + 31) & ~(size_t)31;   // words per block

struct GroupArgs {
    unsigned long long* xb;              // exchange words, kXStride per block and stage (zeroed)
    unsigned char* tdrep;                // counters of members 1..G-1 of each stage:
                                         // (G - 1) x (C2 + C3) per block and stage
    unsigned long long* hb;              // hand-off words, kHStride per block (zeroed; 2 stages)
    const float* goT[4];                 // OutPackT goW fragments of L4..L7
    const float* ipT[4];                 // OutPackT input_proj fragments (L4, L6; else null)
    unsigned* vsh;                       // prediction-version copies, C3 words per block
    unsigned long long wait_ticks;
    int G;
    int stages;                          // 1, or 2 (live drain only)
};

// Stage A's member 0: hand-off `hseq` (slot hseq mod kHSlots) of B records,
// or of an exit flag; false when the slot's previous hand-off was not
// acknowledged in time.  S.hack holds the acknowledged count last read.
__device__ __forceinline__ bool handoff_put(LdsG& S, unsigned long long* hb, unsigned hseq, int B,
                                            int flag, unsigned long long wait_ticks) {
    const int tid = threadIdx.x;
    unsigned long long* hs = hb + (size_t)(hseq % kHSlots) * kHSlot;
    if (tid == 0) {
        bool late = false;
        const unsigned need = hseq - kHSlots + 1u;       // taken count that frees the slot
        if (hseq >= kHSlots && (int)(S.hack - need) < 0) {
            const unsigned long long dl = (unsigned long long)wall_clock64() + wait_ticks;
            unsigned long long v = __hip_atomic_load(hb + kHAck, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
            while ((int)((unsigned)(v >> 32) - need) < 0) {
                if ((unsigned long long)wall_clock64() > dl) {
                    late = true;
                    break;
                }
                __builtin_amdgcn_s_sleep(1);
                v = __hip_atomic_load(hb + kHAck, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
            }
            S.hack = (unsigned)(v >> 32);
        }
        S.abort_ = late ? 1 : 0;
    }
    __syncthreads();
    if (S.abort_) return false;
    const unsigned tag = hseq + 1u;
    for (int w = tid; w < B * kHRec; w += LT) {
        const int e = w / kHRec, q = w - e * kHRec;
        unsigned v;
        if (q == 0)      // 12-bit s2 coordinates (W2, H2 <= 4096) of valid records only
            v = (S.vld[e] ? ((unsigned)S.ex[e] & 0xfffu) | (((unsigned)S.ey[e] & 0xfffu) << 12) : 0u) |
                ((unsigned)S.vld[e] << 24) | ((unsigned)S.own[e] << 25) | ((unsigned)S.p2[e] << 26);
        else if (q == 1) v = (unsigned)S.tpush[e];
        else if (q == 2) v = (unsigned)(S.tpush[e] >> 32);
        else if (q == 3) v = (unsigned)S.temit[e];
        else if (q == 4) v = (unsigned)(S.temit[e] >> 32);
        else v = __float_as_uint(S.X[e][q - 5]);
        xput(hs + 3 + w, xword(v, tag));
    }
    if (tid == 0) {
        xput(hs + 1, xword((unsigned)S.t_pop, tag));
        xput(hs + 2, xword((unsigned)(S.t_pop >> 32), tag));
        xput(hs, xword((unsigned)B | ((unsigned)flag << 8), tag));
    }
    return true;
}

// Stage B of a two-stage live group: takes hand-offs in order, runs L6, L7
// and the head, and publishes (timing slots, events_done; member 0).
__device__ __forceinline__ void group_live_stage_b(LdsG& S, const LiveDesc& d,
                                                   const LiveWeights& W, const Geometry& G,
                                                   const GroupArgs& ga, GroupCtx gc,
                                                   unsigned char* td3,
                                                   unsigned long long idle_ticks,
                                                   unsigned int spin_ns, int* status,
                                                   unsigned long long* hb, unsigned* vsh) {
    const int tid = threadIdx.x, k = gc.k;
    const int sleep_iters = (int)(spin_ns / 40u) + 1;
    unsigned long long t = d.t0;
    unsigned long long last_work = (unsigned long long)wall_clock64();
    unsigned hseq = 0;
    while (true) {
        __syncthreads();
        unsigned long long* hs = hb + (size_t)(hseq % kHSlots) * kHSlot;
        const unsigned tag = hseq + 1u;
        if (tid == 0) {
            // stage A hands off at least once per idle timeout (then it stops)
            const unsigned long long dl = last_work + idle_ticks + gc.wait_ticks;
            unsigned long long v = __hip_atomic_load(hs, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
            bool late = false;
            while ((unsigned)(v >> 32) != tag) {
                if ((unsigned long long)wall_clock64() > dl) {
                    late = true;
                    break;
                }
                for (int i = 0; i < sleep_iters; ++i) __builtin_amdgcn_s_sleep(1);
                v = __hip_atomic_load(hs, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
            }
            S.flag = late ? 4 : (int)((v >> 8) & 0xffu);
            S.bsize = (int)(v & 0xffu);
            S.abort_ = 0;
        }
        __syncthreads();
        const int flag = S.flag, B = S.bsize;
        if (flag) {
            if (tid == 0 && flag == 4) atomicMax(status, 4);
            if (k == 0) prof_end(S, d, 1);
            return;
        }
        {
            const unsigned long long dl = (unsigned long long)wall_clock64() + gc.wait_ticks;
            bool late = false;
            // a thread's words are loaded together, then the ones whose tag
            // has not arrived yet are waited for one by one
            constexpr int NW = (LB * kHRec + LT - 1) / LT;
            unsigned long long hv[NW];
            #pragma unroll
            for (int i = 0; i < NW; ++i) {
                const int w = tid + i * LT;
                hv[i] = w < B * kHRec ? __hip_atomic_load(hs + 3 + w, __ATOMIC_RELAXED,
                                                          __HIP_MEMORY_SCOPE_AGENT)
                                      : 0ull;
            }
            #pragma unroll
            for (int i = 0; i < NW; ++i) {
                const int w = tid + i * LT;
                if (w >= B * kHRec) continue;
                if ((unsigned)(hv[i] >> 32) != tag) hv[i] = xwait(hs + 3 + w, tag, dl, late);
                const unsigned u = (unsigned)hv[i];
                const int e = w / kHRec, q = w - e * kHRec;
                if (q == 0) {
                    S.ex[e] = (int)(u & 0xfffu);
                    S.ey[e] = (int)((u >> 12) & 0xfffu);
                    S.vld[e] = (unsigned char)((u >> 24) & 1u);
                    S.own[e] = (unsigned char)((u >> 25) & 1u);
                    S.p2[e] = (unsigned char)((u >> 26) & 1u);
                    S.p3[e] = 0;
                } else if (q <= 4) {
                    unsigned* w2 = reinterpret_cast<unsigned*>(q <= 2 ? &S.tpush[e] : &S.temit[e]);
                    w2[(q - 1) & 1] = u;
                } else {
                    S.X[e][q - 5] = __uint_as_float(u);
                }
            }
            if (tid == 0) {
                const unsigned lo = (unsigned)xwait(hs + 1, tag, dl, late);
                const unsigned hi = (unsigned)xwait(hs + 2, tag, dl, late);
                S.t_pop = (unsigned long long)lo | ((unsigned long long)hi << 32);
                S.tprev = (unsigned long long)wall_clock64();
            }
            if (late) S.abort_ = 1;
        }
        __syncthreads();
        if (S.abort_) {
            if (tid == 0) atomicMax(status, 4);
            if (k == 0) prof_end(S, d, 1);
            return;
        }
        // L6's exchange has every member's partial sums, so every member has
        // read the hand-off: member 0 acknowledges it (the count taken)
        const bool ok = group_stage_b(B, d, W, G, gc, ga.goT, ga.ipT, td3, vsh, [&] {
            if (k == 0 && threadIdx.x == 0) xput(hb + kHAck, xword(0u, tag));
        });
        if (!ok) {
            if (tid == 0) atomicMax(status, 4);
            if (k == 0) prof_end(S, d, 1);
            return;
        }
        const unsigned long long t_done = (unsigned long long)wall_clock64();
        if (k == 0) {
            if (tid < B && d.timing) {
                const unsigned long long seq = t + (unsigned long long)tid;
                SSLA_GLOBAL GpuTimingSlot* ts = gmem(d.timing) + (seq & d.timing_mask);
                ts->t_pop_clk = S.t_pop;
                ts->t_done_clk = t_done;
                ts->seq = (unsigned int)seq;
                ts->owner = (S.own[tid] && S.p2[tid] && S.p3[tid]) ? 1u : 0u;
                ts->t_push_ns = S.tpush[tid];
                ts->t_emit_ns = S.temit[tid];
            }
            // the batch's timing slots and predictions: written by the record
            // threads, all in wave 0
            if (tid < 64) __threadfence_system();
            __syncthreads();
            if (tid == 0) {
                // the batch's ring slots (stage A read them before handing
                // the batch over); one release for both stores (a second
                // release store would wait for the first to reach host memory)
                __atomic_thread_fence(__ATOMIC_RELEASE);
                __hip_atomic_store(gmem(d.tail), t + (unsigned long long)B, __ATOMIC_RELAXED,
                                   __HIP_MEMORY_SCOPE_SYSTEM);
                if (d.events_done)
                    __hip_atomic_store(gmem(d.events_done), t + (unsigned long long)B, __ATOMIC_RELAXED,
                                       __HIP_MEMORY_SCOPE_SYSTEM);
            }
            mark(S, PF_PUBLISH);
        }
        t += (unsigned long long)B;
        last_work = t_done;
        ++hseq;
    }
}

// Batch mode (LIVE false: d.n records in batches of max_batch) or the
// persistent live drain; blocks of G consecutive workgroups (G per stage,
// stage A first, with two stages).
template <bool LIVE, int ST>
__global__ void __launch_bounds__(LT)
k_group(const LiveDesc* __restrict__ ld, LiveWeights W, Geometry G, GroupArgs ga,
        const int* stop_flag, unsigned int spin_ns, unsigned long long idle_ticks, int max_batch,
        int* __restrict__ status) {
    LdsG& S = g_ldsg;
    const int tid = threadIdx.x;
    // block b's workgroups: stage 0 (A) members 0..G-1, then stage 1 (B)
    static_assert(ST == 1 || (ST == 2 && LIVE), "two stages: live drain only");
    const int GS = ga.G * ST;
    const int b = blockIdx.x / GS, m = blockIdx.x - b * GS;
    const int stage = m / ga.G, k = m - stage * ga.G;
    const LiveDesc& d = ld[b];
    const GroupCtx gc{ga.xb + ((size_t)b * ST + stage) * kXStride, ga.wait_ticks, k, ga.G};
    unsigned char* td2 = d.td2;
    unsigned char* td3 = d.td3;
    if (k > 0) {
        td2 = ga.tdrep + (((size_t)b * ST + stage) * (ga.G - 1) + (k - 1)) * (size_t)(G.C2 + G.C3);
        td3 = td2 + G.C2;
    }
    if (k == 0) prof_begin(S, d);
    if (tid == 0) {
        if (k != 0) S.prof_on = 0;
        S.abort_ = 0;
        S.xseq = 0;
        S.hack = 0;
    }
    // the workgroup that publishes predictions starts its copy of the
    // block's version words
    unsigned* vsh = nullptr;
    if (k == 0 && stage == ST - 1 && W.have_head && d.version && ga.vsh) {
        vsh = ga.vsh + (size_t)b * G.C3;
        const HybridStrip& s = d.strip;
        const int nc = (s.s3_owned_hi - s.s3_owned_lo) * (s.s3_owned_y_hi - s.s3_owned_y_lo);
        for (int c = tid; c < nc; c += LT) gmem(vsh)[c] = pred_version(d.version + c);
    }
    __syncthreads();
    if constexpr (ST == 2) {
        if (stage == 1) {
            group_live_stage_b(S, d, W, G, ga, gc, td3, idle_ticks, spin_ns, status,
                               ga.hb + (size_t)b * kHStride, vsh);
            return;
        }
    }
    unsigned long long* const hb = ST == 2 ? ga.hb + (size_t)b * kHStride : nullptr;
    const int pstage = ST == 2 ? 0 : -1;            // profile slots member 0 writes
    if constexpr (!LIVE) {
        int bi = 0;
        for (int base = 0; base < d.n; base += max_batch, ++bi) {
            const int B = min(max_batch, d.n - base);
            if (tid == 0) {
                S.t_pop = (unsigned long long)wall_clock64();
                S.tprev = S.t_pop;
            }
            load_batch(S, B, d.ring, (unsigned long long)base, ~0ull, d.strip, G);
            __syncthreads();
            mark(S, PF_LOAD);
            if (!process_group(B, d, W, G, gc, ga.goT, ga.ipT, td2, td3, vsh)) {
                if (tid == 0) atomicMax(status, 4);
                return;
            }
            if (k == 0) {
                for (int t = tid; t < B * SSLA_C3; t += LT) {
                    const int e = t / SSLA_C3, i = t % SSLA_C3;
                    if (d.out) gmem(d.out)[base + e].s3_feat[i] = (S.vld[e] && S.p3[e]) ? S.X[e][i] : 0.f;
                }
                if (tid < B) {
                    const int e = tid;
                    const bool v = S.vld[e], own = S.own[e];
                    if (d.out) {
                        gmem(d.out)[base + e].pass2 = !v ? -2 : (own ? (int)S.p2[e] : -1);
                        gmem(d.out)[base + e].pass3 = !v ? -2 : (own ? (int)S.p3[e] : -1);
                    }
                    if (d.head_out) {
                        const bool hv = W.have_head && own && S.p3[e];
                        #pragma unroll
                        for (int q = 0; q < 7; ++q) gmem(d.head_out)[(size_t)(base + e) * 7 + q] = hv ? S.H7[e][q] : 0.f;
                    }
                }
                if (tid == 0 && d.batch_clk) {
                    gmem(d.batch_clk)[(size_t)bi * 2 + 0] = S.t_pop;
                    gmem(d.batch_clk)[(size_t)bi * 2 + 1] = (unsigned long long)wall_clock64();
                }
            }
            __syncthreads();
            mark(S, PF_PUBLISH);
            if (tid == 0) {
                S.prof[PF_BATCHES] += 1;
                S.prof[PF_RECORDS] += (unsigned long long)B;
            }
        }
        if (k == 0) prof_end(S, d);
        return;
    }
    const unsigned long long mask = d.ring_mask;
    unsigned long long t = d.t0;
    unsigned long long last_work = (unsigned long long)wall_clock64();
    if (k == 0 && tid == 0 && d.kstart)
        __hip_atomic_store(gmem(d.kstart), last_work, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_SYSTEM);
    const int sleep_iters = (int)(spin_ns / 40u) + 1;
    unsigned long long* bc = gc.xb + kXBc;
    unsigned bseq = 0;                   // batches broadcast
    unsigned hseq = 0;                   // hand-offs to stage B (two stages)
    unsigned long long ping_seen = 0;
    while (true) {
        __syncthreads();
        int have = 0;                    // records of the batch already in LDS (members)
        if (k == 0) {
            // poll: lanes 0 .. max_batch - 1 of wave 0 probe consecutive tags
            // (one host-memory read each)
            if (tid < 64) {
                unsigned long long s = 0;
                if (tid < max_batch) {
                    SSLA_GLOBAL unsigned long long* tag =
                        gmem(const_cast<unsigned long long*>(&d.ring[(t + tid) & mask].seq_done));
                    s = __hip_atomic_load(tag, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_SYSTEM);
                }
                const bool ready = tid < max_batch && s == t + (unsigned long long)tid + 1ull;
                const unsigned long long bal = __ballot(ready);
                const int lead = (int)__ffsll((long long)~bal) - 1;
                const int n = lead < 0 ? 64 : lead;    // <= max_batch
                const bool lapped = (tid == 0) && s > t + 1ull;
                if (tid == 0) {
                    clock_sync(d.clk_sync, ping_seen);
                    const int stop = __hip_atomic_load(stop_flag, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_SYSTEM);
                    const unsigned long long now = (unsigned long long)wall_clock64();
                    int f = 0;
                    if (stop) f = 1;
                    else if (lapped) f = 2;
                    else if (n == 0 && now - last_work > idle_ticks) f = 3;
                    S.flag = f;
                    S.bsize = n;
                    if (f || n) xput(bc, xword((unsigned)n | ((unsigned)f << 8), bseq + 1u));
                }
            }
            __syncthreads();
            if (S.flag == 0 && S.bsize == 0) {
                for (int i = 0; i < sleep_iters; ++i) __builtin_amdgcn_s_sleep(1);
                continue;
            }
        } else {
            // the ring's ready prefix as this member sees it (its first
            // kSpecTags slots at most: each probe is a host-memory read, and
            // every member of every block polls), loaded while member 0
            // decides the batch (records beyond that batch are loaded again
            // with the next one)
            if (tid < 64) {
                const int np = min(max_batch, kSpecTags);
                unsigned long long s = 0;
                if (tid < np) {
                    SSLA_GLOBAL unsigned long long* tag =
                        gmem(const_cast<unsigned long long*>(&d.ring[(t + tid) & mask].seq_done));
                    s = __hip_atomic_load(tag, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_SYSTEM);
                }
                const unsigned long long bal = __ballot(tid < np && s == t + (unsigned long long)tid + 1ull);
                const int lead = (int)__ffsll((long long)~bal) - 1;
                if (tid == 0) S.nspec = lead < 0 ? 64 : lead;    // <= np
            }
            __syncthreads();
            have = S.nspec;
            if (have > 0) {
                // pairs with the producer's release store of the tags
                __atomic_thread_fence(__ATOMIC_ACQUIRE);
                load_batch(S, have, d.ring, t, mask, d.strip, G);
            }
            if (tid == 0) {
                // member 0 broadcasts at least once per idle timeout (then it stops)
                const unsigned long long dl = last_work + idle_ticks + gc.wait_ticks;
                unsigned long long v = __hip_atomic_load(bc, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
                bool late = false;
                while ((unsigned)(v >> 32) != bseq + 1u) {
                    if ((unsigned long long)wall_clock64() > dl) {
                        late = true;
                        break;
                    }
                    for (int i = 0; i < sleep_iters; ++i) __builtin_amdgcn_s_sleep(1);
                    v = __hip_atomic_load(bc, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
                }
                S.flag = late ? 4 : (int)((v >> 8) & 0xffu);
                S.bsize = (int)(v & 0xffu);
            }
            __syncthreads();
        }
        const int flag = S.flag, B = S.bsize;
        ++bseq;
        if (flag) {
            if (tid == 0) {
                if ((k == 0 && flag > 1) || flag == 4) atomicMax(status, flag);
                if (k == 0 && d.kend)
                    __hip_atomic_store(gmem(d.kend), (unsigned long long)wall_clock64(), __ATOMIC_RELAXED,
                                       __HIP_MEMORY_SCOPE_SYSTEM);
            }
            // stage B ends on the same flag once it has taken every batch
            if (ST == 2 && k == 0 && !handoff_put(S, hb, hseq, 0, flag, gc.wait_ticks) &&
                tid == 0)
                atomicMax(status, 4);
            if (k == 0) prof_end(S, d, pstage);
            return;
        }
        if (k != 0 && tid >= have && tid < B) {
            // the producer's tags of the rest of this batch (member 0 has
            // seen them)
            SSLA_GLOBAL unsigned long long* tag = gmem(const_cast<unsigned long long*>(&d.ring[(t + tid) & mask].seq_done));
            const unsigned long long want = t + (unsigned long long)tid + 1ull;
            const unsigned long long dl = (unsigned long long)wall_clock64() + gc.wait_ticks;
            while (__hip_atomic_load(tag, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_SYSTEM) != want) {
                if ((unsigned long long)wall_clock64() > dl) {
                    S.abort_ = 1;
                    break;
                }
                __builtin_amdgcn_s_sleep(1);
            }
        }
        __syncthreads();
        if (S.abort_) {
            if (tid == 0) atomicMax(status, 4);
            return;
        }
        // pairs with the producer's release store of the tags
        if (B > have) __atomic_thread_fence(__ATOMIC_ACQUIRE);
        if (tid == 0) {
            S.t_pop = (unsigned long long)wall_clock64();
            S.tprev = S.t_pop;
        }
        if (B > have) load_batch(S, B, d.ring, t, mask, d.strip, G, have);
        __syncthreads();
        mark(S, PF_LOAD);
        bool ok;
        if constexpr (ST == 2)
            ok = group_stage_a(B, d, W, G, gc, ga.goT, ga.ipT, td2, k == 0 ? hb + kHAck : nullptr);
        else ok = process_group(B, d, W, G, gc, ga.goT, ga.ipT, td2, td3, vsh);
        if (!ok) {
            if (tid == 0) {
                atomicMax(status, 4);
                if (k == 0 && d.kend)
                    __hip_atomic_store(gmem(d.kend), (unsigned long long)wall_clock64(), __ATOMIC_RELAXED,
                                       __HIP_MEMORY_SCOPE_SYSTEM);
            }
            if (ST == 2 && k == 0) (void)handoff_put(S, hb, hseq, 0, 4, gc.wait_ticks);
            if (k == 0) prof_end(S, d, pstage);
            return;
        }
        if constexpr (ST == 2) {
            // stage A: the batch goes to stage B
            if (k == 0) {
                if (!handoff_put(S, hb, hseq, B, 0, gc.wait_ticks)) {
                    if (tid == 0) atomicMax(status, 4);
                    prof_end(S, d, pstage);
                    return;
                }
                if (tid == 0) {
                    S.prof[PF_BATCHES] += 1;
                    S.prof[PF_RECORDS] += (unsigned long long)B;
                }
            }
            ++hseq;
            t += (unsigned long long)B;
            last_work = (unsigned long long)wall_clock64();
            continue;
        }
        const unsigned long long t_done = (unsigned long long)wall_clock64();
        if (k == 0) {
            if (tid < B && d.timing) {
                const unsigned long long seq = t + (unsigned long long)tid;
                SSLA_GLOBAL GpuTimingSlot* ts = gmem(d.timing) + (seq & d.timing_mask);
                ts->t_pop_clk = S.t_pop;
                ts->t_done_clk = t_done;
                ts->seq = (unsigned int)seq;
                ts->owner = (S.own[tid] && S.p2[tid] && S.p3[tid]) ? 1u : 0u;
                ts->t_push_ns = S.tpush[tid];
                ts->t_emit_ns = S.temit[tid];
            }
            // the batch's timing slots and predictions: written by the record
            // threads, all in wave 0
            if (tid < 64) __threadfence_system();
            __syncthreads();
            if (tid == 0) {
                // one release for both stores (a second release store would
                // wait for the first to reach host memory)
                __atomic_thread_fence(__ATOMIC_RELEASE);
                __hip_atomic_store(gmem(d.tail), t + (unsigned long long)B, __ATOMIC_RELAXED,
                                   __HIP_MEMORY_SCOPE_SYSTEM);
                if (d.events_done)
                    __hip_atomic_store(gmem(d.events_done), t + (unsigned long long)B, __ATOMIC_RELAXED,
                                       __HIP_MEMORY_SCOPE_SYSTEM);
            }
            mark(S, PF_PUBLISH);
            if (tid == 0) {
                S.prof[PF_BATCHES] += 1;
                S.prof[PF_RECORDS] += (unsigned long long)B;
            }
        }
        t += (unsigned long long)B;
        last_work = t_done;
    }
}


#define LHIP(call)                                                            \
    do {                                                                      \
        hipError_t e_ = (call);                                               \
        if (e_ != hipSuccess) {                                               \
            set_error(std::string(#call) + ": " + hipGetErrorString(e_));    \
            return SSLA_ERR_HIP;                                              \
        }                                                                     \
    } while (0)

size_t scratch_floats() { return (size_t)LP * NCMAX; }

// batch-mode workspace: per-block scratch rows + the device block table
std::mutex g_bmu;
float* g_bscratch = nullptr;
LiveDesc* g_bdesc = nullptr;
LiveDesc* g_bdesc_host = nullptr;
hipEvent_t g_bcopied = nullptr;
unsigned long long* g_bprof = nullptr;
float* g_bpack = nullptr;
hipEvent_t g_bdone = nullptr;   // the last batch drain's kernel
unsigned long long* g_bprof_host = nullptr;

}  // namespace

static int live_weights(const HybridS2S3Config* cfg, LiveWeights* W, Geometry* G) {
    const int nb = cfg->n_blocks;
    if (nb < 1 || nb > SSLA_MAX_BLOCKS) {
        set_error("n_blocks must be in [1, 16]");
        return SSLA_ERR_ARG;
    }
    if (cfg->H2 <= 0 || cfg->W2 <= 0 || (cfg->H2 & 1) || (cfg->W2 & 1) ||
        cfg->H3 != cfg->H2 / 2 || cfg->W3 != cfg->W2 / 2) {
        set_error("grid must have even H2, W2 and H3 = H2/2, W3 = W2/2");
        return SSLA_ERR_ARG;
    }
    for (int b = 0; b < nb; ++b)
        for (int li = 0; li < 4; ++li) {
            const LayerWeightsS2S3& L = cfg->layers[b][li];
            const LayerWeightsS2S3& L0 = cfg->layers[0][li];
            if (!L.qvgIn || !L.goW || !L.ln_gamma || !L.ln_beta || L.qvgIn != L0.qvgIn ||
                L.goW != L0.goW || L.input_proj != L0.input_proj || L.ln_gamma != L0.ln_gamma ||
                L.ln_beta != L0.ln_beta) {
                set_error("all blocks must share one bound set of layer weights");
                return SSLA_ERR_ARG;
            }
            if (!cfg->hidden[b][li] || !cfg->tdrop_s2[b] || !cfg->tdrop_s3[b]) {
                set_error("block state not allocated");
                return SSLA_ERR_ARG;
            }
        }
    if (!cfg->layers[0][0].input_proj || !cfg->layers[0][2].input_proj ||
        cfg->layers[0][1].input_proj || cfg->layers[0][3].input_proj) {
        set_error("L4/L6 need input_proj and L5/L7 must not have one");
        return SSLA_ERR_ARG;
    }
    for (int li = 0; li < 4; ++li) W->L[li] = cfg->layers[0][li];
    if (const char* m = head_missing(cfg)) {
        set_error(m);
        return SSLA_ERR_ARG;
    }
    W->head = head_ptrs(cfg);
    W->have_head = head_kind(cfg);
    G->H2 = cfg->H2; G->W2 = cfg->W2; G->H3 = cfg->H3; G->W3 = cfg->W3;
    G->C2 = G->H2 * G->W2; G->C3 = G->H3 * G->W3; G->nb = nb; G->window = cfg->tdrop_window;
    return SSLA_OK;
}

static void live_desc_state(const HybridS2S3Config* cfg, int b, LiveDesc* d) {
    for (int li = 0; li < 4; ++li) d->hidden[li] = cfg->hidden[b][li];
    d->td2 = cfg->tdrop_s2[b];
    d->td3 = cfg->tdrop_s3[b];
    d->strip = cfg->strip[b];
    const bool head = head_kind(cfg) != kHeadNone;
    d->preds = head ? cfg->preds[b] : nullptr;
    d->version = head ? cfg->version[b] : nullptr;
}

// Adds the per-block profile sums in `dev` (NPROF x nb, wall-clock ticks and
// counts) to phase_us: times in microseconds, the last two slots as counts.
static void add_profile(const unsigned long long* host, int nb, double* phase_us) {
    int khz = 0;
    if (hipDeviceGetAttribute(&khz, hipDeviceAttributeWallClockRate, 0) != hipSuccess || khz <= 0)
        khz = 100000;
    for (int b = 0; b < nb; ++b)
        for (int k = 0; k < NPROF; ++k) {
            const double v = (double)host[(size_t)b * NPROF + k];
            phase_us[k] += (k == PF_BATCHES || k == PF_RECORDS) ? v : v * 1000.0 / (double)khz;
        }
}

int batch_drain(const HybridS2S3Config* cfg, const HybridInputRec* const* rings, const int* ns,
                HybridS2S3OutputSlot* const* outs, float* const* head_outs,
                unsigned long long* const* batch_clks, int batch, hipStream_t st, bool sync,
                double* phase_us) {
    LiveWeights W;
    Geometry G;
    int rc = live_weights(cfg, &W, &G);
    if (rc) return rc;
    if (batch < 1 || batch > LB) {
        set_error("batch must be in [1, 32]");
        return SSLA_ERR_ARG;
    }
    const int nb = cfg->n_blocks;
    for (int b = 0; b < nb; ++b)
        if (ns[b] < 0 || (ns[b] > 0 && !rings[b])) {
            set_error("bad ring / count for block " + std::to_string(b));
            return SSLA_ERR_ARG;
        }
    if (phase_us && !sync) {
        set_error("batch_phase_us needs sync");
        return SSLA_ERR_ARG;
    }
    std::lock_guard<std::mutex> lk(g_bmu);
    if (!g_bscratch) {
        const size_t bytes = sizeof(float) * scratch_floats() * SSLA_MAX_BLOCKS;
        LHIP(hipMalloc(&g_bscratch, bytes));
        LHIP(hipMemset(g_bscratch, 0, bytes));
        LHIP(hipMalloc(&g_bprof, sizeof(unsigned long long) * NPROF * SSLA_MAX_BLOCKS));
        LHIP(hipMalloc(&g_bpack, sizeof(float) * packed_weight_floats()));
        LHIP(hipHostMalloc((void**)&g_bprof_host, sizeof(unsigned long long) * NPROF * SSLA_MAX_BLOCKS,
                           hipHostMallocDefault));
        LHIP(hipMalloc(&g_bdesc, sizeof(LiveDesc) * SSLA_MAX_BLOCKS));
        LHIP(hipHostMalloc((void**)&g_bdesc_host, sizeof(LiveDesc) * SSLA_MAX_BLOCKS, hipHostMallocDefault));
        LHIP(hipEventCreateWithFlags(&g_bcopied, hipEventDisableTiming));
        LHIP(hipEventCreateWithFlags(&g_bdone, hipEventDisableTiming));
        LHIP(hipDeviceSynchronize());
    }
    // calls share the scratch rows and weight copies: a call on another
    // stream runs after the previous call's kernel (device-side wait)
    LHIP(hipStreamWaitEvent(st, g_bdone, 0));
    LHIP(hipEventSynchronize(g_bcopied));
    std::memset(g_bdesc_host, 0, sizeof(LiveDesc) * SSLA_MAX_BLOCKS);
    for (int b = 0; b < nb; ++b) {
        LiveDesc& d = g_bdesc_host[b];
        live_desc_state(cfg, b, &d);
        d.ring = rings[b];
        d.ring_mask = ~0ull;
        d.n = ns[b];
        d.scratch = g_bscratch + scratch_floats() * b;
        d.out = outs ? outs[b] : nullptr;
        d.head_out = head_outs ? head_outs[b] : nullptr;
        d.batch_clk = batch_clks ? batch_clks[b] : nullptr;
        d.prof = phase_us ? g_bprof + (size_t)NPROF * b : nullptr;
    }
    LHIP(hipMemcpyAsync(g_bdesc, g_bdesc_host, sizeof(LiveDesc) * nb, hipMemcpyHostToDevice, st));
    LHIP(hipEventRecord(g_bcopied, st));
    LHIP(pack_weights(W.L, g_bpack, &W.pk, st));
    hipLaunchKernelGGL(k_batch_drain, dim3(nb), dim3(LT), 0, st, g_bdesc, W, G, batch);
    LHIP(hipGetLastError());
    LHIP(hipEventRecord(g_bdone, st));
    if (sync) LHIP(hipStreamSynchronize(st));
    if (phase_us) {
        LHIP(hipMemcpy(g_bprof_host, g_bprof, sizeof(unsigned long long) * NPROF * nb,
                       hipMemcpyDeviceToHost));
        add_profile(g_bprof_host, nb, phase_us);
    }
    return SSLA_OK;
}

// ---------------------------------------------------------------------------
// batch drain that allocates nothing (ssla_hip_drain_batch_noalloc)
// ---------------------------------------------------------------------------
namespace {

// Device memory the batch kernel uses beyond its inputs and outputs, for up
// to kNaMaxBlocks blocks: each block's pair rows (LP x NCMAX floats), the
// fragment-order weight copy and the block table.  One array per device,
// held until the process ends; every call on a device shares it, so calls
// that overlap on one device race.  Nothing in it has to start at zero: a
// batch writes every pair row it reads, and each call rewrites the weight
// copy and the block table before its kernel runs.
constexpr int kNaMaxBlocks = SSLA_MAX_BLOCKS;
constexpr size_t kNaRowFloats = (size_t)LP * NCMAX;                     // per block
constexpr size_t kNaPackOff = sizeof(float) * kNaRowFloats * kNaMaxBlocks;
constexpr size_t kNaDescOff =
    (kNaPackOff + sizeof(float) * PackLayout<false>::off[8] + 255) & ~size_t(255);
constexpr size_t kNaBytes = kNaDescOff + sizeof(LiveDesc) * kNaMaxBlocks;
static_assert(kNaBytes <= (size_t)16 << 20, "the no-allocation scratch stays modest");

static __device__ __align__(256) unsigned char scratch[kNaBytes];

// The block table travels as kernel arguments, eight entries per launch.
constexpr int kNaDescChunk = 8;
struct DescChunk {
    LiveDesc d[kNaDescChunk];
};
static_assert(sizeof(DescChunk) <= 3072, "kernel argument block");

__global__ void k_put_desc(DescChunk c, int n, LiveDesc* __restrict__ dst) {
    if ((int)threadIdx.x < n) dst[threadIdx.x] = c.d[threadIdx.x];
}

constexpr int kNaMaxDevices = 64;
std::mutex g_na_mu;
unsigned char* g_na_ptr[kNaMaxDevices] = {};

// The device address of the current device's `scratch` (host code may not
// use the symbol itself: its host-side name is not a device address).
int na_scratch(unsigned char** out) {
    int dev = 0;
    LHIP(hipGetDevice(&dev));
    if (dev < 0 || dev >= kNaMaxDevices) {
        set_error("drain_batch_noalloc: device index out of range");
        return SSLA_ERR_ARG;
    }
    std::lock_guard<std::mutex> lk(g_na_mu);
    if (!g_na_ptr[dev]) {
        void* p = nullptr;
        LHIP(hipGetSymbolAddress(&p, HIP_SYMBOL(scratch)));
        g_na_ptr[dev] = static_cast<unsigned char*>(p);
    }
    *out = g_na_ptr[dev];
    return SSLA_OK;
}

}  // namespace

size_t noalloc_scratch_bytes() { return kNaBytes; }

int batch_drain_noalloc(const HybridS2S3Config* cfg, const HybridInputRec* const* rings,
                        const int* ns, HybridS2S3OutputSlot* const* outs,
                        float* const* head_outs, int batch, hipStream_t st) {
    LiveWeights W;
    Geometry G;
    int rc = live_weights(cfg, &W, &G);
    if (rc) return rc;
    const int nb = cfg->n_blocks;
    if (nb > kNaMaxBlocks) {
        set_error("drain_batch_noalloc: n_blocks exceeds the scratch's " +
                  std::to_string(kNaMaxBlocks) + " blocks");
        return SSLA_ERR_ARG;
    }
    if (batch < 1 || batch > LB) {
        set_error("drain_batch_noalloc: batch must be in [1, 32]");
        return SSLA_ERR_ARG;
    }
    for (int b = 0; b < nb; ++b)
        if (ns[b] < 0 || (ns[b] > 0 && !rings[b])) {
            set_error("drain_batch_noalloc: bad ring / count for block " + std::to_string(b));
            return SSLA_ERR_ARG;
        }
    unsigned char* base = nullptr;
    rc = na_scratch(&base);
    if (rc) return rc;
    float* rows = reinterpret_cast<float*>(base);
    float* pack = reinterpret_cast<float*>(base + kNaPackOff);
    LiveDesc* desc = reinterpret_cast<LiveDesc*>(base + kNaDescOff);
    for (int c0 = 0; c0 < nb; c0 += kNaDescChunk) {
        DescChunk c;
        std::memset(&c, 0, sizeof c);
        const int n = std::min(kNaDescChunk, nb - c0);
        for (int k = 0; k < n; ++k) {
            const int b = c0 + k;
            LiveDesc& d = c.d[k];
            live_desc_state(cfg, b, &d);
            d.ring = rings[b];
            d.ring_mask = ~0ull;
            d.n = ns[b];
            d.scratch = rows + kNaRowFloats * b;
            d.out = outs ? outs[b] : nullptr;
            d.head_out = head_outs ? head_outs[b] : nullptr;
        }
        hipLaunchKernelGGL(k_put_desc, dim3(1), dim3(64), 0, st, c, n, desc + c0);
    }
    LHIP(hipGetLastError());
    LHIP(pack_weights(W.L, pack, &W.pk, st));
    hipLaunchKernelGGL(k_batch_drain, dim3(nb), dim3(LT), 0, st, (const LiveDesc*)desc, W, G,
                       batch);
    LHIP(hipGetLastError());
    return SSLA_OK;
}

// ---------------------------------------------------------------------------
// group launches: device resources and checks
// ---------------------------------------------------------------------------
// Exchange words, the tdrop counter copies of members 1..G-1 and both weight
// packings (ProjPack for the projections, OutPackT for the goW fragments).
struct GroupRes {
    unsigned long long* xb = nullptr;
    unsigned long long* hb = nullptr;
    unsigned char* tdrep = nullptr;
    float* pack = nullptr;
    float* packT = nullptr;
    unsigned* vsh = nullptr;
    size_t xcap = 0, hcap = 0, tdcap = 0, vcap = 0;      // bytes allocated
    void release() {
        if (vsh) (void)hipFree(vsh);
        if (xb) (void)hipFree(xb);
        if (hb) (void)hipFree(hb);
        if (tdrep) (void)hipFree(tdrep);
        if (pack) (void)hipFree(pack);
        if (packT) (void)hipFree(packT);
        *this = GroupRes{};
    }
};

// Grows a buffer to at least `need` bytes (keeps it when large enough).
static int grow(void** p, size_t* cap, size_t need) {
    if (*cap >= need && *p) return SSLA_OK;
    if (*p) LHIP(hipFree(*p));
    *p = nullptr;
    *cap = 0;
    LHIP(hipMalloc(p, need));
    *cap = need;
    return SSLA_OK;
}

// Every member of every group must be resident at once: members wait on
// each other.
static int group_check(int nb, int group, int stages = 1) {
    if (group < kGroupMin || group > kGroupMax) {
        set_error("group must be 1 or in [" + std::to_string(kGroupMin) + ", " +
                  std::to_string(kGroupMax) + "]");
        return SSLA_ERR_ARG;
    }
    if (stages != 1 && stages != 2) {
        set_error("stages must be 1 or 2");
        return SSLA_ERR_ARG;
    }
    int per_cu = 0, cus = 0, dev = 0;
    LHIP(hipOccupancyMaxActiveBlocksPerMultiprocessor(&per_cu, k_group<true, 1>, LT, 0));
    LHIP(hipGetDevice(&dev));
    LHIP(hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev));
    if ((long long)nb * group * stages > (long long)per_cu * cus) {
        set_error("n_blocks x group x stages workgroups (" + std::to_string(nb * group * stages) +
                  ") do not fit on the device at once (" + std::to_string(per_cu * cus) + ")");
        return SSLA_ERR_ARG;
    }
    return SSLA_OK;
}

// Allocates r, clears the exchange (and hand-off) words, copies each block's
// counters for members 1..group-1 of each stage and packs the weights, all
// on st; fills ga and W->pk.  On error the caller releases r.
static int group_setup(const HybridS2S3Config* cfg, const Geometry& G, int group, hipStream_t st,
                       LiveWeights* W, GroupRes* r, GroupArgs* ga, int stages = 1) {
    const int nb = G.nb;
    const size_t xbytes = sizeof(unsigned long long) * kXStride * nb * stages;
    const size_t per = (size_t)(G.C2 + G.C3);
    // buffers are grown only when r's are too small (a cached r allocates
    // nothing on later calls of the same or smaller sizes)
    int rc = grow((void**)&r->xb, &r->xcap, xbytes);
    if (!rc) rc = grow((void**)&r->tdrep, &r->tdcap, (size_t)nb * stages * (group - 1) * per);
    if (!rc) rc = grow((void**)&r->vsh, &r->vcap, sizeof(unsigned) * nb * (size_t)G.C3);
    if (rc) return rc;
    if (!r->pack) LHIP(hipMalloc(&r->pack, sizeof(float) * packed_weight_floats()));
    if (!r->packT) LHIP(hipMalloc(&r->packT, sizeof(float) * packed_weight_floats_d()));
    LHIP(hipMemsetAsync(r->xb, 0, xbytes, st));
    if (stages == 2) {
        const size_t hbytes = sizeof(unsigned long long) * kHStride * nb;
        if ((rc = grow((void**)&r->hb, &r->hcap, hbytes))) return rc;
        LHIP(hipMemsetAsync(r->hb, 0, hbytes, st));
    }
    for (int b = 0; b < nb * stages; ++b)
        for (int m = 0; m < group - 1; ++m) {
            unsigned char* dst = r->tdrep + ((size_t)b * (group - 1) + m) * per;
            const int blk = b / stages;
            LHIP(hipMemcpyAsync(dst, cfg->tdrop_s2[blk], (size_t)G.C2, hipMemcpyDeviceToDevice, st));
            LHIP(hipMemcpyAsync(dst + G.C2, cfg->tdrop_s3[blk], (size_t)G.C3, hipMemcpyDeviceToDevice, st));
        }
    LHIP(pack_weights(W->L, r->pack, &W->pk, st));
    PackedWeights pt{};
    LHIP(pack_weights_d(W->L, r->packT, &pt, st));
    ga->xb = r->xb;
    ga->hb = r->hb;
    ga->tdrep = r->tdrep;
    ga->vsh = r->vsh;
    ga->stages = stages;
    ga->goT[0] = pt.po[0] + OutPackT<SSLA_C1, SSLA_C2>::Q;
    ga->goT[1] = pt.po[1] + OutPackT<SSLA_C2, SSLA_C2>::Q;
    ga->goT[2] = pt.po[2] + OutPackT<SSLA_C2, SSLA_C3>::Q;
    ga->goT[3] = pt.po[3] + OutPackT<SSLA_C3, SSLA_C3>::Q;
    ga->ipT[0] = ga->goT[0] + OutPackT<SSLA_C1, SSLA_C2>::GO;
    ga->ipT[1] = nullptr;
    ga->ipT[2] = ga->goT[2] + OutPackT<SSLA_C2, SSLA_C3>::GO;
    ga->ipT[3] = nullptr;
    int khz = 0;
    LHIP(hipDeviceGetAttribute(&khz, hipDeviceAttributeWallClockRate, 0));
    if (khz <= 0) khz = 100000;
    ga->wait_ticks = 2000ull * (unsigned long long)khz;   // 2 s
    ga->G = group;
    return SSLA_OK;
}

// The group batch drain's device resources, kept per device across calls
// (under g_bmu): after a device's first call of a size, calls allocate nothing.
struct GroupBatchCache {
    GroupRes r;
    LiveDesc* desc = nullptr;                  // SSLA_MAX_BLOCKS
    int* status = nullptr;
    unsigned long long* prof = nullptr;        // NPROF x SSLA_MAX_BLOCKS
};
static std::map<int, GroupBatchCache> g_group_batch;

int batch_drain_group(const HybridS2S3Config* cfg, const HybridInputRec* const* rings, const int* ns,
                      HybridS2S3OutputSlot* const* outs, float* const* head_outs, int batch,
                      int group, hipStream_t st, double* phase_us) {
    LiveWeights W;
    Geometry G;
    int rc = live_weights(cfg, &W, &G);
    if (rc) return rc;
    if (batch < 1 || batch > LB) {
        set_error("batch must be in [1, 32]");
        return SSLA_ERR_ARG;
    }
    const int nb = cfg->n_blocks;
    for (int b = 0; b < nb; ++b)
        if (ns[b] < 0 || (ns[b] > 0 && !rings[b])) {
            set_error("bad ring / count for block " + std::to_string(b));
            return SSLA_ERR_ARG;
        }
    if ((rc = group_check(nb, group))) return rc;
    int dev = 0;
    LHIP(hipGetDevice(&dev));
    std::lock_guard<std::mutex> lk(g_bmu);
    GroupBatchCache& c = g_group_batch[dev];
    // every exit waits for the stream: work queued on the cached buffers must
    // be done before the next call reuses them (also after an error)
    struct SyncAtExit {
        hipStream_t st;
        ~SyncAtExit() { (void)hipStreamSynchronize(st); }
    } sync_at_exit{st};
    GroupArgs ga{};
    if ((rc = group_setup(cfg, G, group, st, &W, &c.r, &ga))) return rc;
    if (!c.desc) LHIP(hipMalloc(&c.desc, sizeof(LiveDesc) * SSLA_MAX_BLOCKS));
    if (!c.status) LHIP(hipMalloc(&c.status, sizeof(int)));
    if (phase_us && !c.prof)
        LHIP(hipMalloc(&c.prof, sizeof(unsigned long long) * NPROF * SSLA_MAX_BLOCKS));
    LHIP(hipMemsetAsync(c.status, 0, sizeof(int), st));
    std::vector<LiveDesc> hd(nb);
    std::memset(hd.data(), 0, sizeof(LiveDesc) * nb);
    for (int b = 0; b < nb; ++b) {
        LiveDesc& d = hd[b];
        live_desc_state(cfg, b, &d);
        d.ring = rings[b];
        d.ring_mask = ~0ull;
        d.n = ns[b];
        d.out = outs ? outs[b] : nullptr;
        d.head_out = head_outs ? head_outs[b] : nullptr;
        d.prof = phase_us ? c.prof + (size_t)NPROF * b : nullptr;
    }
    LHIP(hipMemcpyAsync(c.desc, hd.data(), sizeof(LiveDesc) * nb, hipMemcpyHostToDevice, st));
    hipLaunchKernelGGL((k_group<false, 1>), dim3(nb * group), dim3(LT), 0, st, c.desc, W, G, ga,
                       (const int*)nullptr, 0u, 0ull, batch, c.status);
    LHIP(hipGetLastError());
    LHIP(hipStreamSynchronize(st));
    int hs = 0;
    LHIP(hipMemcpy(&hs, c.status, sizeof(int), hipMemcpyDeviceToHost));
    if (hs) {
        set_error("group drain: a member's wait ran out (status " + std::to_string(hs) + ")");
        return SSLA_ERR_STATE;
    }
    if (phase_us) {
        std::vector<unsigned long long> h((size_t)NPROF * nb);
        LHIP(hipMemcpy(h.data(), c.prof, sizeof(unsigned long long) * h.size(),
                       hipMemcpyDeviceToHost));
        add_profile(h.data(), nb, phase_us);
    }
    return SSLA_OK;
}

// ---------------------------------------------------------------------------
// persistent session
// ---------------------------------------------------------------------------
struct LiveSession {
    hipStream_t stream = nullptr;
    LiveDesc* desc = nullptr;
    float* scratch = nullptr;
    int* status = nullptr;
    unsigned long long* prof = nullptr;
    double* phase_us = nullptr;
    float* pack = nullptr;
    int nb = 0;
    GroupRes grp;                       // group > 1 only
};

int live_start(const HybridS2S3Config* cfg, HybridInputRec* const* rings,
               unsigned long long ring_mask, unsigned long long* const* tails, int* stop_flag,
               unsigned long long* const* events_done, unsigned int spin_ns, int max_batch,
               unsigned int idle_timeout_ms, double* phase_us, int group, int stages,
               LiveSession** out) {
    *out = nullptr;
    LiveWeights W;
    Geometry G;
    int rc = live_weights(cfg, &W, &G);
    if (rc) return rc;
    if ((ring_mask & (ring_mask + 1)) != 0) {
        set_error("ring capacity must be a power of two (ring_mask = capacity - 1)");
        return SSLA_ERR_ARG;
    }
    if (max_batch < 1 || max_batch > LB) {
        set_error("max_batch must be in [1, 32]");
        return SSLA_ERR_ARG;
    }
    if (!stop_flag) {
        set_error("stop_flag is required");
        return SSLA_ERR_ARG;
    }
    const int nb = cfg->n_blocks;
    if (stages < 1) stages = 1;
    if (stages > 1 && (cfg->W2 > 4096 || cfg->H2 > 4096)) {
        set_error("two stages hand s2 coordinates over in 12 bits: W2 and H2 must be <= 4096");
        return SSLA_ERR_ARG;
    }
    if (stages > 1 && group <= 1) {
        set_error("two stages need a group (3..6 workgroups per stage)");
        return SSLA_ERR_ARG;
    }
    if (group > 1 && (rc = group_check(nb, group, stages))) return rc;
    for (int b = 0; b < nb; ++b) {
        if (!rings[b] || !tails[b]) {
            set_error("every block needs a ring and a tail");
            return SSLA_ERR_ARG;
        }
        if (cfg->timing[b] && (cfg->timing_mask & (cfg->timing_mask + 1)) != 0) {
            set_error("timing_mask must be capacity - 1 of a power of two");
            return SSLA_ERR_ARG;
        }
    }
    int khz = 0;
    LHIP(hipDeviceGetAttribute(&khz, hipDeviceAttributeWallClockRate, 0));
    if (khz <= 0) khz = 100000;
    LiveSession* s = new LiveSession();
    s->nb = nb;
    auto fail = [&](const char* what) {
        set_error(std::string(what) + " failed while starting the live drain");
        if (s->stream) (void)hipStreamDestroy(s->stream);
        if (s->desc) (void)hipFree(s->desc);
        if (s->scratch) (void)hipFree(s->scratch);
        if (s->status) (void)hipFree(s->status);
        if (s->prof) (void)hipFree(s->prof);
        if (s->pack) (void)hipFree(s->pack);
        s->grp.release();
        delete s;
        return SSLA_ERR_HIP;
    };
    if (hipStreamCreateWithFlags(&s->stream, hipStreamNonBlocking) != hipSuccess) return fail("stream");
    const size_t sbytes = sizeof(float) * scratch_floats() * nb;
    if (hipMalloc(&s->scratch, sbytes) != hipSuccess) return fail("scratch");
    if (hipMalloc(&s->desc, sizeof(LiveDesc) * nb) != hipSuccess) return fail("desc");
    if (hipMalloc(&s->status, sizeof(int)) != hipSuccess) return fail("status");
    GroupArgs ga{};
    if (group > 1) {
        if (group_setup(cfg, G, group, s->stream, &W, &s->grp, &ga, stages) != SSLA_OK)
            return fail("group set-up");
    } else {
        if (hipMalloc(&s->pack, sizeof(float) * packed_weight_floats()) != hipSuccess) return fail("weights");
        if (pack_weights(W.L, s->pack, &W.pk, s->stream) != hipSuccess) return fail("weight packing");
    }
    if (phase_us) {
        if (hipMalloc(&s->prof, sizeof(unsigned long long) * NPROF * nb) != hipSuccess) return fail("profile");
        s->phase_us = phase_us;
    }
    std::vector<LiveDesc> hd(nb);
    std::memset(hd.data(), 0, sizeof(LiveDesc) * nb);
    for (int b = 0; b < nb; ++b) {
        LiveDesc& d = hd[b];
        live_desc_state(cfg, b, &d);
        d.ring = rings[b];
        d.ring_mask = ring_mask;
        d.tail = tails[b];
        d.events_done = events_done ? events_done[b] : nullptr;
        d.scratch = s->scratch + scratch_floats() * b;
        d.timing = cfg->timing[b];
        d.timing_mask = cfg->timing_mask;
        d.kstart = cfg->kernel_start_clk[b];
        d.kend = cfg->kernel_end_clk[b];
        d.clk_sync = timing_clock_sync(cfg, b);
        d.prof = s->prof ? s->prof + (size_t)NPROF * b : nullptr;
        // the tail (host memory) does not move while no kernel drains the ring
        d.t0 = *reinterpret_cast<volatile unsigned long long*>(tails[b]);
    }
    if (hipMemsetAsync(s->scratch, 0, sbytes, s->stream) != hipSuccess) return fail("memset");
    if (hipMemsetAsync(s->status, 0, sizeof(int), s->stream) != hipSuccess) return fail("memset");
    if (hipMemcpyAsync(s->desc, hd.data(), sizeof(LiveDesc) * nb, hipMemcpyHostToDevice, s->stream) != hipSuccess)
        return fail("copy");
    if (hipStreamSynchronize(s->stream) != hipSuccess) return fail("sync");
    const unsigned long long idle = (unsigned long long)idle_timeout_ms * (unsigned long long)khz;
    if (group > 1 && stages == 2)
        hipLaunchKernelGGL((k_group<true, 2>), dim3(nb * group * 2), dim3(LT), 0, s->stream, s->desc, W, G, ga,
                           stop_flag, spin_ns, idle, max_batch, s->status);
    else if (group > 1)
        hipLaunchKernelGGL((k_group<true, 1>), dim3(nb * group), dim3(LT), 0, s->stream, s->desc, W, G, ga,
                           stop_flag, spin_ns, idle, max_batch, s->status);
    else
        hipLaunchKernelGGL(k_live, dim3(nb), dim3(LT), 0, s->stream, s->desc, W, G, stop_flag, spin_ns,
                           idle, max_batch, s->status);
    if (hipGetLastError() != hipSuccess) return fail("launch");
    *out = s;
    return SSLA_OK;
}

int live_wait(LiveSession* s, int timeout_ms, int* status_out) {
    if (!s) {
        set_error("null session");
        return SSLA_ERR_ARG;
    }
    const auto t0 = std::chrono::steady_clock::now();
    while (true) {
        const hipError_t q = hipStreamQuery(s->stream);
        if (q == hipSuccess) break;
        if (q != hipErrorNotReady) {
            set_error(std::string("live drain failed: ") + hipGetErrorString(q));
            return SSLA_ERR_HIP;
        }
        const double ms = std::chrono::duration<double, std::milli>(std::chrono::steady_clock::now() - t0).count();
        if (timeout_ms >= 0 && ms > timeout_ms) {
            set_error("live drain still running (set *stop_flag first; the kernel also stops on its idle timeout)");
            return SSLA_ERR_STATE;
        }
        std::this_thread::sleep_for(std::chrono::microseconds(200));
    }
    int st = 0;
    LHIP(hipMemcpy(&st, s->status, sizeof(int), hipMemcpyDeviceToHost));
    if (status_out) *status_out = st;
    if (s->prof) {
        std::vector<unsigned long long> h((size_t)NPROF * s->nb);
        LHIP(hipMemcpy(h.data(), s->prof, sizeof(unsigned long long) * h.size(), hipMemcpyDeviceToHost));
        add_profile(h.data(), s->nb, s->phase_us);
        (void)hipFree(s->prof);
    }
    if (s->pack) (void)hipFree(s->pack);
    s->grp.release();
    (void)hipStreamDestroy(s->stream);
    (void)hipFree(s->desc);
    (void)hipFree(s->scratch);
    (void)hipFree(s->status);
    delete s;
    return SSLA_OK;
}

}  // namespace ssla
