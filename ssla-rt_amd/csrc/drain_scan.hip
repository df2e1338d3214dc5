// drain_scan.hip -- whole-ring drain of SSLA-S s2 + s3 + YOLOX head on gfx950.
//
// The reference drains a ring 8 records at a time in one 9-warp block per
// ring (orin/kernels/ssla_s2_s3_head_celled.cuh:914-1255), so at most 8
// records are in flight per block.  This file re-derives the same result
// for a whole pre-filled ring at once, using the structure of one SSLA layer
// (orin/orin/ssla_ref.py:17-93):
//
//   for every in-bounds patch cell c of event e (offset delta):
//       q, v, g = qvgIn[delta] x_e                    (depends on x_e only)
//       h_c     = sigmoid(g) * h_c + v                (ordered per cell)
//       qh      = q * h_c
//   y_e = LN( sum_delta goW[delta] qh + residual(x_e) )
//
// Only the h_c recurrence is ordered, and only among events touching the
// same cell.  Per layer the drain therefore runs three phases over all
// records of all rings:
//   P  (k_qvg)   v, g for every (record, delta) pair as MFMA tiles,
//                written in per-cell ring order (pair rows sorted by
//                target cell)
//   S  (k_scan)  chunked per-cell scan: turns (v, g) rows into h rows in
//                place, in ring order, where the layer's output is used
//   O  (k_out)   per output record: q = qvgIn[delta] x by MFMA, times the
//                <= 9 h rows, contracted with goW by MFMA, residual, fp64
//                LayerNorm
// The temporal-dropout decisions (ssla_ref.py:190-195) depend only on the
// per-cell arrival rank of a record, so they come from a stable sort of
// records by cell: pass = ((counter + rank) mod 256) % window == 0.
// Results equal sequential processing in ring order up to fp32 summation
// order; drop decisions are bit-exact.
//
// Device layouts are those of include/ssla_abi.h.
#include <hip/hip_runtime.h>

#include <cstdint>
#include <cstdio>
#include <atomic>
#include <cstring>
#include <mutex>
#include <string>
#include <vector>

#include "drain_common.h"
#include "drain_scan.h"
#include "mfma_pack.h"

namespace ssla {

namespace {


struct BlockDesc {
    const HybridInputRec* ring;
    HybridS2S3OutputSlot* out;
    float*                head_out;
    float*                hidden[4];
    unsigned char*        td2;
    unsigned char*        td3;
    float*                preds;
    unsigned int*         version;
    HybridStrip           strip;
    int                   n;
    int                   offset;
};

// The block table travels to the device as kernel arguments of k_decode
// (the runtime copies them at launch, so a call never waits on the host for
// a staging buffer the previous call may still be reading); k_decode reads
// it there and writes the copy the later kernels read.
struct BlockTable {
    BlockDesc d[SSLA_MAX_BLOCKS];
};
static_assert(sizeof(BlockTable) <= 2048, "kernel argument block");

__device__ __forceinline__ int find_block(const BlockDesc* bd, int nb, int g) {
    int b = 0;
    for (int i = 1; i < nb; ++i)
        if (g >= bd[i].offset) b = i;
    return b;
}

// ---------------------------------------------------------------------------
// decode: ring records -> compact features, centre cells, sort keys
// ---------------------------------------------------------------------------
// Eight lanes per 128-byte record, one 16-byte load each: lanes 1..6 move the
// feat1 quarters, lane 0 also writes the keys.
constexpr int kDecRec = 32;          // records per 256-thread workgroup

// Up to kFills int arrays set to a value each (k_decode's extra blocks).
constexpr int kFills = 7;
struct FillSet {
    int* p[kFills];
    int n[kFills];
    int v[kFills];
};

// One launch for the call's set-up: blocks [0, ndec) decode the records,
// then fblk blocks per fill array, then npk blocks rebuild the fragment-order
// weight copies (one float per thread), and the last block writes the block
// table for the later kernels.  Nothing in this launch reads what another of
// its blocks writes.
__global__ void __launch_bounds__(256)
k_decode(int E, BlockTable tab, BlockDesc* __restrict__ bd_out, Geometry G,
         float* __restrict__ X0, int* __restrict__ cell2,
         unsigned char* __restrict__ owner,
         uint32_t* __restrict__ key2, uint32_t* __restrict__ val2, int ndec, FillSet f, int fblk,
         PackSrc ps, float* __restrict__ pbuf, int npk) {
    const int nfill = fblk * kFills;
    if ((int)blockIdx.x >= ndec) {
        const int xb = (int)blockIdx.x - ndec;
        if (xb < nfill) {
            // the call's fills: fblk blocks of 256 per array
            const int a = xb / fblk;
            const int i = (xb - a * fblk) * 256 + (int)threadIdx.x;
            if (i < f.n[a]) f.p[a][i] = f.v[a];
        } else if (xb < nfill + npk) {
            const size_t q = (size_t)(xb - nfill) * 256 + threadIdx.x;
            if (q < PackLayout<true>::off[8]) pack_elem<true>(ps, pbuf, q);
        } else if (threadIdx.x < SSLA_MAX_BLOCKS) {
            bd_out[threadIdx.x] = tab.d[threadIdx.x];
        }
        return;
    }
    const int g = blockIdx.x * kDecRec + (threadIdx.x >> 3);
    const int c = threadIdx.x & 7;
    if (g >= E) return;
    int b = 0;
    for (int i = 1; i < G.nb; ++i)
        if (g >= tab.d[i].offset) b = i;
    const HybridInputRec* r = tab.d[b].ring + (g - tab.d[b].offset);
    const float4 v = reinterpret_cast<const float4*>(r)[c];
    const int x = r->x, y = r->y;
    const bool valid = x < G.W2 && y < G.H2;
    if (c >= 1 && c <= SSLA_C1 / 4)
        reinterpret_cast<float4*>(X0 + (size_t)g * SSLA_C1)[c - 1] =
            valid ? v : make_float4(0.f, 0.f, 0.f, 0.f);
    if (c != 0) return;
    const HybridStrip& s = tab.d[b].strip;
    owner[g] = (valid && x >= s.owned_lo && x < s.owned_hi &&
                y >= s.owned_y_lo && y < s.owned_y_hi) ? 1 : 0;
    const uint32_t none = (uint32_t)(G.nb * G.C2);
    cell2[g] = valid ? y * G.W2 + x : -1;
    key2[g] = valid ? (uint32_t)(b * G.C2 + y * G.W2 + x) : none;
    val2[g] = (uint32_t)g;
}



// ---------------------------------------------------------------------------
// Stable LSD radix sort of (key, record) pairs, digits of up to 9 bits.
// Records are taken in tiles of kRTile (256 threads x 8 rounds, round r =
// records base + 256 r .. + 255).  Per pass:
//   k_rs_hist     digit counts of every tile            -> bh[digit * T + tile]
//   k_exscan      exclusive scan of bh (digit-major)    -> first slot of every
//                                                          (digit, tile)
//   k_rs_scatter  each record to its (digit, tile) start + its rank among
//                 the tile's earlier records of the digit: inside a wave from
//                 the lanes whose digit equals its own (one ballot per digit
//                 bit), across the round's waves and rounds from LDS counts.
// ---------------------------------------------------------------------------
constexpr int kRThreads = 256, kRRounds = 8, kRTile = kRThreads * kRRounds;
constexpr int kRMaxBits = 9;

__global__ void __launch_bounds__(kRThreads)
k_rs_hist(int n, const uint32_t* __restrict__ keys, int shift, int bits, int nbins, int T,
          int* __restrict__ bh) {
    __shared__ int h[1 << kRMaxBits];
    const int nb = 1 << bits, tid = threadIdx.x;
    for (int i = tid; i < nb; i += kRThreads) h[i] = 0;
    __syncthreads();
    const int base = blockIdx.x * kRTile;
    #pragma unroll 4
    for (int r = 0; r < kRRounds; ++r) {
        const int idx = base + r * kRThreads + tid;
        if (idx < n) atomicAdd(&h[(keys[idx] >> shift) & (nb - 1)], 1);
    }
    __syncthreads();
    for (int i = tid; i < nbins; i += kRThreads) bh[(size_t)i * T + blockIdx.x] = h[i];
}

// vin null: the values are the record indices.  sidx (last pass, optional):
// sidx[value] = the value's sorted position.
__global__ void __launch_bounds__(kRThreads)
k_rs_scatter(int n, const uint32_t* __restrict__ kin, const uint32_t* __restrict__ vin,
             uint32_t* __restrict__ kout, uint32_t* __restrict__ vout, int* __restrict__ sidx,
             int shift, int bits, int nbins, int T, const int* __restrict__ boff) {
    __shared__ int cnt[1 << kRMaxBits];
    __shared__ int wcnt[kRThreads / 64][1 << kRMaxBits];
    const int nb = 1 << bits, tid = threadIdx.x, wv = tid >> 6, lane = tid & 63;
    for (int i = tid; i < nbins; i += kRThreads) {
        cnt[i] = boff[(size_t)i * T + blockIdx.x];
        #pragma unroll
        for (int w = 0; w < kRThreads / 64; ++w) wcnt[w][i] = 0;
    }
    __syncthreads();
    const unsigned long long below = (1ull << lane) - 1ull;
    const int base = blockIdx.x * kRTile;
    for (int r = 0; r < kRRounds; ++r) {
        const int idx = base + r * kRThreads + tid;
        const bool valid = idx < n;
        const uint32_t key = valid ? kin[idx] : 0u;
        const int dig = (int)((key >> shift) & (uint32_t)(nb - 1));
        unsigned long long peers = __ballot(valid);
        for (int b = 0; b < bits; ++b) {
            const bool bit = (dig >> b) & 1;
            const unsigned long long m = __ballot(bit);
            peers &= bit ? m : ~m;
        }
        const int rank = __popcll(peers & below), size = __popcll(peers);
        const bool leader = valid && rank == 0;
        if (leader) wcnt[wv][dig] = size;
        __syncthreads();
        if (valid) {
            int pos = cnt[dig] + rank;
            for (int w = 0; w < wv; ++w) pos += wcnt[w][dig];
            const uint32_t v = vin ? vin[idx] : (uint32_t)idx;
            kout[pos] = key;
            vout[pos] = v;
            if (sidx) sidx[v] = pos;
        }
        __syncthreads();
        if (leader) {
            atomicAdd(&cnt[dig], size);
            wcnt[wv][dig] = 0;
        }
        __syncthreads();
    }
}

// ---------------------------------------------------------------------------
// One workgroup scans arrays of any length in rounds of kScanThreads x 8
// elements: each thread loads 8 consecutive elements with two 16-byte loads,
// the thread totals are scanned in LDS, and a running carry joins the rounds.
// Arrays are 256-byte aligned workspace buffers (16-byte loads stay in them;
// elements at or past n read as zero and are not written).
// ---------------------------------------------------------------------------
constexpr int kScanThreads = 1024, kScanPer = 8, kScanRound = kScanThreads * kScanPer;

// exclusive prefix of v over the workgroup; *total receives the sum
__device__ __forceinline__ int block_exscan(int v, int* lds, int* total) {
    const int tid = threadIdx.x, lane = tid & 63, wv = tid >> 6;
    int x = v;
    #pragma unroll
    for (int o = 1; o < 64; o <<= 1) {
        const int y = __shfl_up(x, o, 64);
        if (lane >= o) x += y;
    }
    if (lane == 63) lds[wv] = x;
    __syncthreads();
    if (wv == 0) {
        int w = lane < kScanThreads / 64 ? lds[lane] : 0;
        #pragma unroll
        for (int o = 1; o < kScanThreads / 64; o <<= 1) {
            const int y = __shfl_up(w, o, 64);
            if (lane >= o) w += y;
        }
        if (lane < kScanThreads / 64) lds[kScanThreads / 64 + lane] = w;
    }
    __syncthreads();
    const int before = (wv ? lds[kScanThreads / 64 + wv - 1] : 0) + x - v;
    *total = lds[2 * (kScanThreads / 64) - 1];
    __syncthreads();
    return before;
}

__device__ __forceinline__ void load8(const int* a, int i0, int n, int (&v)[kScanPer]) {
    if (i0 + kScanPer <= n) {
        const int4 x = reinterpret_cast<const int4*>(a + i0)[0];
        const int4 y = reinterpret_cast<const int4*>(a + i0)[1];
        v[0] = x.x; v[1] = x.y; v[2] = x.z; v[3] = x.w;
        v[4] = y.x; v[5] = y.y; v[6] = y.z; v[7] = y.w;
    } else {
        #pragma unroll
        for (int q = 0; q < kScanPer; ++q) v[q] = i0 + q < n ? a[i0 + q] : 0;
    }
}

__device__ __forceinline__ void store8(int* a, int i0, int n, const int (&v)[kScanPer]) {
    if (i0 + kScanPer <= n) {
        reinterpret_cast<int4*>(a + i0)[0] = make_int4(v[0], v[1], v[2], v[3]);
        reinterpret_cast<int4*>(a + i0)[1] = make_int4(v[4], v[5], v[6], v[7]);
    } else {
        #pragma unroll
        for (int q = 0; q < kScanPer; ++q)
            if (i0 + q < n) a[i0 + q] = v[q];
    }
}

// in place: a[i] <- sum of a[0 .. i)
__global__ void __launch_bounds__(kScanThreads) k_exscan(int n, int* __restrict__ a) {
    __shared__ int lds[2 * (kScanThreads / 64)];
    int carry = 0;
    for (int r0 = 0; r0 < n; r0 += kScanRound) {
        const int i0 = r0 + (int)threadIdx.x * kScanPer;
        int v[kScanPer];
        load8(a, i0, n, v);
        int sum = 0;
        #pragma unroll
        for (int q = 0; q < kScanPer; ++q) sum += v[q];
        int total;
        int run = carry + block_exscan(sum, lds, &total);
        #pragma unroll
        for (int q = 0; q < kScanPer; ++q) {
            const int x = v[q];
            v[q] = run;
            run += x;
        }
        store8(a, i0, n, v);
        carry += total;
    }
}

constexpr int kCH = 32;     // pairs per scan chunk
constexpr int kSG = 8;      // chunks per group (workgroup) of the one-pass scan, s2 layers
constexpr int kSG3 = 4;     // ... s3 layers (two waves per chunk)

// Chunk tables: one wave per key writes its chunks (ckey, cbeg, cend) and
// counts the key's groups of the one-pass scan (ghist, gw: k_group_order).
__global__ void __launch_bounds__(256)
k_chunks(uint32_t nk, const int* __restrict__ start, const int* __restrict__ end,
         const int* __restrict__ coff, int* __restrict__ ckey, int* __restrict__ cbeg,
         int* __restrict__ cend, int* __restrict__ ghist, int* __restrict__ gw) {
    const uint32_t k = blockIdx.x * 4u + (threadIdx.x >> 6);
    if (k >= nk) return;
    const int s = start[k], e = end[k], c0 = coff[k];
    for (int q = threadIdx.x & 63; s + q * kCH < e; q += 64) {
        ckey[c0 + q] = (int)k;
        cbeg[c0 + q] = s + q * kCH;
        cend[c0 + q] = min(e, s + (q + 1) * kCH);
    }
    if ((threadIdx.x & 63) == 0) {
        const int gc = ((e - s + kCH - 1) / kCH + kSG3 - 1) / kSG3;
        if (gc > 0) gw[k] = atomicAdd(&ghist[gc], 1);
    }
}

// [start, end) of every key present in a sorted key array.
__global__ void k_runs(int n, const uint32_t* __restrict__ keys, uint32_t nk,
                       int* __restrict__ start, int* __restrict__ end) {
    const int p = blockIdx.x * blockDim.x + threadIdx.x;
    if (p >= n) return;
    const uint32_t k = keys[p];
    if (k >= nk) return;
    if (p == 0 || keys[p - 1] != k) start[k] = p;
    if (p == n - 1 || keys[p + 1] != k) end[k] = p + 1;
}

// ---------------------------------------------------------------------------
// Temporal dropout (ssla_ref.py:190-195): a cell's counter c (uint8) takes
// pre = c + rank (mod 256) for the record of arrival rank `rank`, and the
// record passes when window <= 1 or pre % window == 0.  passes(c, r, w) is
// the number of passing ranks in [0, r): with F(x) = the number of
// u in [0, x) whose (u mod 256) is a multiple of w,
//   F(x) = (x / 256) (255 / w + 1) + ceil((x mod 256) / w),
// passes(c, r, w) = F(c + r) - F(c).
// ---------------------------------------------------------------------------
__device__ __forceinline__ bool tdrop_pass(unsigned c, unsigned rank, int window) {
    return window <= 1 || ((c + rank) & 255u) % (unsigned)window == 0u;
}

__device__ __forceinline__ int tdrop_passes(unsigned c, int r, int window) {
    if (window <= 1) return r;
    const unsigned w = (unsigned)window, per = 255u / w + 1u;
    auto F = [&](unsigned x) { return (x >> 8) * per + ((x & 255u) + w - 1u) / w; };
    return (int)(F(c + (unsigned)r) - F(c));
}

// tdrop_s2 over the sorted records (position p, record g, rank r in the
// key's run, counter c before the call): pass2[g], and the pass-2 list in
// s2 order -- the record's place is the key's offset plus the number of
// passing ranks below r.  Returns pass2[g].
__device__ __forceinline__ bool
tdrop2_at(int p, int n, const uint32_t* __restrict__ keys, const uint32_t* __restrict__ vals,
          uint32_t nk, const int* __restrict__ start, const unsigned char* __restrict__ old,
          const int* __restrict__ off, int window, unsigned char* __restrict__ pass,
          int* __restrict__ list) {
    if (p >= n) return false;
    const uint32_t k = keys[p];
    const int g = (int)vals[p];
    if (k >= nk) {
        pass[g] = 0;
        return false;
    }
    const int r = p - start[k];
    const unsigned c = old[k];
    const bool take = tdrop_pass(c, (unsigned)r, window);
    pass[g] = take ? 1 : 0;
    if (take) list[off[k] + tdrop_passes(c, r, window)] = g;
    return take;
}


// Per s2 key: the counter before this call (old[k]), the counter after it,
// the number of pass-2 records of the run (n2[k]) and the pair count of the
// key (the run lengths of its 3 x 3 neighbourhood).
__global__ void k_keys2(uint32_t nk, int C, int W, int H, const int* __restrict__ st,
                        const int* __restrict__ en, const BlockDesc* __restrict__ bd, int window,
                        unsigned char* __restrict__ old, int* __restrict__ n2,
                        int* __restrict__ pcnt) {
    const uint32_t t = blockIdx.x * blockDim.x + threadIdx.x;
    if (t >= nk) return;
    const int b = (int)t / C, cell = (int)t % C, ty = cell / W, tx = cell % W;
    const int len = en[t] - st[t];
    unsigned char* td = bd[b].td2 + cell;
    const unsigned c = *td;
    old[t] = (unsigned char)c;
    n2[t] = tdrop_passes(c, len, window);
    *td = (unsigned char)((c + (unsigned)len) & 255u);
    int np = 0;
    #pragma unroll
    for (int oy = -1; oy <= 1; ++oy)
        #pragma unroll
        for (int ox = -1; ox <= 1; ++ox) {
            const int sy = ty + oy, sx = tx + ox;
            if (sy < 0 || sy >= H || sx < 0 || sx >= W) continue;
            const int s = b * C + sy * W + sx;
            np += en[s] - st[s];
        }
    pcnt[t] = np;
}

// The per-key tables of k_keys2 (and k_runs) for a one-pass record sort,
// whose digit is the whole key: the scanned tile histogram bh (bin-major, T
// tiles) holds the run bounds, key t's run being [bh[t T], bh[(t + 1) T]).
// key2_at writes st / en / old and the committed counter, and returns the
// key's pair count and pass-2 count (used by k_keyscan<true>).
struct KeyHist {
    int C, W, H, T, window;
    const int* bh;
    int* st;
    int* en;
    const BlockDesc* bd;
    unsigned char* old;
};

__device__ __forceinline__ void key2_at(uint32_t t, const KeyHist& kh, int& pc, int& n2v) {
    const int b = (int)t / kh.C, cell = (int)t % kh.C, ty = cell / kh.W, tx = cell % kh.W;
    const int s0 = kh.bh[(size_t)t * kh.T], len = kh.bh[(size_t)(t + 1) * kh.T] - s0;
    kh.st[t] = s0;
    kh.en[t] = s0 + len;
    unsigned char* td = kh.bd[b].td2 + cell;
    const unsigned c = *td;
    kh.old[t] = (unsigned char)c;
    n2v = tdrop_passes(c, len, kh.window);
    *td = (unsigned char)((c + (unsigned)len) & 255u);
    int np = 0;
    #pragma unroll
    for (int oy = -1; oy <= 1; ++oy)
        #pragma unroll
        for (int ox = -1; ox <= 1; ++ox) {
            const int sy = ty + oy, sx = tx + ox;
            if (sy < 0 || sy >= kh.H || sx < 0 || sx >= kh.W) continue;
            const size_t q = (size_t)(b * kh.C + sy * kh.W + sx);
            np += kh.bh[(q + 1) * kh.T] - kh.bh[q * kh.T];
        }
    pc = np;
}

// Per-key tables from per-key counts (k < nk), in one launch:
//   cnt  -> start (exclusive scan), end = start + cnt (end may be cnt itself);
//           with coff: coff[k] = the key's first chunk of kCH, *n_chunks;
//   cnt2 (optional) -> off2 (exclusive scan), *total2.
// KH: the counts come from key2_at (a one-pass sort's histogram, kh; nk <=
// kScanThreads) instead of cnt / cnt2, and cnt2 then receives the pass-2
// counts.
template <bool KH>
__global__ void __launch_bounds__(kScanThreads)
k_keyscan(int nk, const int* cnt, int* __restrict__ start, int* end, int* __restrict__ coff,
          int* __restrict__ n_chunks, const int* __restrict__ cnt2, int* __restrict__ off2,
          int* __restrict__ total2, KeyHist kh) {
    __shared__ int lds[2 * (kScanThreads / 64)];
    __shared__ int kv[KH ? kScanThreads : 1], ku[KH ? kScanThreads : 1];
    int carry = 0, ccarry = 0, carry2 = 0;
    for (int r0 = 0; r0 < nk; r0 += kScanRound) {
        const int i0 = r0 + (int)threadIdx.x * kScanPer;
        int v[kScanPer], c[kScanPer], u[kScanPer];
        if constexpr (KH) {
            // one key per thread (nk <= kScanThreads), through LDS into the
            // eight-per-thread layout of the scan
            const int t = (int)threadIdx.x;
            int pc = 0, p2 = 0;
            if (t < nk) {
                key2_at((uint32_t)t, kh, pc, p2);
                const_cast<int*>(cnt2)[t] = p2;
            }
            kv[t] = pc;
            ku[t] = p2;
            __syncthreads();
            #pragma unroll
            for (int q = 0; q < kScanPer; ++q) {
                const bool in = i0 + q < kScanThreads;
                v[q] = in ? kv[i0 + q] : 0;
                u[q] = in ? ku[i0 + q] : 0;
            }
        } else {
            load8(cnt, i0, nk, v);
            if (cnt2) load8(cnt2, i0, nk, u);
        }
        int s = 0, sc = 0, su = 0;
        #pragma unroll
        for (int q = 0; q < kScanPer; ++q) {
            s += v[q];
            c[q] = (v[q] + kCH - 1) / kCH;
            sc += c[q];
            if (cnt2) su += u[q];
        }
        int total;
        int run = carry + block_exscan(s, lds, &total);
        carry += total;
        int crun = 0, urun = 0;
        if (coff) {
            crun = ccarry + block_exscan(sc, lds, &total);
            ccarry += total;
        }
        if (cnt2) {
            urun = carry2 + block_exscan(su, lds, &total);
            carry2 += total;
        }
        int st[kScanPer], en[kScanPer];
        #pragma unroll
        for (int q = 0; q < kScanPer; ++q) {
            st[q] = run;
            run += v[q];
            en[q] = run;
            const int x = c[q];
            c[q] = crun;
            crun += x;
            const int y = u[q];
            u[q] = urun;
            urun += y;
        }
        store8(start, i0, nk, st);
        store8(end, i0, nk, en);
        if (coff) store8(coff, i0, nk, c);
        if (cnt2) store8(off2, i0, nk, u);
    }
    if (threadIdx.x == 0) {
        if (coff) *n_chunks = ccarry;
        if (cnt2) *total2 = carry2;
    }
}

// Per s3 key: the number of pass-2 records of its four s2 cells (t3, the
// length of its run in the s3 order) and how many of them pass tdrop_s3.
__global__ void k_keys3a(uint32_t nk3, Geometry G, const int* __restrict__ n2,
                         const BlockDesc* __restrict__ bd, int* __restrict__ t3,
                         int* __restrict__ n3) {
    const uint32_t k = blockIdx.x * blockDim.x + threadIdx.x;
    if (k >= nk3) return;
    const int b = (int)k / G.C3, cell = (int)k % G.C3;
    const int x = 2 * (cell % G.W3), y = 2 * (cell / G.W3);
    const int s = b * G.C2 + y * G.W2 + x;
    const int t = n2[s] + n2[s + 1] + n2[s + G.W2] + n2[s + G.W2 + 1];
    t3[k] = t;
    n3[k] = tdrop_passes(bd[b].td3[cell], t, G.window);
}

// Lower bound of g in vals[lo, lo + len): the index of the first value >= g.
__device__ __forceinline__ int lower_bound_u32(const uint32_t* __restrict__ vals, int lo, int len,
                                               uint32_t g) {
    while (len > 0) {
        const int half = len >> 1;
        if (vals[lo + half] < g) {
            lo += half + 1;
            len -= half + 1;
        } else {
            len = half;
        }
    }
    return lo;
}

// The s3 order of the pass-2 records without a sort: a pass-2 record's rank
// in its s3 cell is the number of pass-2 records before it (record order)
// in the four s2 runs of that cell.  In its own run that is the number of
// passing ranks below its own; in the other three it is the number of
// passing ranks below its lower bound there.  Slot = start3 + rank:
// keys3 / vals3 is the s3 record order, key3g the record's s3 key.
__global__ void __launch_bounds__(256)
k_place3(const int* __restrict__ n_dev, const int* __restrict__ list,
         const BlockDesc* __restrict__ bd, Geometry G, const int* __restrict__ cell2,
         const int* __restrict__ sidx, const uint32_t* __restrict__ vals2,
         const int* __restrict__ st2, const int* __restrict__ en2,
         const unsigned char* __restrict__ old2, const int* __restrict__ st3,
         uint32_t* __restrict__ keys3, uint32_t* __restrict__ vals3,
         uint32_t* __restrict__ key3g) {
    const int j = blockIdx.x * blockDim.x + threadIdx.x;
    if (j >= *n_dev) return;
    const int g = list[j];
    const int b = find_block(bd, G.nb, g);
    const int cell = cell2[g], x = cell % G.W2, y = cell / G.W2;
    const int k2 = b * G.C2 + cell;
    const int x0 = x & ~1, y0 = y & ~1;
    const uint32_t k3 = (uint32_t)(b * G.C3 + (y >> 1) * G.W3 + (x >> 1));
    int rank = 0;
    #pragma unroll
    for (int q = 0; q < 4; ++q) {
        const int s = b * G.C2 + (y0 + (q >> 1)) * G.W2 + x0 + (q & 1);
        const int lo = st2[s];
        const int r = s == k2 ? sidx[g] - lo
                              : lower_bound_u32(vals2, lo, en2[s] - lo, (uint32_t)g) - lo;
        rank += tdrop_passes(old2[s], r, G.window);
    }
    const int slot = st3[k3] + rank;
    if (slot < 0 || slot >= *n_dev) return;     // (ranks are a permutation of [0, n))
    keys3[slot] = k3;
    vals3[slot] = (uint32_t)g;
    key3g[g] = k3;
}

// tdrop_s3 over the s3 record order: pass3, the pass-3 list (placed as in
// k_tdrop2; the counters are committed afterwards by k_keys3b) and, for the
// head, each s3 key's last owned pass-3 record (largest record index) and
// their number.
__global__ void __launch_bounds__(256)
k_tdrop3(const int* __restrict__ n_dev, const uint32_t* __restrict__ keys,
         const uint32_t* __restrict__ vals, uint32_t nk, int C, const int* __restrict__ start,
         const int* __restrict__ off, const BlockDesc* __restrict__ bd, int window,
         const unsigned char* __restrict__ owner, int have_head, unsigned char* __restrict__ pass,
         int* __restrict__ list, int* __restrict__ last, int* __restrict__ count) {
    const int p = blockIdx.x * blockDim.x + threadIdx.x;
    const uint32_t k = p < *n_dev ? keys[p] : nk;
    const bool valid = k < nk;
    int g = -1;
    bool own = false;
    if (valid) {
        g = (int)vals[p];
        const int b = (int)k / C, cell = (int)k % C;
        const int r = p - start[k];
        const unsigned c = bd[b].td3[cell];
        const bool take = tdrop_pass(c, (unsigned)r, window);
        pass[g] = take ? 1 : 0;
        if (take) list[off[k] + tdrop_passes(c, r, window)] = g;
        own = take && have_head && owner[g];
    }
    // last / count per key: the records are sorted by key, so a wave holds a
    // few key segments; one lane per segment adds its count and maximum (a
    // per-record atomic put thousands of updates on each of the few keys)
    unsigned long long m = __ballot(own);
    while (m) {
        const uint32_t kl = (uint32_t)__builtin_amdgcn_readlane((int)k, __builtin_ctzll(m));
        const bool in = own && k == kl;
        const unsigned long long sm = __ballot(in);
        int gm = in ? g : -1;
        #pragma unroll
        for (int o = 32; o > 0; o >>= 1) gm = max(gm, __shfl_xor(gm, o));
        if ((threadIdx.x & 63) == __builtin_ctzll(sm)) {
            atomicMax(last + kl, gm);
            atomicAdd(count + kl, __popcll(sm));
        }
        m &= ~sm;
    }
}

// Per s3 key: commit the counter and the pair count of the key.
__global__ void k_keys3b(uint32_t nk3, Geometry G, const int* __restrict__ t3,
                         const BlockDesc* __restrict__ bd, int* __restrict__ pcnt) {
    const uint32_t t = blockIdx.x * blockDim.x + threadIdx.x;
    if (t >= nk3) return;
    const int b = (int)t / G.C3, cell = (int)t % G.C3, ty = cell / G.W3, tx = cell % G.W3;
    unsigned char* td = bd[b].td3 + cell;
    *td = (unsigned char)(((unsigned)*td + (unsigned)t3[t]) & 255u);
    int np = 0;
    #pragma unroll
    for (int oy = -1; oy <= 1; ++oy)
        #pragma unroll
        for (int ox = -1; ox <= 1; ++ox) {
            const int sy = ty + oy, sx = tx + ox;
            if (sy < 0 || sy >= G.H3 || sx < 0 || sx >= G.W3) continue;
            np += t3[b * G.C3 + sy * G.W3 + sx];
        }
    pcnt[t] = np;
}

// Pair order without a pair sort.  Pair (record g, delta d) updates the
// patch cell t = (y + 1 - d / 3, x + 1 - d % 3) of g's centre cell (x, y),
// delta = (1 - dy) * 3 + (1 - dx), when t is on the grid.  Pairs are ordered
// by t, and inside t by g: a record adds at most one pair to a cell, so this
// is the stable order of (t, g * 9 + d).  With the records sorted stably by
// centre cell (run [st, en) of ascending record ids per key), t's pair count
// is the sum of the run lengths over its 3 x 3 neighbourhood, and a pair's
// rank inside t is the number of records below g in those nine runs.
//
// One thread per sorted record i (record g = vals[i], key k = keys[i]): the
// ranks of g in the 5 x 5 runs around its centre cell (its own run gives
// i - st[k]), folded row by row into three horizontal 3-sums; a delta's rank
// is the sum of three of them.  pos[g * 9 + d] = the pair's place in the pair
// order (-1 when the target is off the grid or the record has no key), and
// pair_need[place] = whether g needs the layer's output (pass[g], or `take`
// when pass is null: the tdrop decision the same thread just made), so the
// scan's apply pass reads one byte per pair in its own order instead of a
// record id and then that record's flag.  The lanes of a wave that share a
// centre cell (records are sorted by cell) rank together: every load then
// serves the whole segment, which keeps the L2 request count low.
constexpr int kSegMax = 4;   // cell segments of a wave ranked together; more: per lane
constexpr int kChunkWide = 512;   // widest window counted in 64-value chunks

// r25[c] for the lanes `in` of one segment (lanes l0..l1 holding records of
// key ks, ids ascending): in each neighbour run c of the 5 x 5 block, every
// such lane's lower bound lies between those of lanes l0 and l1, which 48
// lanes find by binary search at once.  The windows are then read 64 values
// at a time, one coalesced load per window (chunk j of every window together),
// and each lane counts the values below its id by a six-step search across
// the lanes (ds_bpermute), the 24 windows' searches interleaved.  Windows
// wider than kChunkWide are searched per lane inside their bounds, all of
// them advanced together.  Every lane of the wave takes part.
__device__ __forceinline__ void
rank_segment(uint32_t ks, int l0, int l1, bool in, uint32_t g, const uint32_t* __restrict__ vals,
             int C, int W, int H, const int* __restrict__ st, const int* __restrict__ en,
             int* r25) {
    const int lane = threadIdx.x & 63;
    const int b = (int)ks / C, cell = (int)ks % C, y = cell / W, x = cell % W;
    const uint32_t g_first = (uint32_t)__builtin_amdgcn_readlane((int)g, l0);
    const uint32_t g_last = (uint32_t)__builtin_amdgcn_readlane((int)g, l1);
    // lanes c and 32 + c (c < 25): run c's bounds for the first and last id
    int bnd = 0, s0 = 0;
    {
        const int c = lane & 31;
        const int sy = y + c / 5 - 2, sx = x + c % 5 - 2;
        if (c < 25 && c != 12 && sy >= 0 && sy < H && sx >= 0 && sx < W) {
            const int s = b * C + sy * W + sx;
            s0 = st[s];
            bnd = lower_bound_u32(vals, s0, en[s] - s0, lane < 32 ? g_first : g_last);
        }
    }
    // windows up to kChunkWide values: read 64 values at a time, one coalesced
    // load per window (chunk j of every window together); each lane counts
    // the values below its id by a six-step search across the lanes
    // (ds_bpermute), the 24 windows' searches interleaved
    int wmax = 0;
    #pragma unroll
    for (int c = 0; c < 25; ++c) {
        const int wa = __builtin_amdgcn_readlane(bnd, c);
        const int we = __builtin_amdgcn_readlane(bnd, 32 + c);
        if (c != 12 && we - wa <= kChunkWide) wmax = max(wmax, we - wa);
    }
    int lo25[25];
    #pragma unroll
    for (int c = 0; c < 25; ++c) lo25[c] = 0;
    for (int base = 0; base < wmax; base += 64) {
        uint32_t pw[25];
        #pragma unroll
        for (int c = 0; c < 25; ++c) {
            const int wa = __builtin_amdgcn_readlane(bnd, c);
            const int we = __builtin_amdgcn_readlane(bnd, 32 + c);
            pw[c] = (c != 12 && we - wa <= kChunkWide && wa + base + lane < we)
                        ? vals[wa + base + lane] : 0xffffffffu;
        }
        int lc[25];
        #pragma unroll
        for (int c = 0; c < 25; ++c) lc[c] = 0;
        #pragma unroll
        for (int step = 32; step > 0; step >>= 1) {
            #pragma unroll
            for (int c = 0; c < 25; ++c) {
                const uint32_t q = (uint32_t)__builtin_amdgcn_ds_bpermute(
                    (lc[c] + step - 1) << 2, (int)pw[c]);
                if (q < g) lc[c] += step;
            }
        }
        #pragma unroll
        for (int c = 0; c < 25; ++c) {
            const uint32_t q = (uint32_t)__builtin_amdgcn_ds_bpermute(lc[c] << 2, (int)pw[c]);
            lo25[c] += lc[c] + (q < g ? 1 : 0);
        }
    }
    // wider still: per-lane binary searches inside the windows, all of them
    // advanced together
    int wlo[25], wlen[25];
    bool wide = false;
    #pragma unroll
    for (int c = 0; c < 25; ++c) {
        const int wa = __builtin_amdgcn_readlane(bnd, c);
        const int we = __builtin_amdgcn_readlane(bnd, 32 + c);
        wlo[c] = wa;
        wlen[c] = (in && c != 12 && we - wa > kChunkWide) ? we - wa : 0;
        wide |= c != 12 && we - wa > kChunkWide;
    }
    if (wide) {
        for (;;) {
            int active = 0;
            #pragma unroll
            for (int c = 0; c < 25; ++c) {
                if (wlen[c] > 0) {
                    const int half = wlen[c] >> 1;
                    if (vals[wlo[c] + half] < g) {
                        wlo[c] += half + 1;
                        wlen[c] -= half + 1;
                    } else {
                        wlen[c] = half;
                    }
                }
                active |= wlen[c];
            }
            if (!active) break;
        }
    }
    #pragma unroll
    for (int c = 0; c < 25; ++c) {
        const int wa = __builtin_amdgcn_readlane(bnd, c);
        const int we = __builtin_amdgcn_readlane(bnd, 32 + c);
        const int ws = __builtin_amdgcn_readlane(s0, c);
        if (in && c != 12) r25[c] = wa - ws + (we - wa > kChunkWide ? wlo[c] - wa : lo25[c]);
    }
}

// A wave's lanes are consecutive records of the sorted order.  When they
// span at most kSegMax keys (the usual case), each key's segment is ranked
// by rank_segment; otherwise each lane searches the 24 whole runs, all 24
// binary searches advanced together.
__device__ __forceinline__ void
pair_rank_at(int i, int n, const uint32_t* __restrict__ keys,
             const uint32_t* __restrict__ vals, uint32_t nk, int C, int W, int H,
             const int* __restrict__ st, const int* __restrict__ en, const int* __restrict__ pst,
             int* __restrict__ pos, unsigned char* __restrict__ pair_need,
             const unsigned char* __restrict__ pass, bool take) {
    const int lane = threadIdx.x & 63;
    const bool valid = i < n;
    const uint32_t k = valid ? keys[i] : nk;
    const uint32_t g = valid ? vals[i] : 0u;
    const bool keyed = valid && k < nk;
    const uint32_t kprev = (uint32_t)__builtin_amdgcn_ds_bpermute(((lane + 63) & 63) << 2, (int)k);
    const unsigned long long kmask = __ballot(keyed);
    const int nseg = __popcll(__ballot(keyed && (lane == 0 || kprev != k)));
    // r25[c]: the number of records below g in run c of the 5 x 5 block
    // (c = 5 row + column, c = 12 the record's own run)
    int r25[25];
    #pragma unroll
    for (int c = 0; c < 25; ++c) r25[c] = 0;
    if (nseg <= kSegMax) {
        unsigned long long left = kmask;
        while (left) {
            const int l0 = (int)__ffsll((long long)left) - 1;
            const uint32_t ks = (uint32_t)__builtin_amdgcn_readlane((int)k, l0);
            const unsigned long long seg = __ballot(keyed && k == ks);
            const int l1 = 63 - (int)__clzll((long long)seg);
            rank_segment(ks, l0, l1, (seg >> lane) & 1ull, g, vals, C, W, H, st, en, r25);
            left &= ~seg;
        }
    } else if (keyed) {
        const int b = (int)k / C, cell = (int)k % C, y = cell / W, x = cell % W;
        int lo[25], len[25];
        #pragma unroll
        for (int c = 0; c < 25; ++c) {
            const int sy = y + c / 5 - 2, sx = x + c % 5 - 2;
            const bool on = c != 12 && sy >= 0 && sy < H && sx >= 0 && sx < W;
            const int s = on ? b * C + sy * W + sx : 0;
            lo[c] = r25[c] = on ? st[s] : 0;
            len[c] = on ? en[s] - lo[c] : 0;
        }
        for (;;) {
            int active = 0;
            #pragma unroll
            for (int c = 0; c < 25; ++c) {
                if (len[c] > 0) {
                    const int half = len[c] >> 1;
                    if (vals[lo[c] + half] < g) {
                        lo[c] += half + 1;
                        len[c] -= half + 1;
                    } else {
                        len[c] = half;
                    }
                }
                active |= len[c];
            }
            if (!active) break;
        }
        #pragma unroll
        for (int c = 0; c < 25; ++c) r25[c] = lo[c] - r25[c];
    }
    if (!valid) return;
    int* pg = pos + (size_t)g * kPatch;
    if (k >= nk) {
        #pragma unroll
        for (int d = 0; d < kPatch; ++d) pg[d] = -1;
        return;
    }
    const int b = (int)k / C, cell = (int)k % C, y = cell / W, x = cell % W;
    const unsigned char need = pass ? pass[g] : (unsigned char)take;
    r25[12] = i - st[k];
    int hs[5][3];                  // hs[row][dx + 1]: runs (row, dx - 1 .. dx + 1)
    #pragma unroll
    for (int row = 0; row < 5; ++row)
        #pragma unroll
        for (int c = 0; c < 3; ++c)
            hs[row][c] = r25[5 * row + c] + r25[5 * row + c + 1] + r25[5 * row + c + 2];
    #pragma unroll
    for (int d = 0; d < kPatch; ++d) {
        const int dy = 1 - d / 3, dx = 1 - d % 3;      // target offset from the centre
        const int ty = y + dy, tx = x + dx;
        if (ty < 0 || ty >= H || tx < 0 || tx >= W) {
            pg[d] = -1;
            continue;
        }
        const int rank = hs[dy + 1][dx + 1] + hs[dy + 2][dx + 1] + hs[dy + 3][dx + 1];
        const int p = pst[b * C + ty * W + tx] + rank;
        pg[d] = p;
        pair_need[p] = need;
    }
}

__global__ void __launch_bounds__(256)
k_pair_rank(int n_max, const int* __restrict__ n_dev, const uint32_t* __restrict__ keys,
            const uint32_t* __restrict__ vals, uint32_t nk, int C, int W, int H,
            const int* __restrict__ st, const int* __restrict__ en, const int* __restrict__ pst,
            int* __restrict__ pos, unsigned char* __restrict__ pair_need,
            const unsigned char* __restrict__ pass) {
    pair_rank_at(blockIdx.x * blockDim.x + threadIdx.x, n_dev ? *n_dev : n_max, keys, vals, nk,
                 C, W, H, st, en, pst, pos, pair_need, pass, false);
}

// The s2 level's tables that need only the sorted order and the key scan, in
// one launch: per sorted record (blocks [0, nbr)) its tdrop_s2 decision and
// list slot (k_tdrop2) and its pair ranks (k_pair_rank); per key (blocks
// nbr.., one wave each) its chunk table (k_chunks).
__global__ void __launch_bounds__(256)
k_s2_tables(int n, int nbr, const uint32_t* __restrict__ keys, const uint32_t* __restrict__ vals,
            uint32_t nk, int C, int W, int H, const int* __restrict__ st,
            const int* __restrict__ en, const int* __restrict__ pst, const int* __restrict__ pen,
            const int* __restrict__ coff, const unsigned char* __restrict__ old,
            const int* __restrict__ off, int window, unsigned char* __restrict__ pass,
            int* __restrict__ list, int* __restrict__ pos, unsigned char* __restrict__ pair_need,
            int* __restrict__ ckey, int* __restrict__ cbeg, int* __restrict__ cend,
            int* __restrict__ ghist, int* __restrict__ gw) {
    if ((int)blockIdx.x >= nbr) {
        const uint32_t k = (blockIdx.x - (unsigned)nbr) * 4u + (threadIdx.x >> 6);
        if (k >= nk) return;
        const int s0 = pst[k], e = pen[k], c0 = coff[k];
        for (int q = threadIdx.x & 63; s0 + q * kCH < e; q += 64) {
            ckey[c0 + q] = (int)k;
            cbeg[c0 + q] = s0 + q * kCH;
            cend[c0 + q] = min(e, s0 + (q + 1) * kCH);
        }
        // the key's groups of the one-pass scan (k_group_order)
        if ((threadIdx.x & 63) == 0) {
            const int gc = ((e - s0 + kCH - 1) / kCH + kSG - 1) / kSG;
            if (gc > 0) gw[k] = atomicAdd(&ghist[gc], 1);
        }
        return;
    }
    const int i = blockIdx.x * blockDim.x + threadIdx.x;
    const bool take = tdrop2_at(i, n, keys, vals, nk, st, old, off, window, pass, list);
    pair_rank_at(i, n, keys, vals, nk, C, W, H, st, en, pst, pos, pair_need, nullptr, take);
}

// ---------------------------------------------------------------------------
// P: v, g rows as 16 x 16 MFMA tiles (v_mfma_f32_16x16x4_f32, operand layout
// in mfma_pack.h).  A record tile = 64 records (rows, staged in LDS) x all 9
// deltas x the v and g column tiles of qvgIn; each wave owns (delta, column
// tile) items, loads an item's weights (fragment order, one float4 per four
// k-steps) while the previous item's four row tiles run, and writes each
// [v | g] row (2 * OUT floats) to the pair's sorted position.  q is not
// stored: the contraction recomputes it from the record's input.  With the
// weights as the A operand a lane's four results are four consecutive
// channels of one record, stored as one 16-byte piece of its row (staging
// whole rows across waves measured slower: the barriers cost more than the
// partial-line writes).
//
// PT (the layers over all records): a workgroup loops over record tiles
// (tile += gridDim.x) and loads the next tile's rows and pair positions into
// registers while the current tile runs, so the load latency of a tile is
// not paid at the start of a workgroup.  The tiles are 80 records and the
// grid is sized per layer from the CU count (scan_drain) so that each
// workgroup runs about two of them; the launch bounds ask for 5 waves per
// SIMD (L5: 4 waves to 5).  The pass-2 layers keep one 64-record tile per
// workgroup: the prefetch registers cost L7 (IN = 96) a wave per SIMD.
// Their tiles are few (the pass-2 records: ~800 tiles at 200k), so NP
// workgroups share a tile, each running 1/NP of its items (L6: 2, L7: 4):
// with 3-4 tiles per CU, a third of the CUs had one more tile than the rest.
// ---------------------------------------------------------------------------
constexpr int kTM = 64;     // records per projection / contraction workgroup
constexpr int kTMP = 80;    // records per tile of the persistent projection

// Row stride of the LDS tiles read as MFMA A operands, a[(16 m + li) ST + lk
// + 4 s] with li = lane % 16, lk = lane / 16: a stride of 2 (mod 4) puts the
// 32 lanes of each half-wave on 32 distinct banks (a multiple of 4 pairs row
// li with row li + 8).  Rows are then 8-byte aligned: written as float2.
constexpr int lds_stride(int n) { return n + 2; }    // n % 4 == 0

__device__ __forceinline__ void lds_put4(float* p, float4 v) {
    reinterpret_cast<float2*>(p)[0] = make_float2(v.x, v.y);
    reinterpret_cast<float2*>(p)[1] = make_float2(v.z, v.w);
}

// The items of one staged record tile of TM records (TM / 16 row tiles; rows
// past the tile's records are zero in LDS and their pair positions -1), part
// `part` of NP: items [NI part / NP, NI (part + 1) / NP), wave wv taking every
// fourth from the part's item wv.  The item loop is unrolled with a fixed trip
// count and its loads and stores carry no branch: the next item's weights are
// in flight while the current item runs, and the wait before an item covers
// only its own loads.  A result row with no pair (position -1) is written to
// `trash` (one 16-byte slot per lane, never read) instead of being skipped.
template <int IN, int OUT, int TM, int NP>
__device__ __forceinline__ void qvg_items(const float* __restrict__ xs, const int (*prow)[TM],
                                          const float* __restrict__ pp, float* __restrict__ QVG,
                                          float* __restrict__ trash, int part, int tid) {
    using P = ProjPack<IN, OUT>;
    constexpr int XST = lds_stride(IN), NCW = 2 * OUT, MT = TM / kMT, KS = P::KS;
    constexpr int tlo = P::TQ, nti = P::T - tlo, NI = kPatch * nti;
    static_assert(NI % NP == 0 && TM % kMT == 0, "item parts, row tiles");
    constexpr int NPI = NI / NP, KF = NPI / 4, KR = NPI % 4;
    const int lane = tid & 63, wv = tid >> 6, li = lane & 15, lk = lane >> 4;
    const int ib = NPI * part + wv;            // this wave's items: ib + 4 k
    // the weight fragment of an item: KS values per lane, as float4 groups (a
    // final group of two steps as a float2, so no dead register is in flight)
    auto load = [&](int k, float (&b)[KS]) {
        const int it = ib + 4 * k, d = it / nti, t = tlo + (it - d * nti);
        const SSLA_GLOBAL f32x4* src =
            (const SSLA_GLOBAL f32x4*)pp + (size_t)(d * P::T + t) * P::KS4 * 64 + lane;
        #pragma unroll
        for (int g = 0; g < P::KS4; ++g) {
            if (KS - 4 * g >= 4) {
                const f32x4 v = src[g * 64];
                #pragma unroll
                for (int j = 0; j < 4; ++j) b[4 * g + j] = v[j];
            } else {
                const f32x2 v = *(const SSLA_GLOBAL f32x2*)(src + g * 64);
                b[4 * g] = v[0];
                b[4 * g + 1] = v[1];
            }
        }
    };
    // The weight fragment is the A operand and the records the B operand, so
    // the 16 x 16 result is (channel, record): lane (li, lk) holds channels
    // 4 lk .. 4 lk + 3 of record li -- one float4 of that record's row.
    auto run = [&](int k, const float (&b)[KS]) {
        const int it = ib + 4 * k, d = it / nti, t = tlo + (it - d * nti);
        const int c0 = t * kMT - OUT + 4 * lk;
        #pragma unroll
        for (int m = 0; m < MT; ++m) {
            const float* a = &xs[(m * kMT + li) * XST + lk];
            f32x4 acc = {0.f, 0.f, 0.f, 0.f};
            #pragma unroll
            for (int s = 0; s < KS; ++s)
                acc = __builtin_amdgcn_mfma_f32_16x16x4f32(b[s], a[4 * s], acc, 0, 0, 0);
            const int pr = prow[d][m * kMT + li];
            float* dst = pr >= 0 ? QVG + (size_t)pr * NCW + c0 : trash + 4 * lane;
            *(SSLA_GLOBAL f32x4*)dst = acc;
        }
    };
    float bb[2][KS];
    load(0, bb[0]);
    #pragma unroll
    for (int k = 0; k < KF; ++k) {
        if (k + 1 < KF) load(k + 1, bb[(k + 1) & 1]);
        else if (wv < KR) load(KF, bb[KF & 1]);
        __builtin_amdgcn_sched_barrier(0);
        run(k, bb[k & 1]);
        __builtin_amdgcn_sched_barrier(0);
    }
    if (wv < KR) run(KF, bb[KF & 1]);
}

template <int IN, int OUT, bool PT, int TM = kTM, int NP = 1>
__global__ void __launch_bounds__(256, PT ? 5 : 1)
k_qvg(int n_max, const int* __restrict__ n_dev, const int* __restrict__ list,
      const float* __restrict__ X, const int* __restrict__ pos, const float* __restrict__ pp,
      float* __restrict__ QVG, float* __restrict__ trash) {
    constexpr int XST = lds_stride(IN), I4 = IN / 4;
    __shared__ __align__(16) float xs[TM * XST];
    __shared__ int prow[kPatch][TM];
    const int n = n_dev ? *n_dev : n_max;
    const int ntiles = (n + TM - 1) / TM;
    int tile = PT ? (int)blockIdx.x : (int)blockIdx.x / NP;
    if (tile >= ntiles) return;
    const int tid = threadIdx.x;
    if constexpr (!PT) {
        const int base = tile * TM, cnt = min(TM, n - base);
        for (int t = tid; t < TM * I4; t += 256) {
            const int r = t / I4, q = t - r * I4;
            float4 v = make_float4(0.f, 0.f, 0.f, 0.f);
            if (r < cnt) {
                const int g = list ? list[base + r] : base + r;
                v = reinterpret_cast<const float4*>(X)[(size_t)g * I4 + q];
            }
            lds_put4(&xs[r * XST + 4 * q], v);
        }
        for (int t = tid; t < TM * kPatch; t += 256) {
            const int r = t / kPatch, d = t - r * kPatch;
            int pr = -1;
            if (r < cnt) {
                const int g = list ? list[base + r] : base + r;
                pr = pos[(size_t)g * kPatch + d];
            }
            prow[d][r] = pr;
        }
        __syncthreads();
        qvg_items<IN, OUT, TM, NP>(xs, prow, pp, QVG, trash, (int)blockIdx.x % NP, tid);
    } else {
        // this thread's share of a tile: XL float4 of input rows, PL positions
        constexpr int XL = (TM * I4 + 255) / 256, PL = (TM * kPatch + 255) / 256;
        float4 xv[XL];
        int pv[PL];
        auto fetch = [&](int tl) {
            const int base = tl * TM, cnt = min(TM, n - base);
            #pragma unroll
            for (int j = 0; j < XL; ++j) {
                const int t = tid + 256 * j, r = t / I4, q = t - r * I4;
                xv[j] = make_float4(0.f, 0.f, 0.f, 0.f);
                if (t < TM * I4 && r < cnt) {
                    const int g = list ? list[base + r] : base + r;
                    xv[j] = reinterpret_cast<const float4*>(X)[(size_t)g * I4 + q];
                }
            }
            #pragma unroll
            for (int j = 0; j < PL; ++j) {
                const int t = tid + 256 * j, r = t / kPatch, d = t - r * kPatch;
                pv[j] = -1;
                if (t < TM * kPatch && r < cnt) {
                    const int g = list ? list[base + r] : base + r;
                    pv[j] = pos[(size_t)g * kPatch + d];
                }
            }
        };
        fetch(tile);
        while (true) {
            #pragma unroll
            for (int j = 0; j < XL; ++j) {
                const int t = tid + 256 * j, r = t / I4, q = t - r * I4;
                if (t < TM * I4) lds_put4(&xs[r * XST + 4 * q], xv[j]);
            }
            #pragma unroll
            for (int j = 0; j < PL; ++j) {
                const int t = tid + 256 * j, r = t / kPatch, d = t - r * kPatch;
                if (t < TM * kPatch) prow[d][r] = pv[j];
            }
            __syncthreads();
            const int next = tile + (int)gridDim.x;
            if (next < ntiles) fetch(next);
            // the thread index passes through an empty asm each tile, so the
            // compiler does not hoist the items' addresses out of the tile
            // loop (kept live across it, they spilled)
            int tid_t = tid;
            asm volatile("" : "+v"(tid_t));
            qvg_items<IN, OUT, TM, 1>(xs, prow, pp, QVG, trash, 0, tid_t);
            if (next >= ntiles) break;
            __syncthreads();          // every wave is done with the tile
            tile = next;
        }
    }
}

// ---------------------------------------------------------------------------
// S: the per-cell recurrence h = sigmoid(g) h + v over a cell's pairs in ring
// order, in one pass (k_scan): each pair's v, g row is read once.  A cell's
// run is cut into chunks of kCH = 32 pairs and its chunks into groups (kSG = 8
// at s2, kSG3 = 4 at s3: 256 and 128 pairs); one workgroup takes one group,
// one wave per chunk and 64 channels (two waves for the 96 channels of L6 and
// L7):
//   1. each wave loads its chunk's rows into registers (sigmoid(g) in place,
//      nontemporal loads: the projection has just left up to 0.7 GB of rows
//      in the caches) and composes the chunk's map h -> A h + B into LDS;
//   2. the first chunk's waves compose the group's map (SA, SB) in chunk
//      order and find the group's start state: the cell's stored state for
//      its first group, else by looking back over the cell's earlier groups
//      -- the nearest one whose end state is published, then the maps of the
//      groups after it, applied forward.  A group publishes its map before it
//      waits and its end state SA h0 + SB once it has h0, so every state is
//      the same fixed chain of fmaf's whichever word a reader happens to
//      find: the results do not depend on timing.  The cell's last group
//      stores the final state;
//   3. every wave replays its chunk from registers from its start state and
//      writes h where the pair's record needs the layer's output (L4, L5: a
//      compact (pairs, 48) array behind the rows, which their contractions
//      gather 10% faster, stored nontemporal; L6, L7: over v in place).
// Workgroups draw tickets, and ticket t is glist[t] (k_group_order): every
// cell's group 0, then every cell's group 1, ...  A group's predecessors in
// its cell drew earlier tickets (so they have started, and none of them
// waits for a later group), and about one rank of groups earlier, so the
// predecessor has usually published its end state by the time a group
// looks.  Measured at 200k records against the three passes it replaced
// (summary, per-cell carry, apply): L4 0.32 -> 0.26 ms, L5 0.28 -> 0.21,
// L6 0.14 -> 0.14, L7 0.125 -> 0.12; in cell order a cell's groups all ran at
// once and waited on each other down the chain (L4 0.39 ms).  One chunk per
// group at s3 (0.14, 0.13 ms), two or eight at s2 (0.27, 0.31 ms) were slower
// with 64-pair chunks.  Chunks of 32 pairs halve a wave's row registers (123
// VGPRs, no spill, against 168 and 16 B of scratch): L4 0.27 -> 0.26 ms, L5
// 0.21 -> 0.20, L6 0.13 -> 0.11, L7 0.107 -> 0.090 (1.86 -> 1.80 ms per call);
// 16-chunk groups (1024 threads) and 16-pair chunks were slower.
// Published words hold a float and the launch's tag (value | tag << 32)
// and are stored and loaded with relaxed device-scope atomics: a reader that
// sees the tag sees the value, with no fence (a release fence would write
// back the L2).  Every wait is bounded on the wall clock; a wave that runs
// out raises *err (host memory) and goes on with a zero state.
// ---------------------------------------------------------------------------
constexpr int kLB = 4;       // groups looked at per look-back step

__device__ __forceinline__ void sw_put(unsigned long long* p, float v, unsigned tag) {
    __hip_atomic_store(p, ((unsigned long long)tag << 32) | __float_as_uint(v), __ATOMIC_RELAXED,
                       __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ unsigned long long sw_get(const unsigned long long* p) {
    return __hip_atomic_load(p, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ bool sw_ok(unsigned long long x, unsigned tag) {
    return (unsigned)(x >> 32) == tag;
}
__device__ __forceinline__ float sw_val(unsigned long long x) {
    return __uint_as_float((unsigned)x);
}

// Start state of the group of rank r > 0 of a cell (channel cc of a lane;
// `on` marks the lanes that carry a channel).  The cell's group of rank x
// publishes [end | SA | SB] x OUT words at sw + (slot0 + x kSG) 3 OUT; rank
// 0 publishes its end state without waiting.
template <int OUT, int SG>
__device__ float scan_lookback(const unsigned long long* __restrict__ sw, int slot0, int r, int cc,
                               bool on, unsigned tag, unsigned long long deadline,
                               int* __restrict__ err) {
    auto word = [&](int x) { return sw + ((size_t)slot0 + (size_t)x * SG) * 3 * OUT + cc; };
    // phase 1: the nearest group whose end state every lane sees
    int top = r - 1, found = -1;
    float h = 0.f;
    for (;;) {
        unsigned long long x[kLB];
        #pragma unroll
        for (int q = 0; q < kLB; ++q) x[q] = sw_get(word(max(top - q, 0)));
        #pragma unroll
        for (int q = 0; q < kLB; ++q) {
            const bool ok = top - q >= 0 && __all(!on || sw_ok(x[q], tag));
            if (found < 0 && ok) {
                found = top - q;
                h = sw_val(x[q]);
            }
        }
        if (found >= 0) break;
        if (top - kLB >= 0) {
            top -= kLB;                       // none of these: look further back
            continue;
        }
        if ((unsigned long long)wall_clock64() > deadline) {
            if (cc == 0) __hip_atomic_store(err, 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_SYSTEM);
            return 0.f;
        }
        __builtin_amdgcn_s_sleep(2);
        top = r - 1;                          // start again from the nearest group
    }
    // phase 2: the maps of the groups after it, applied forward
    for (int x0 = found + 1; x0 < r; x0 += kLB) {
        unsigned long long a[kLB], b[kLB];
        for (;;) {
            #pragma unroll
            for (int q = 0; q < kLB; ++q) {
                const unsigned long long* p = word(min(x0 + q, r - 1));
                a[q] = sw_get(p + OUT);
                b[q] = sw_get(p + 2 * OUT);
            }
            bool ok = true;
            #pragma unroll
            for (int q = 0; q < kLB; ++q) ok = ok && (x0 + q >= r || (sw_ok(a[q], tag) && sw_ok(b[q], tag)));
            if (__all(!on || ok)) break;
            if ((unsigned long long)wall_clock64() > deadline) {
                if (cc == 0) __hip_atomic_store(err, 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_SYSTEM);
                return 0.f;
            }
            __builtin_amdgcn_s_sleep(2);
        }
        #pragma unroll
        for (int q = 0; q < kLB; ++q)
            if (x0 + q < r) h = fmaf(sw_val(a[q]), h, sw_val(b[q]));
    }
    return h;
}

// The one-pass scan's ticket order (one workgroup): a cell's run of nc
// chunks forms gc = ceil(nc / kSG) groups; tickets take every cell's group
// 0, then every cell's group 1, ..., cells with more groups first.
// ghist[v] counts the cells with gc = v and gw[k] is cell k's place among
// them (k_s2_tables).  start[v] = cells with more than v groups (the groups
// of rank v), base[r] = tickets before rank r; cell k, at place start[gc] +
// gw[k] of every rank below gc, gets glist[base[r] + start[gc] + gw[k]] =
// (k, r).  Writes the group count to *n_groups.
constexpr int kGroupLds = 6144;    // start / base entries k_group_order keeps in LDS

__global__ void __launch_bounds__(kScanThreads)
k_group_order(int nk, int nv, int sg, const int* __restrict__ pst, const int* __restrict__ pen,
              const int* __restrict__ ghist, const int* __restrict__ gw, int* __restrict__ gstart,
              int* __restrict__ gbase, int2* __restrict__ glist, int* __restrict__ n_groups) {
    __shared__ int lds[2 * (kScanThreads / 64)];
    __shared__ int sst[kGroupLds], sba[kGroupLds];
    const bool inl = nv <= kGroupLds;      // else the tables are read from global memory
    int carry = 0;
    for (int r0 = 0; r0 < nv; r0 += kScanRound) {        // start: scan of ghist from the top
        const int i0 = r0 + (int)threadIdx.x * kScanPer;
        int v[kScanPer], sum = 0;
        #pragma unroll
        for (int q = 0; q < kScanPer; ++q) {
            v[q] = i0 + q < nv ? ghist[nv - 1 - (i0 + q)] : 0;
            sum += v[q];
        }
        int total;
        int run = carry + block_exscan(sum, lds, &total);
        carry += total;
        #pragma unroll
        for (int q = 0; q < kScanPer; ++q) {
            const int i = nv - 1 - (i0 + q);
            if (i0 + q < nv) {
                gstart[i] = run;
                if (inl) sst[i] = run;
            }
            run += v[q];
        }
    }
    __syncthreads();
    carry = 0;
    for (int r0 = 0; r0 < nv; r0 += kScanRound) {        // base: prefix of start
        const int i0 = r0 + (int)threadIdx.x * kScanPer;
        int v[kScanPer], sum = 0;
        #pragma unroll
        for (int q = 0; q < kScanPer; ++q) {
            v[q] = i0 + q < nv ? (inl ? sst[i0 + q] : gstart[i0 + q]) : 0;
            sum += v[q];
        }
        int total;
        int run = carry + block_exscan(sum, lds, &total);
        carry += total;
        #pragma unroll
        for (int q = 0; q < kScanPer; ++q) {
            if (i0 + q < nv) {
                gbase[i0 + q] = run;
                if (inl) sba[i0 + q] = run;
            }
            run += v[q];
        }
    }
    if (threadIdx.x == 0) *n_groups = carry;
    __syncthreads();
    const int* st = inl ? sst : gstart;
    const int* ba = inl ? sba : gbase;
    for (int k = threadIdx.x; k < nk; k += kScanThreads) {
        const int nc = (pen[k] - pst[k] + kCH - 1) / kCH, gc = (nc + sg - 1) / sg;
        if (gc == 0) continue;
        const int p = st[gc] + gw[k];
        for (int r = 0; r < gc; ++r) glist[ba[r] + p] = make_int2(k, r);
    }
}

template <int OUT, int HS, int SG>
__global__ void __launch_bounds__(SG * ((OUT + 63) / 64) * 64)
__attribute__((amdgpu_waves_per_eu(3, 8)))
k_scan(const int* __restrict__ n_groups, int* __restrict__ ticket, unsigned tag,
       const int2* __restrict__ glist, const int* __restrict__ cbeg, const int* __restrict__ cend,
       const int* __restrict__ coff, const int* __restrict__ pst, const int* __restrict__ pen, int C,
       const BlockDesc* __restrict__ bd, int li, const unsigned char* __restrict__ pair_need,
       const float* __restrict__ QVG, float* __restrict__ Hout, unsigned long long* __restrict__ sw,
       int* __restrict__ err, unsigned long long wait_ticks) {
    constexpr int WPC = (OUT + 63) / 64;          // waves per chunk (64 channels each)
    constexpr int NC = 2 * OUT;
    __shared__ int stk;
    __shared__ float sA[SG][OUT], sB[SG][OUT], sH[SG][OUT];
    const int t = threadIdx.x, w = t >> 6, lane = t & 63;
    const int m = w / WPC;                        // the wave's chunk in the group
    const int c = (w % WPC) * 64 + lane;          // the lane's channel
    const bool on = c < OUT;
    const int cc = on ? c : 0;
    if (t == 0) stk = atomicAdd(ticket, 1);
    __syncthreads();
    const int gi = stk;
    if (gi >= *n_groups) return;                  // uniform over the workgroup
    const int2 kr = glist[gi];
    const int k = kr.x, r = kr.y;
    const int nc = (pen[k] - pst[k] + kCH - 1) / kCH;
    const int slot0 = coff[k];                    // the cell's first chunk
    const int c0 = slot0 + r * SG;               // the group's first chunk
    const int ng = min(SG, nc - r * SG);
    const bool have = m < ng;
    int s = 0, n = 0;
    float sg[kCH], vv[kCH];
    if (have) {
        s = cbeg[c0 + m];
        n = cend[c0 + m] - s;
        // all kCH rows, eight from one base address (their offsets fit the
        // load's immediate field; a clamped index per row cost a 64-bit
        // address register per load).  Rows past the chunk's end stay inside
        // the row buffer (kCH rows of padding past the largest row count) and
        // are not used.
        const float* row = QVG + (size_t)s * NC + cc;
        #pragma unroll
        for (int q8 = 0; q8 < kCH; q8 += 8) {
            const float* rb = row + (size_t)q8 * NC;
            #pragma unroll
            for (int q = 0; q < 8; ++q) {
                vv[q8 + q] = __builtin_nontemporal_load(rb + q * NC);
                sg[q8 + q] = __builtin_nontemporal_load(rb + q * NC + OUT);
            }
        }
        float A = 1.f, B = 0.f;
        #pragma unroll
        for (int q = 0; q < kCH; ++q) {
            sg[q] = sigmoid_fast(sg[q]);
            if (q < n) {
                A *= sg[q];
                B = fmaf(sg[q], B, vv[q]);
            }
        }
        if (on) {
            sA[m][c] = A;
            sB[m][c] = B;
        }
    }
    __syncthreads();
    if (w < WPC) {                                // the first chunk's waves chain the group
        const bool last = (r + 1) * SG >= nc;    // the cell's last group
        float* hp0 = bd[k / C].hidden[li] + (size_t)(k % C) * OUT + cc;
        unsigned long long* P = sw + (size_t)c0 * 3 * OUT + cc;
        float SA = 1.f, SB = 0.f;
        for (int q = 0; q < ng; ++q) {
            SB = fmaf(sA[q][cc], SB, sB[q][cc]);
            SA *= sA[q][cc];
        }
        float h0;
        if (r == 0) {
            h0 = on ? *hp0 : 0.f;
        } else {
            if (!last && on) {
                sw_put(P + OUT, SA, tag);
                sw_put(P + 2 * OUT, SB, tag);
            }
            h0 = scan_lookback<OUT, SG>(sw, slot0, r, cc, on, tag,
                                    (unsigned long long)wall_clock64() + wait_ticks, err);
        }
        if (on) {
            const float hend = fmaf(SA, h0, SB);
            if (last) *hp0 = hend;
            else sw_put(P, hend, tag);
        }
        float h = h0;
        for (int q = 0; q < ng; ++q) {
            if (on) sH[q][c] = h;
            h = fmaf(sA[q][cc], h, sB[q][cc]);
        }
    }
    __syncthreads();
    if (!have) return;
    // replay from the chunk's start state; lane l reads pair s + l's need flag
    const unsigned long long use =
        __ballot(lane < n && (!pair_need || pair_need[s + lane]));
    float h = on ? sH[m][c] : 0.f;
    float* hp = Hout + (size_t)s * HS + cc;
    #pragma unroll
    for (int q = 0; q < kCH; ++q) {
        if (q < n) {
            h = fmaf(sg[q], h, vv[q]);
            if (on && ((use >> q) & 1ull)) {
                // the compact h rows (L4, L5) go out nontemporal: the
                // contraction that gathers them next runs faster (L4 179 ->
                // 160 us for +9 us here); L6's in-place rows lose by it
                if constexpr (HS == OUT) __builtin_nontemporal_store(h, hp + (size_t)q * HS);
                else gstore(hp + (size_t)q * HS, h);
            }
        }
    }
}

// ---------------------------------------------------------------------------
// O: per record y = sum_delta goW[delta]^T (q_delta * h_delta) + residual,
// fp64 LayerNorm -- computed transposed, with the weights as MFMA A operands
// and the records as columns (layouts in mfma_pack.h, OutPackT):
//   q^T tile (16 channels x 16 records) = Wq[delta]^T X^T
//   Y^T     += goW[delta]^T (q^T * h^T)        for every output tile
//   Y^T     += input_proj^T X^T (IN != OUT) or + X (IN == OUT)
// Each wave owns RT tiles of 16 records and runs every K part itself, so no
// LDS and no barrier are involved: a lane keeps its record's input row
// (the B operand of q and input_proj, one float4 per four steps) in
// registers for the whole kernel; the h values arrive as one float4 per
// lane in the MFMA output layout of the q tile and are multiplied there;
// and with the K order of OutPackT those four products are the lane's B
// values of the goW steps.  The weights stream from the L2 (shared by all
// waves) one (delta, channel tile) item ahead.  LayerNorm in fp64 over the
// four lanes that hold a record's outputs (ds_swizzle and ds_bpermute sums).
// HR rows are HS floats apart (the scan's h output rows).
// WPS asks the compiler for at least that many waves per SIMD; with the
// unrolled item loop L4 (RT = 2) compiles to 120 registers, 4 waves per SIMD.
// ---------------------------------------------------------------------------
__device__ __forceinline__ double xor_lanes_d(double v, int pattern_or_lane, bool swizzle) {
    const unsigned long long b = __builtin_bit_cast(unsigned long long, v);
    unsigned lo, hi;
    if (swizzle) {
        lo = (unsigned)__builtin_amdgcn_ds_swizzle((int)(unsigned)b, 0x401F);       // xor 16
        hi = (unsigned)__builtin_amdgcn_ds_swizzle((int)(unsigned)(b >> 32), 0x401F);
    } else {
        lo = (unsigned)__builtin_amdgcn_ds_bpermute(pattern_or_lane, (int)(unsigned)b);
        hi = (unsigned)__builtin_amdgcn_ds_bpermute(pattern_or_lane, (int)(unsigned)(b >> 32));
    }
    return __builtin_bit_cast(double, ((unsigned long long)hi << 32) | lo);
}

// sum over lanes j, j + 16, j + 32, j + 48 (all 64 lanes active)
__device__ __forceinline__ double sum4_lanes(double v, int lane) {
    v += xor_lanes_d(v, 0, true);
    return v + xor_lanes_d(v, (lane ^ 32) << 2, false);
}

// L5-L7 contraction launch shape: 16-record tiles (RT = 1), the nine deltas
// split over three waves (KS = 3).  Measured at 200k records: nine waves per
// tile (one delta each) took L5.out 61 -> 91 us and L6.out 146 -> 214 us
// (L7 spills at the 168-register cap of nine waves); two record tiles per
// wave left L5.out unchanged and took L6.out to 161 us (L7: 202 registers,
// one wave per SIMD).
constexpr int kOutKS5 = 3, kOutKS6 = 3, kOutKS7 = 3;
constexpr int kOutRT5 = 1, kOutRT6 = 1, kOutRT7 = 1;

template <int IN, int OUT, int RT, int KS, int WPS = 1, int HS = 2 * OUT>
__global__ void __launch_bounds__(64 * KS, WPS)
k_outt(int n_max, const int* __restrict__ n_dev, const int* __restrict__ list,
       const float* __restrict__ X, const int* __restrict__ pos, const float* __restrict__ HR,
       const float* __restrict__ po, const float* __restrict__ gamma,
       const float* __restrict__ beta, float* __restrict__ Y) {
    using O = OutPackT<IN, OUT>;
    constexpr int NT = O::NT, KG = O::KG, R = 16 * RT;
    // the workgroup's pair rows, and the partial sums of waves 1..KS-1
    __shared__ int sp[R][kPatch];
    __shared__ f32x4 part[KS > 1 ? KS - 1 : 1][RT * NT][64];
    const int n = n_dev ? *n_dev : n_max;
    const int base = blockIdx.x * R;
    if (base >= n) return;
    const int wv = threadIdx.x >> 6, lane = threadIdx.x & 63, g = lane >> 4, j = lane & 15;
    for (int t = threadIdx.x; t < R * kPatch; t += 64 * KS) {
        const int r = t / kPatch, d = t - r * kPatch;
        const int q = base + r;
        const int rr = q < n ? (list ? list[q] : q) : -1;
        sp[r][d] = rr >= 0 ? pos[(size_t)rr * kPatch + d] : -1;
    }
    int rec[RT];
    #pragma unroll
    for (int rt = 0; rt < RT; ++rt) {
        const int r = base + 16 * rt + j;
        rec[rt] = r < n ? (list ? list[r] : r) : -1;
    }
    // this lane's B values of the input steps: X[rec][16 t + 4 g .. + 3]
    // (a half group: X[rec][16 t + 2 g .. + 1])
    f32x4 xr[RT][KG];
    #pragma unroll
    for (int rt = 0; rt < RT; ++rt)
        #pragma unroll
        for (int t = 0; t < KG; ++t) {
            const float* xp = X + (size_t)(rec[rt] < 0 ? 0 : rec[rt]) * IN + O::kidx(t, g, 0);
            f32x4 v = {0.f, 0.f, 0.f, 0.f};
            if (rec[rt] >= 0) {
                if (O::steps(t) == 4) {
                    v = *(const SSLA_GLOBAL f32x4*)xp;
                } else {
                    v[0] = gload(xp);
                    v[1] = gload(xp + 1);
                }
            }
            xr[rt][t] = v;
        }
    f32x4 acc[RT][NT];
    #pragma unroll
    for (int rt = 0; rt < RT; ++rt)
        #pragma unroll
        for (int ot = 0; ot < NT; ++ot) acc[rt][ot] = f32x4{0.f, 0.f, 0.f, 0.f};
    __syncthreads();

    const SSLA_GLOBAL f32x4* wq = (const SSLA_GLOBAL f32x4*)po + lane;
    const SSLA_GLOBAL f32x4* wg = (const SSLA_GLOBAL f32x4*)(po + O::Q) + lane;
    // item it = delta * NT + ct: its q and goW fragments and the h values (an
    // absent pair, p < 0, reads row 0 and is zeroed where it is used, so the
    // loads carry no branch and the next item's stay in flight)
    auto load = [&](int it, f32x4 (&aq)[KG], f32x4 (&ag)[NT], f32x4 (&hv)[RT], int (&pv)[RT]) {
        const int d = it / NT, ct = it - d * NT;
        #pragma unroll
        for (int t = 0; t < KG; ++t) {
            const SSLA_GLOBAL f32x4* src = wq + ((size_t)it * KG + t) * 64;
            if (O::steps(t) == 4) {
                aq[t] = *src;
            } else {
                // a half group: the two live values only (a 16-byte load
                // would keep two dead registers in flight)
                const f32x2 v = *(const SSLA_GLOBAL f32x2*)src;
                aq[t] = f32x4{v[0], v[1], 0.f, 0.f};
            }
        }
        #pragma unroll
        for (int ot = 0; ot < NT; ++ot) ag[ot] = wg[((size_t)it * NT + ot) * 64];
        #pragma unroll
        for (int rt = 0; rt < RT; ++rt) {
            const int p = sp[16 * rt + j][d];
            pv[rt] = p;
            hv[rt] = *(const SSLA_GLOBAL f32x4*)(HR + (size_t)(p < 0 ? 0 : p) * HS + 16 * ct + 4 * g);
        }
    };
    auto compute = [&](const f32x4 (&aq)[KG], const f32x4 (&ag)[NT], const f32x4 (&hv)[RT],
                       const int (&pv)[RT]) {
        f32x4 q[RT];
        #pragma unroll
        for (int rt = 0; rt < RT; ++rt) q[rt] = f32x4{0.f, 0.f, 0.f, 0.f};
        #pragma unroll
        for (int t = 0; t < KG; ++t)
            #pragma unroll
            for (int i = 0; i < O::steps(t); ++i)
                #pragma unroll
                for (int rt = 0; rt < RT; ++rt)
                    q[rt] = __builtin_amdgcn_mfma_f32_16x16x4f32(aq[t][i], xr[rt][t][i], q[rt],
                                                                 0, 0, 0);
        #pragma unroll
        for (int rt = 0; rt < RT; ++rt)
            q[rt] = pv[rt] >= 0 ? q[rt] * hv[rt] : f32x4{0.f, 0.f, 0.f, 0.f};
        #pragma unroll
        for (int i = 0; i < 4; ++i)
            #pragma unroll
            for (int rt = 0; rt < RT; ++rt)
                #pragma unroll
                for (int ot = 0; ot < NT; ++ot)
                    acc[rt][ot] = __builtin_amdgcn_mfma_f32_16x16x4f32(ag[ot][i], q[rt][i],
                                                                       acc[rt][ot], 0, 0, 0);
    };
    // this wave's items: deltas [wv * 9 / KS, (wv + 1) * 9 / KS), the K parts
    // split over the KS waves.  The loop is unrolled (a fixed trip count, no
    // branches), and the scheduling barriers keep item k + 1's loads ahead of
    // item k's MFMAs: the wait before item k then covers only its own loads,
    // issued one item earlier.
    static_assert(kPatch % KS == 0, "K parts of whole deltas");
    constexpr int NI = kPatch / KS * NT;
    const int i0 = wv * NI;
    f32x4 aqb[2][KG], agb[2][NT], hvb[2][RT];
    int pvb[2][RT];
    load(i0, aqb[0], agb[0], hvb[0], pvb[0]);
    #pragma unroll
    for (int k = 0; k < NI; ++k) {
        if (k + 1 < NI)
            load(i0 + k + 1, aqb[(k + 1) & 1], agb[(k + 1) & 1], hvb[(k + 1) & 1], pvb[(k + 1) & 1]);
        __builtin_amdgcn_sched_barrier(0);
        compute(aqb[k & 1], agb[k & 1], hvb[k & 1], pvb[k & 1]);
        if constexpr (KS == 1) __builtin_amdgcn_sched_barrier(0);
    }
    if constexpr (KS > 1) {
        if (wv > 0) {
            #pragma unroll
            for (int rt = 0; rt < RT; ++rt)
                #pragma unroll
                for (int ot = 0; ot < NT; ++ot) part[wv - 1][rt * NT + ot][lane] = acc[rt][ot];
        }
        __syncthreads();
        if (wv > 0) return;
        #pragma unroll
        for (int w = 0; w < KS - 1; ++w)
            #pragma unroll
            for (int rt = 0; rt < RT; ++rt)
                #pragma unroll
                for (int ot = 0; ot < NT; ++ot) acc[rt][ot] += part[w][rt * NT + ot][lane];
    }
    if constexpr (O::IP) {
        const SSLA_GLOBAL f32x4* wi = (const SSLA_GLOBAL f32x4*)(po + O::Q + O::GO) + lane;
        #pragma unroll
        for (int ot = 0; ot < NT; ++ot) {
            f32x4 ai[KG];
            #pragma unroll
            for (int t = 0; t < KG; ++t) ai[t] = wi[((size_t)ot * KG + t) * 64];
            #pragma unroll
            for (int t = 0; t < KG; ++t)
                #pragma unroll
                for (int i = 0; i < O::steps(t); ++i)
                    #pragma unroll
                    for (int rt = 0; rt < RT; ++rt)
                        acc[rt][ot] = __builtin_amdgcn_mfma_f32_16x16x4f32(ai[t][i], xr[rt][t][i],
                                                                           acc[rt][ot], 0, 0, 0);
        }
    } else {
        // residual: the lane holds X[rec][16 ot + 4 g + i] as xr[rt][ot][i]
        #pragma unroll
        for (int rt = 0; rt < RT; ++rt)
            #pragma unroll
            for (int ot = 0; ot < NT; ++ot) acc[rt][ot] += xr[rt][ot];
    }
    // fp64 LayerNorm (eps 1e-5): lane (g, j) holds outputs 16 ot + 4 g + i of
    // record j of each tile; the record's sums are over lanes j + 16 g
    #pragma unroll
    for (int rt = 0; rt < RT; ++rt) {
        double s = 0.0;
        #pragma unroll
        for (int ot = 0; ot < NT; ++ot)
            #pragma unroll
            for (int i = 0; i < 4; ++i) s += (double)acc[rt][ot][i];
        const double mean = sum4_lanes(s, lane) / (double)OUT;
        double v = 0.0;
        #pragma unroll
        for (int ot = 0; ot < NT; ++ot)
            #pragma unroll
            for (int i = 0; i < 4; ++i) {
                const double dd = (double)acc[rt][ot][i] - mean;
                v += dd * dd;
            }
        const double inv = 1.0 / sqrt(sum4_lanes(v, lane) / (double)OUT + 1e-5);
        #pragma unroll
        for (int ot = 0; ot < NT && rec[rt] >= 0; ++ot) {
            const int c = 16 * ot + 4 * g;
            const f32x4 ga = *(const SSLA_GLOBAL f32x4*)(gamma + c);
            const f32x4 be = *(const SSLA_GLOBAL f32x4*)(beta + c);
            f32x4 o;
            #pragma unroll
            for (int i = 0; i < 4; ++i)
                o[i] = (float)(((double)acc[rt][ot][i] - mean) * inv * (double)ga[i] +
                               (double)be[i]);
            *(SSLA_GLOBAL f32x4*)(Y + (size_t)rec[rt] * OUT + c) = o;
        }
    }
}

// The sum over each quad of lanes, in every lane of it: DPP quad_perm moves
// (xor 1, then xor 2) instead of LDS-permute shuffles.
__device__ __forceinline__ float quad_sum(float v) {
    v += __builtin_bit_cast(
        float, __builtin_amdgcn_mov_dpp(__builtin_bit_cast(int, v), 0xB1, 0xF, 0xF, false));
    v += __builtin_bit_cast(
        float, __builtin_amdgcn_mov_dpp(__builtin_bit_cast(int, v), 0x4E, 0xF, 0xF, false));
    return v;
}

// ---------------------------------------------------------------------------
// head: raw [reg0..3, obj, cls0, cls1] for pass-3 records
// (...celled.cuh:841-902).  One workgroup = 64 records (list order): their
// 96-channel features staged in LDS; the two 1x1 convolutions (cls, reg; BN
// folded) as one 64 x 192 x 96 product of 16 x 16 MFMA tiles whose B
// operands are read straight from the row-major (IN, OUT) weights (lane l
// takes row 4s + l/16, column l%16 of step s); SiLU into LDS; then the
// seven prediction dot products, four threads per record.
// ---------------------------------------------------------------------------
__global__ void __launch_bounds__(256)
k_head(const int* __restrict__ n_dev, const int* __restrict__ list,
       const float* __restrict__ X, HeadPtrs hp, float* __restrict__ H7) {
    constexpr int C = SSLA_C3, XST = lds_stride(C), HST = 2 * C + 4, CT = 2 * C / kMT;
    __shared__ __align__(16) float xs[kTM * XST];
    __shared__ float hs[kTM * HST];           // [yc | yr] per record
    __shared__ int rows[kTM];
    const int n = *n_dev;
    const int base = blockIdx.x * kTM;
    if (base >= n) return;
    const int cnt = min(kTM, n - base);
    const int tid = threadIdx.x;
    if (tid < kTM) rows[tid] = tid < cnt ? list[base + tid] : -1;
    __syncthreads();
    constexpr int C4 = C / 4;
    for (int t = tid; t < kTM * C4; t += 256) {
        const int r = t / C4, q = t - r * C4;
        float4 v = make_float4(0.f, 0.f, 0.f, 0.f);
        if (rows[r] >= 0) v = reinterpret_cast<const float4*>(X)[(size_t)rows[r] * C4 + q];
        lds_put4(&xs[r * XST + 4 * q], v);
    }
    __syncthreads();
    const int lane = tid & 63, wv = tid >> 6, li = lane & 15, lk = lane >> 4;
    const int mtiles = (cnt + kMT - 1) / kMT;
    // column tiles 0..5: cls conv, 6..11: reg conv; wave wv takes tiles wv, wv+4, wv+8
    for (int ct = wv; ct < CT; ct += 4) {
        const bool reg = ct >= CT / 2;
        const float* W = reg ? hp.reg_conv_W : hp.cls_conv_W;
        const float* bias = reg ? hp.reg_conv_b : hp.cls_conv_b;
        const int col = (reg ? ct - CT / 2 : ct) * kMT + li;
        float b[C / 4];
        #pragma unroll
        for (int s = 0; s < C / 4; ++s) b[s] = gload(W + (size_t)(4 * s + lk) * C + col);
        const float bc = bias[col];
        for (int m = 0; m < mtiles; ++m) {
            const float* a = &xs[(m * kMT + li) * XST + lk];
            f32x4 acc = {0.f, 0.f, 0.f, 0.f};
            #pragma unroll
            for (int s = 0; s < C / 4; ++s)
                acc = __builtin_amdgcn_mfma_f32_16x16x4f32(a[4 * s], b[s], acc, 0, 0, 0);
            #pragma unroll
            for (int r = 0; r < 4; ++r) {
                const float y = acc[r] + bc;
                hs[(m * kMT + 4 * lk + r) * HST + ct * kMT + li] = y * sigmoid_fast(y);
            }
        }
    }
    __syncthreads();
    // predictions: record r = tid / 4, channels part, part + 4, ... (24 each)
    const int r = tid >> 2, part = tid & 3;
    float o[7];
    #pragma unroll
    for (int k = 0; k < 7; ++k) o[k] = 0.f;
    if (r < cnt) {
        const float* yc = &hs[r * HST];
        const float* yr = yc + C;
        for (int i = part; i < C; i += 4) {
            #pragma unroll
            for (int k = 0; k < 4; ++k) o[k] = fmaf(hp.reg_pred_W[(size_t)i * 4 + k], yr[i], o[k]);
            o[4] = fmaf(hp.obj_pred_W[i], yr[i], o[4]);
            #pragma unroll
            for (int k = 0; k < 2; ++k) o[5 + k] = fmaf(hp.cls_pred_W[(size_t)i * 2 + k], yc[i], o[5 + k]);
        }
    }
    #pragma unroll
    for (int k = 0; k < 7; ++k) o[k] = quad_sum(o[k]);
    if (r < cnt && part == 0) {
        float* out = H7 + (size_t)rows[r] * 7;
        #pragma unroll
        for (int k = 0; k < 4; ++k) out[k] = o[k] + hp.reg_pred_b[k];
        out[4] = o[4] + hp.obj_pred_b[0];
        out[5] = o[5] + hp.cls_pred_b[0];
        out[6] = o[6] + hp.cls_pred_b[1];
    }
}

// Single-linear head (...celled.cuh:1476-1481, matvec_w<C3, 7> over
// head_W (C3, 7) row-major, plus head_b) for pass-3 records: 64 records per
// workgroup in list order, four threads per record (channels part, part + 4,
// ...), the quad's partial sums added with two DPP moves.
__global__ void __launch_bounds__(256)
k_head_linear(const int* __restrict__ n_dev, const int* __restrict__ list,
              const float* __restrict__ X, HeadPtrs hp, float* __restrict__ H7) {
    constexpr int C = SSLA_C3;
    const int n = *n_dev;
    const int base = blockIdx.x * kTM;
    if (base >= n) return;
    const int j = base + (threadIdx.x >> 2), part = threadIdx.x & 3;
    const bool on = j < n;
    const int g = on ? list[j] : 0;
    float o[7];
    #pragma unroll
    for (int k = 0; k < 7; ++k) o[k] = 0.f;
    if (on) {
        const float* x = X + (size_t)g * C;
        for (int i = part; i < C; i += 4) {
            const float xi = x[i];
            #pragma unroll
            for (int k = 0; k < 7; ++k) o[k] = fmaf(hp.lin_W[(size_t)i * 7 + k], xi, o[k]);
        }
    }
    #pragma unroll
    for (int k = 0; k < 7; ++k) o[k] = quad_sum(o[k]);
    if (on && part == 0) {
        float* out = H7 + (size_t)g * 7;
        #pragma unroll
        for (int k = 0; k < 7; ++k) out[k] = o[k] + hp.lin_b[k];
    }
}

__global__ void k_pred_write(const int* __restrict__ n_dev, const int* __restrict__ list,
                             const unsigned char* __restrict__ owner,
                             const uint32_t* __restrict__ key3_by_g,
                             const int* __restrict__ last, const int* __restrict__ count,
                             const BlockDesc* __restrict__ bd, Geometry G,
                             const float* __restrict__ H7) {
    const int j = blockIdx.x * blockDim.x + threadIdx.x;
    if (j >= *n_dev) return;
    const int g = list[j];
    if (!owner[g]) return;
    const uint32_t k = key3_by_g[g];
    if (last[k] != g) return;
    const int b = (int)k / G.C3, cell = (int)k % G.C3;
    const HybridStrip& s = bd[b].strip;
    const int sx = cell % G.W3, sy = cell / G.W3;
    const int hx = sx - s.s3_owned_lo, hy = sy - s.s3_owned_y_lo;
    const int w = s.s3_owned_hi - s.s3_owned_lo, h = s.s3_owned_y_hi - s.s3_owned_y_lo;
    if (hx < 0 || hx >= w || hy < 0 || hy >= h) return;
    const int idx = hy * w + hx;
    float v7[7];
    #pragma unroll
    for (int q = 0; q < 7; ++q) v7[q] = H7[(size_t)g * 7 + q];
    publish_pred(bd[b].preds ? bd[b].preds + (size_t)idx * 7 : nullptr,
                 bd[b].version ? bd[b].version + idx : nullptr, v7, (unsigned)count[k]);
}

// Output slots (...celled.cuh:1233-1247 conventions) and raw head rows.
// Output slots (392 B = 49 eight-byte words) and head rows as coalesced
// 8-byte stores: 32 records per 256-thread workgroup.
constexpr int kEmitRec = 128;

__global__ void __launch_bounds__(256)
k_emit(int E, const BlockDesc* __restrict__ bd, int nb,
       const int* __restrict__ cell2,
       const unsigned char* __restrict__ owner,
       const unsigned char* __restrict__ pass2,
       const unsigned char* __restrict__ pass3,
       const float* __restrict__ X4, const float* __restrict__ H7,
       int have_head) {
    constexpr int NW = (int)(sizeof(HybridS2S3OutputSlot) / 8);
    static_assert(sizeof(HybridS2S3OutputSlot) % 8 == 0 && SSLA_C3 % 2 == 0, "slot words");
    __shared__ int sb[kEmitRec], sk[kEmitRec], sp2[kEmitRec], sp3[kEmitRec];
    __shared__ unsigned char sfeat[kEmitRec], shead[kEmitRec];
    const int g0 = blockIdx.x * kEmitRec;
    const int t = threadIdx.x;
    if (t < kEmitRec) {
        const int g = g0 + t;
        int b = 0, k = -1, q2 = -2, q3 = -2;
        bool feat = false, head = false;
        if (g < E) {
            b = find_block(bd, nb, g);
            k = g - bd[b].offset;
            const bool valid = cell2[g] >= 0;
            const bool p2 = valid && pass2[g], p3 = p2 && pass3[g], own = owner[g];
            if (valid) {
                q2 = own ? (p2 ? 1 : 0) : -1;
                q3 = own ? (p3 ? 1 : 0) : -1;
            }
            feat = p3;
            head = have_head && p3 && own;
        }
        sb[t] = b; sk[t] = k; sp2[t] = q2; sp3[t] = q3;
        sfeat[t] = feat; shead[t] = head;
    }
    __syncthreads();
    for (int j = t; j < kEmitRec * NW; j += 256) {
        const int r = j / NW, w = j - r * NW;
        const int k = sk[r];
        HybridS2S3OutputSlot* out = k >= 0 ? bd[sb[r]].out : nullptr;
        if (!out) continue;
        if (w == 0) {
            reinterpret_cast<int2*>(out + k)[0] = make_int2(sp2[r], sp3[r]);
        } else {
            const int i = 2 * (w - 1);
            float2 f = make_float2(0.f, 0.f);
            if (sfeat[r]) f = *reinterpret_cast<const float2*>(X4 + (size_t)(g0 + r) * SSLA_C3 + i);
            reinterpret_cast<float2*>(out[k].s3_feat)[w - 1] = f;
        }
    }
    for (int j = t; j < kEmitRec * 7; j += 256) {
        const int r = j / 7, c = j - r * 7;
        const int k = sk[r];
        float* ho = k >= 0 ? bd[sb[r]].head_out : nullptr;
        if (ho) ho[(size_t)k * 7 + c] = shead[r] ? H7[(size_t)(g0 + r) * 7 + c] : 0.f;
    }
}

// ---------------------------------------------------------------------------
// workspace
// ---------------------------------------------------------------------------
struct Workspace {
    int cap = 0;            // records
    int cap_blocks = 0;
    int cap_keys = 0;
    void* base = nullptr;
    size_t bytes = 0;
    float *X0, *X1, *X2, *X3, *X4, *QVG, *H7;
    int *cell2, *pos2, *pos3, *list2, *list3, *counts;
    int *st2, *en2, *st3, *en3, *pst2, *pen2, *pst3, *pen3, *last3, *cnt3;
    unsigned char *pneed2, *pneed3;            // per sorted pair: its record needs the output
    int *coff2, *coff3;                        // first chunk of every key
    int *ckey2, *cbeg2, *cend2, *ckey3, *cbeg3, *cend3;
    int *sidx;                                 // sorted s2 position of every record
    int *n2, *t3, *n3;                         // pass-2 records per s2 / s3 key, pass-3 per s3 key
    int *off2, *off3;                          // first pass-2 / pass-3 list slot of every key
    int *bh;                                   // radix-sort tile histograms
    unsigned char* old2;                       // s2 counters before the call
    unsigned long long* sw;                    // one-pass scan: published words, per group's first chunk
    int *ghist, *gw, *gstart, *gbase;          // one-pass scan: s2 group order tables
    int2* glist;                               // one-pass scan: (cell, rank) of every s2 ticket
    int *ghist3, *gw3, *gstart3, *gbase3;      // ... and of the s3 level
    int2* glist3;
    int nv = 0;                                // entries of ghist / gstart / gbase
    int* scan_err = nullptr;                   // host memory: a one-pass scan wait ran out
    float* trash;                              // sink of the projection's absent rows
    unsigned char *owner, *pass2, *pass3;
    uint32_t *ka, *kb, *va, *vb, *key3g;
    BlockDesc* bd;
    hipEvent_t done = nullptr;         // the last drain's work on the workspace
    hipStream_t side = nullptr;        // s3 ordering, concurrent with L4 and L5
    hipEvent_t s2_ordered = nullptr;   // s2 tables and pass2 are complete
    hipEvent_t s3_ordered = nullptr;   // s3 tables and pass3 are complete
    hipEvent_t side_done = nullptr;    // the side stream's last work of a call
    hipEvent_t s2_groups = nullptr;    // the one-pass scan's group order is built
    int bh_ints = 0;
    int cus = 0;                       // compute units of the device
    int clk_khz = 0;                   // wall-clock (s_memrealtime) rate
    float* packed = nullptr;           // fragment-order weight copies (packed_weight_floats_d)
    PackedWeights pk = {};
    // phase timings of calls made without sync: their events, read and added
    // to the caller's array when a later call with sync returns
    struct Pending {
        hipEvent_t ev[SSLA_DRAIN_PHASES + 1];
        float* phase_ms;
        unsigned long long pmask;
    };
    std::vector<Pending> pending;
};
constexpr size_t kMaxPending = 256;    // more waiting calls: the oldest is waited for

// Adds the phase times of the oldest `n` pending calls to their arrays and
// frees their events (waiting for each event first).
int flush_pending(Workspace& w, size_t n) {
    n = std::min(n, w.pending.size());
    int rc = SSLA_OK;
    for (size_t i = 0; i < n; ++i) {
        Workspace::Pending& p = w.pending[i];
        for (int k = 0; k < SSLA_DRAIN_PHASES && rc == SSLA_OK; ++k) {
            if (!((p.pmask >> k) & 1ull) || !p.ev[k] || !p.ev[k + 1]) continue;
            float ms = 0.f;
            hipError_t e = hipEventSynchronize(p.ev[k + 1]);
            if (e == hipSuccess) e = hipEventElapsedTime(&ms, p.ev[k], p.ev[k + 1]);
            if (e != hipSuccess) {
                set_error(std::string("drain phase timing: ") + hipGetErrorString(e));
                rc = SSLA_ERR_HIP;
                break;
            }
            p.phase_ms[k] += ms;
        }
        for (int k = 0; k <= SSLA_DRAIN_PHASES; ++k)
            if (p.ev[k]) (void)hipEventDestroy(p.ev[k]);
    }
    w.pending.erase(w.pending.begin(), w.pending.begin() + n);
    return rc;
}

std::mutex g_ws_mu;
Workspace g_ws;
unsigned g_scan_tag = 0;     // tag of the one-pass scan's last launch (under g_ws_mu)

#define HIPCHK(call)                                                          \
    do {                                                                      \
        hipError_t e_ = (call);                                               \
        if (e_ != hipSuccess) {                                               \
            set_error(std::string(#call) + ": " + hipGetErrorString(e_));    \
            return SSLA_ERR_HIP;                                              \
        }                                                                     \
    } while (0)

size_t align_up(size_t v) { return (v + 255) & ~size_t(255); }

int ensure_workspace(int E, int nkeys) {
    if (E <= g_ws.cap && nkeys <= g_ws.cap_keys) return SSLA_OK;
    if (g_ws.base) {
        // the last drain's kernels (both streams, joined into `done`) are the
        // only users of the old workspace
        HIPCHK(hipEventSynchronize(g_ws.done));
        HIPCHK(hipFree(g_ws.base));
        g_ws.base = nullptr;
        g_ws.cap = 0;
    }
    const int cap = std::max(E, std::max(g_ws.cap, 1024));
    const int ck = std::max(nkeys, g_ws.cap_keys);
    const size_t P = (size_t)cap * kPatch;
    const size_t mc = P / kCH + (size_t)ck + 1;    // chunk bound: full chunks + one tail per key
    // a cell's pairs come from distinct records: at most cap, so a cell has at
    // most cap / (kCH kSG) + 2 groups of the one-pass scan
    const size_t nv = (size_t)cap / (kCH * std::min(kSG, kSG3)) + 3;
    // radix-sort tile histograms: (1 << kRMaxBits) digits x tiles
    const size_t bh = ((size_t)1 << kRMaxBits) * (size_t)((cap + kRTile - 1) / kRTile);
    struct Item { void** dst; size_t bytes; };
    Workspace& w = g_ws;
    std::vector<Item> items = {
        {(void**)&w.X0, sizeof(float) * (size_t)cap * SSLA_C1},
        {(void**)&w.X1, sizeof(float) * (size_t)cap * SSLA_C2},
        {(void**)&w.X2, sizeof(float) * (size_t)cap * SSLA_C2},
        {(void**)&w.X3, sizeof(float) * (size_t)cap * SSLA_C3},
        {(void**)&w.X4, sizeof(float) * (size_t)cap * SSLA_C3},
        // [v | g] rows, and kCH rows of padding that a scan chunk may read past
        // the last one
        {(void**)&w.QVG, sizeof(float) * (P + kCH) * 2 * SSLA_C3},
        {(void**)&w.H7, sizeof(float) * (size_t)cap * 7},
        {(void**)&w.cell2, sizeof(int) * (size_t)cap},
        {(void**)&w.pos2, sizeof(int) * P},
        {(void**)&w.pos3, sizeof(int) * P},
        {(void**)&w.list2, sizeof(int) * (size_t)cap},
        {(void**)&w.list3, sizeof(int) * (size_t)cap},
        {(void**)&w.counts, sizeof(int) * 16},
        {(void**)&w.st2, sizeof(int) * (size_t)ck},
        {(void**)&w.en2, sizeof(int) * (size_t)ck},
        {(void**)&w.st3, sizeof(int) * (size_t)ck},
        {(void**)&w.en3, sizeof(int) * (size_t)ck},
        {(void**)&w.pst2, sizeof(int) * (size_t)ck},
        {(void**)&w.pen2, sizeof(int) * (size_t)ck},
        {(void**)&w.pst3, sizeof(int) * (size_t)ck},
        {(void**)&w.pen3, sizeof(int) * (size_t)ck},
        {(void**)&w.last3, sizeof(int) * (size_t)ck},
        {(void**)&w.cnt3, sizeof(int) * (size_t)ck},
        {(void**)&w.owner, (size_t)cap},
        {(void**)&w.pass2, (size_t)cap},
        {(void**)&w.pass3, (size_t)cap},
        {(void**)&w.ka, sizeof(uint32_t) * (size_t)cap},
        {(void**)&w.kb, sizeof(uint32_t) * (size_t)cap},
        {(void**)&w.va, sizeof(uint32_t) * (size_t)cap},
        {(void**)&w.vb, sizeof(uint32_t) * (size_t)cap},
        {(void**)&w.key3g, sizeof(uint32_t) * (size_t)cap},
        {(void**)&w.pneed2, P},
        {(void**)&w.pneed3, P},
        {(void**)&w.sidx, sizeof(int) * (size_t)cap},
        {(void**)&w.coff2, sizeof(int) * (size_t)ck},
        {(void**)&w.coff3, sizeof(int) * (size_t)ck},
        {(void**)&w.n2, sizeof(int) * (size_t)ck},
        {(void**)&w.t3, sizeof(int) * (size_t)ck},
        {(void**)&w.n3, sizeof(int) * (size_t)ck},
        {(void**)&w.off2, sizeof(int) * (size_t)ck},
        {(void**)&w.off3, sizeof(int) * (size_t)ck},
        {(void**)&w.bh, sizeof(int) * bh},
        {(void**)&w.old2, (size_t)ck},
        {(void**)&w.ckey2, sizeof(int) * mc},
        {(void**)&w.cbeg2, sizeof(int) * mc},
        {(void**)&w.cend2, sizeof(int) * mc},
        {(void**)&w.ckey3, sizeof(int) * mc},
        {(void**)&w.cbeg3, sizeof(int) * mc},
        {(void**)&w.cend3, sizeof(int) * mc},
        {(void**)&w.sw, sizeof(unsigned long long) * mc * 3 * SSLA_C3},
        {(void**)&w.ghist, sizeof(int) * nv},
        {(void**)&w.gstart, sizeof(int) * nv},
        {(void**)&w.gbase, sizeof(int) * nv},
        {(void**)&w.gw, sizeof(int) * (size_t)ck},
        {(void**)&w.glist, sizeof(int2) * (mc / kSG + (size_t)ck + 1)},
        {(void**)&w.ghist3, sizeof(int) * nv},
        {(void**)&w.gstart3, sizeof(int) * nv},
        {(void**)&w.gbase3, sizeof(int) * nv},
        {(void**)&w.gw3, sizeof(int) * (size_t)ck},
        {(void**)&w.glist3, sizeof(int2) * (mc / kSG3 + (size_t)ck + 1)},
        {(void**)&w.trash, sizeof(float) * 4 * 64},
        {(void**)&w.bd, sizeof(BlockDesc) * SSLA_MAX_BLOCKS},
    };
    size_t total = 0;
    for (auto& it : items) total += align_up(it.bytes);
    void* base = nullptr;
    HIPCHK(hipMalloc(&base, total));
    char* p = static_cast<char*>(base);
    for (auto& it : items) {
        *it.dst = p;
        p += align_up(it.bytes);
    }
    // no stale word may carry a future launch's tag
    HIPCHK(hipMemset(w.sw, 0, sizeof(unsigned long long) * mc * 3 * SSLA_C3));
    w.nv = (int)nv;
    if (!w.scan_err) {
        HIPCHK(hipHostMalloc((void**)&w.scan_err, sizeof(int), hipHostMallocCoherent));
        *w.scan_err = 0;
    }
    if (!w.done) {
        HIPCHK(hipEventCreateWithFlags(&w.done, hipEventDisableTiming));
        HIPCHK(hipEventCreateWithFlags(&w.s2_ordered, hipEventDisableTiming));
        HIPCHK(hipEventCreateWithFlags(&w.s3_ordered, hipEventDisableTiming));
        HIPCHK(hipEventCreateWithFlags(&w.side_done, hipEventDisableTiming));
        HIPCHK(hipEventCreateWithFlags(&w.s2_groups, hipEventDisableTiming));
        HIPCHK(hipStreamCreateWithFlags(&w.side, hipStreamNonBlocking));
        HIPCHK(hipMalloc(&w.packed, sizeof(float) * packed_weight_floats_d()));
        int dev = 0;
        HIPCHK(hipGetDevice(&dev));
        HIPCHK(hipDeviceGetAttribute(&w.cus, hipDeviceAttributeMultiprocessorCount, dev));
        HIPCHK(hipDeviceGetAttribute(&w.clk_khz, hipDeviceAttributeWallClockRate, dev));
    }
    w.base = base;
    w.bytes = total;
    w.cap = cap;
    w.cap_keys = ck;
    w.bh_ints = (int)bh;
    return SSLA_OK;
}

int bits_for(uint32_t v) {
    int b = 1;
    while ((1u << b) <= v && b < 32) ++b;
    return b;
}

inline unsigned grid1(long long n, int bs) { return (unsigned)((n + bs - 1) / bs); }

// Every return of a call after its first launch passes through finish():
// the side stream's work joins `st`, and `done` marks the end of the call's
// use of the workspace, so the next call (on any stream) and a workspace
// regrowth wait for all of it -- also when the call stops at an error.
struct CallEnd {
    Workspace& w;
    hipStream_t st;
    bool ended = false;
    void finish() {
        if (ended) return;
        ended = true;
        (void)hipEventRecord(w.side_done, w.side);
        (void)hipStreamWaitEvent(st, w.side_done, 0);
        (void)hipEventRecord(w.done, st);
    }
    ~CallEnd() { finish(); }
};

}  // namespace

namespace {
// zero fill of n bytes at p (16-byte stores for the aligned body)
__global__ void k_zero_bytes(unsigned char* __restrict__ p, size_t n) {
    const size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x;
    const size_t n16 = n >> 4;
    if (i < n16) reinterpret_cast<uint4*>(p)[i] = make_uint4(0u, 0u, 0u, 0u);
    if (i < (n & 15)) p[(n16 << 4) + i] = 0;
}
}  // namespace

int zero_async(void* p, size_t nbytes, hipStream_t st) {
    if (!nbytes) return SSLA_OK;
    if (!p || (reinterpret_cast<uintptr_t>(p) & 15)) {
        set_error("zero_async: null or unaligned pointer");
        return SSLA_ERR_ARG;
    }
    const size_t n16 = std::max<size_t>(nbytes >> 4, 16);
    hipLaunchKernelGGL(k_zero_bytes, dim3((unsigned)((n16 + 255) / 256)), dim3(256), 0, st,
                       static_cast<unsigned char*>(p), nbytes);
    const hipError_t e = hipGetLastError();
    if (e != hipSuccess) {
        set_error(std::string("zero_async: ") + hipGetErrorString(e));
        return SSLA_ERR_HIP;
    }
    return SSLA_OK;
}

int drain_reserve(const HybridS2S3Config* cfg, int max_records) {
    if (!cfg || cfg->n_blocks < 1 || cfg->n_blocks > SSLA_MAX_BLOCKS || cfg->H2 <= 0 ||
        cfg->W2 <= 0 || cfg->H2 > 65535 || cfg->W2 > 65535 || max_records < 0 ||
        (long long)max_records * kPatch > 0x7fffffffLL ||
        (long long)cfg->n_blocks * cfg->H2 * cfg->W2 >= 0x7fffffffLL) {
        set_error("drain_reserve: bad configuration or record count");
        return SSLA_ERR_ARG;
    }
    std::lock_guard<std::mutex> lock(g_ws_mu);
    return ensure_workspace(std::max(max_records, 1), cfg->n_blocks * cfg->H2 * cfg->W2 + 1);
}

int scan_drain(const HybridS2S3Config* cfg, const HybridInputRec* const* rings,
               const int* ns, HybridS2S3OutputSlot* const* outs,
               float* const* head_outs, hipStream_t st, bool sync,
               float* phase_ms, unsigned long long phase_mask) {
    const int nb = cfg->n_blocks;
    if (nb < 1 || nb > SSLA_MAX_BLOCKS) {
        set_error("n_blocks must be in [1, 16]");
        return SSLA_ERR_ARG;
    }
    if (cfg->H2 <= 0 || cfg->W2 <= 0 || (cfg->H2 & 1) || (cfg->W2 & 1) ||
        cfg->H3 != cfg->H2 / 2 || cfg->W3 != cfg->W2 / 2 ||
        cfg->H2 > 65535 || cfg->W2 > 65535) {
        set_error("grid must have even H2, W2 and H3 = H2/2, W3 = W2/2");
        return SSLA_ERR_ARG;
    }
    for (int b = 0; b < nb; ++b) {
        for (int li = 0; li < 4; ++li) {
            const LayerWeightsS2S3& L = cfg->layers[b][li];
            const LayerWeightsS2S3& L0 = cfg->layers[0][li];
            if (!L.qvgIn || !L.goW || !L.ln_gamma || !L.ln_beta) {
                set_error("layer weights not bound for block " + std::to_string(b));
                return SSLA_ERR_ARG;
            }
            if (L.qvgIn != L0.qvgIn || L.goW != L0.goW || L.input_proj != L0.input_proj ||
                L.ln_gamma != L0.ln_gamma || L.ln_beta != L0.ln_beta) {
                set_error("all blocks must share one set of layer weights");
                return SSLA_ERR_ARG;
            }
            if (!cfg->hidden[b][li]) {
                set_error("hidden state not allocated for block " + std::to_string(b));
                return SSLA_ERR_ARG;
            }
        }
        if (!cfg->tdrop_s2[b] || !cfg->tdrop_s3[b]) {
            set_error("tdrop counters not allocated for block " + std::to_string(b));
            return SSLA_ERR_ARG;
        }
        if (ns[b] < 0 || (ns[b] > 0 && !rings[b])) {
            set_error("bad ring / count for block " + std::to_string(b));
            return SSLA_ERR_ARG;
        }
    }
    if ((cfg->layers[0][0].input_proj == nullptr) || (cfg->layers[0][2].input_proj == nullptr) ||
        cfg->layers[0][1].input_proj != nullptr || cfg->layers[0][3].input_proj != nullptr) {
        set_error("L4/L6 need input_proj and L5/L7 must not have one");
        return SSLA_ERR_ARG;
    }
    long long E64 = 0;
    for (int b = 0; b < nb; ++b) E64 += ns[b];
    if (E64 * kPatch > 0x7fffffffLL) {
        set_error("too many records in one call");
        return SSLA_ERR_ARG;
    }
    const int E = (int)E64;
    Geometry G;
    G.H2 = cfg->H2; G.W2 = cfg->W2; G.H3 = cfg->H3; G.W3 = cfg->W3;
    G.C2 = G.H2 * G.W2; G.C3 = G.H3 * G.W3; G.nb = nb; G.window = cfg->tdrop_window;
    const uint32_t nk2 = (uint32_t)(nb * G.C2), nk3 = (uint32_t)(nb * G.C3);
    const int head = head_kind(cfg);
    const bool have_head = head != kHeadNone;
    if (const char* m = head_missing(cfg)) {
        set_error(m);
        return SSLA_ERR_ARG;
    }

    std::lock_guard<std::mutex> lock(g_ws_mu);
    if (E == 0) return SSLA_OK;
    {
        const int rc = ensure_workspace(E, (int)nk2 + 1);
        if (rc) return rc;
    }
    Workspace& w = g_ws;
    CallEnd end{w, st};

    BlockTable tab;
    std::memset(&tab, 0, sizeof tab);
    BlockDesc* hbd = tab.d;
    int off = 0;
    for (int b = 0; b < nb; ++b) {
        BlockDesc& d = hbd[b];
        d.ring = rings[b];
        d.out = outs ? outs[b] : nullptr;
        d.head_out = head_outs ? head_outs[b] : nullptr;
        for (int li = 0; li < 4; ++li) d.hidden[li] = cfg->hidden[b][li];
        d.td2 = cfg->tdrop_s2[b];
        d.td3 = cfg->tdrop_s3[b];
        d.preds = have_head ? cfg->preds[b] : nullptr;
        d.version = have_head ? cfg->version[b] : nullptr;
        d.strip = cfg->strip[b];
        d.n = ns[b];
        d.offset = off;
        off += ns[b];
    }
    // blocks with n == 0 must not capture records: move their offset past E.
    for (int b = 0; b < nb; ++b)
        if (hbd[b].n == 0) hbd[b].offset = E + 1;
    // Calls share one workspace: a call on another stream runs after the
    // previous call's kernels (device-side wait, the host does not block).
    HIPCHK(hipStreamWaitEvent(st, w.done, 0));

    // Phase timing (optional): events recorded on `st` at the boundaries of
    // the phases in pmask only -- each event costs a few microseconds of
    // queue time between the kernels it separates.
    hipEvent_t ev[SSLA_DRAIN_PHASES + 1] = {};
    int n_mark = 0;
    const unsigned long long pmask = phase_ms ? (phase_mask ? phase_mask : ~0ull) : 0ull;
    struct EvFree {
        hipEvent_t* ev;
        ~EvFree() {
            for (int k = 0; k <= SSLA_DRAIN_PHASES; ++k)
                if (ev[k]) (void)hipEventDestroy(ev[k]);
        }
    } ev_free{ev};
    auto mark = [&]() -> int {
        const int b = n_mark++;                       // boundary b opens phase b
        if (b > SSLA_DRAIN_PHASES) return SSLA_OK;
        if (!((pmask >> b) & 1ull) && !(b > 0 && ((pmask >> (b - 1)) & 1ull))) return SSLA_OK;
        HIPCHK(hipEventCreate(&ev[b]));
        HIPCHK(hipEventRecord(ev[b], st));
        return SSLA_OK;
    };
#define MARK() do { const int rc_ = mark(); if (rc_) return rc_; } while (0)
    // fragment-order copies of the layer weights for the MFMA kernels, rebuilt
    // by every call (in k_decode's launch), so weights rewritten in place by
    // any means are always the ones used
    const PackSrc psrc = pack_setup<true>(cfg->layers[0], w.packed, &w.pk);
    const PackedWeights& pk = w.pk;
    MARK();
    // per-call fills: run bounds of the s2 keys (k_runs writes those that
    // occur), the list and chunk counters, the prediction-grid writers
    // one-pass scan: the group-count bound of this call's cells (see ensure_workspace)
    const int nv2 = E / (kCH * kSG) + 3, nv3 = E / (kCH * kSG3) + 3;
    FillSet f{};
    {
        int* arr[kFills] = {w.st2, w.en2, w.counts, w.last3, w.cnt3, w.ghist, w.ghist3};
        const int len[kFills] = {(int)nk2, (int)nk2, 16, have_head ? (int)nk3 : 0,
                                 have_head ? (int)nk3 : 0, nv2, nv3};
        const int val[kFills] = {0, 0, 0, -1, 0, 0, 0};
        for (int i = 0; i < kFills; ++i) {
            f.p[i] = arr[i];
            f.n[i] = len[i];
            f.v[i] = val[i];
        }
    }
    // ---- decode (and the fills); stable radix sort of the records by s2 key --
    {
        const int ndec = (int)grid1(E, kDecRec), fblk = (int)grid1(std::max<int>(std::max<int>((int)nk2, 16), nv3), 256);
        const int npk = (int)((PackLayout<true>::off[8] + 255) / 256);
        hipLaunchKernelGGL(k_decode, dim3(ndec + fblk * kFills + npk + 1), dim3(256), 0, st, E, tab,
                           w.bd, G, w.X0, w.cell2, w.owner, w.ka, w.va, ndec, f, fblk, psrc,
                           w.packed, npk);
    }
    const int bits2 = bits_for(nk2);
    const int passes = (bits2 + kRMaxBits - 1) / kRMaxBits;
    const int T = (int)grid1(E, kRTile);
    uint32_t *kin = w.ka, *vin = nullptr, *kout = w.kb, *vout = w.vb;
    for (int ps = 0, shift = 0; ps < passes; ++ps) {
        const int bits = (bits2 - shift + (passes - ps) - 1) / (passes - ps);
        if ((1 << bits) * T > w.bh_ints) {
            set_error("drain: radix histogram larger than its workspace");
            return SSLA_ERR_STATE;
        }
        // a one-pass sort's digit is the whole key: bins for the keys present
        // (nk2 values and the keyless records' nk2) only
        const int nbins = passes == 1 ? (int)nk2 + 1 : 1 << bits;
        hipLaunchKernelGGL(k_rs_hist, dim3(T), dim3(kRThreads), 0, st, E, kin, shift, bits, nbins,
                           T, w.bh);
        hipLaunchKernelGGL(k_exscan, dim3(1), dim3(kScanThreads), 0, st, nbins * T, w.bh);
        hipLaunchKernelGGL(k_rs_scatter, dim3(T), dim3(kRThreads), 0, st, E, kin, vin, kout, vout,
                           ps == passes - 1 ? w.sidx : nullptr, shift, bits, nbins, T, w.bh);
        shift += bits;
        // the next pass writes the pair of buffers this pass read from
        uint32_t* const k2 = kout == w.kb ? w.ka : w.kb;
        uint32_t* const v2 = vout == w.vb ? w.va : w.vb;
        kin = kout;
        vin = vout;
        kout = k2;
        vout = v2;
    }
    // the sorted s2 order, and the buffers the s3 order is placed in
    uint32_t* const K2 = kin;
    uint32_t* const V2 = vin;
    uint32_t* const K3 = kout;
    uint32_t* const V3 = vout;
    // ---- counters, tdrop_s2, the pass-2 list, s2 pair and chunk tables -----
    if (passes == 1 && nk2 <= (uint32_t)kScanThreads) {
        // the one pass's histogram holds the run bounds: the key tables and
        // their scans in one workgroup
        const KeyHist kh{G.C2, G.W2, G.H2, T, G.window, (const int*)w.bh, w.st2, w.en2, w.bd,
                         w.old2};
        hipLaunchKernelGGL(k_keyscan<true>, dim3(1), dim3(kScanThreads), 0, st, (int)nk2,
                           (const int*)nullptr, w.pst2, w.pen2, w.coff2, w.counts + 2, w.n2,
                           w.off2, w.counts + 0, kh);
    } else {
        hipLaunchKernelGGL(k_runs, dim3(grid1(E, 256)), dim3(256), 0, st, E, K2, nk2, w.st2, w.en2);
        hipLaunchKernelGGL(k_keys2, dim3(grid1(nk2, 256)), dim3(256), 0, st, nk2, G.C2, G.W2, G.H2,
                           w.st2, w.en2, w.bd, G.window, w.old2, w.n2, w.pen2);
        hipLaunchKernelGGL(k_keyscan<false>, dim3(1), dim3(kScanThreads), 0, st, (int)nk2, w.pen2,
                           w.pst2, w.pen2, w.coff2, w.counts + 2, w.n2, w.off2, w.counts + 0,
                           KeyHist{});
    }
    {
        const unsigned nbr = grid1(E, 256);
        hipLaunchKernelGGL(k_s2_tables, dim3(nbr + grid1(nk2, 4)), dim3(256), 0, st, E, (int)nbr,
                           K2, V2, nk2, G.C2, G.W2, G.H2, w.st2, w.en2, w.pst2, w.pen2, w.coff2,
                           w.old2, w.off2, G.window, w.pass2, w.list2, w.pos2, w.pneed2, w.ckey2,
                           w.cbeg2, w.cend2, w.ghist, w.gw);
    }
    // The s3 ordering needs only the s2 order, pass2 and the old counters, so
    // it runs on the side stream while L4 and L5 run here; L6 waits for it.
    // Its launches are sized by E; the pass-2 count stays on the device.  Its
    // event sits before L4's projection, so the side stream's small kernels
    // start beside the projection rather than beside the latency-bound parts
    // that follow it.
    HIPCHK(hipEventRecord(w.s2_ordered, st));
    hipStream_t s3 = w.side;
    HIPCHK(hipStreamWaitEvent(s3, w.s2_ordered, 0));
    MARK();
    const LayerWeightsS2S3* L = cfg->layers[0];
    // The pass-2 and pass-3 counts stay on the device; the launches over their
    // lists are sized by bounds the host has.  A cell's L records in a row take
    // at most L P / 256 + 2 passes of the tdrop gate, P = ceil(256 / window)
    // the passing counter values per 256: any 256 consecutive values hold P,
    // and a shorter run, cut in two by the wrap, at most a1 / w + a2 / w + 2.
    const long long Pw = G.window <= 1 ? 256 : (256 + G.window - 1) / G.window;
    const int nmax2 = (int)std::min<long long>(E, ((long long)E * Pw + 255) / 256 + 2LL * nk2);
    const int nmax3 = (int)std::min<long long>(nmax2, ((long long)nmax2 * Pw + 255) / 256 + 2LL * nk3);
    const unsigned tiles2 = grid1(nmax2, kTM), tiles3 = grid1(nmax3, kTM);
    // persistent projection grids (80-record tiles loop over the workgroups):
    // measured at 200k records (2500 tiles), L4 is fastest with 6 workgroups
    // per CU, L5 with 5 (both: all resident, about two tiles each); 64-record
    // tiles (3125, some workgroups running a third) were 10% slower.
    const unsigned tilesP = grid1(E, kTMP);
    const unsigned cus = w.cus > 0 ? (unsigned)w.cus : tilesP;
    const unsigned gridP4 = std::min(tilesP, 6u * cus);
    const unsigned gridP5 = std::min(tilesP, 5u * cus);
    const unsigned char* all = nullptr;             // every pair's record needs h
    // L4's and L5's h, compact (pairs, 48), behind their (pairs, 96) rows
    float* const Hc = w.QVG + (size_t)w.cap * kPatch * 2 * SSLA_C2;
    // S: the recurrence of layer LI over the chunk tables of level LV (2: s2,
    // 3: s3; n_chunks in counts[NC]), h written at HOUT (rows of HS floats)
    // where the pair's record needs the output (NEED, or every pair), in one
    // pass (k_scan; ticket counter counts[8 + LI], group count counts[NG]).
    const unsigned long long wait_ticks = (unsigned long long)std::max(w.clk_khz, 1) * 500ull;
#define SCAN1(OUT, HS, SGV, LI, LV, NG, GL, NEED, HOUT, CELLS, GRID)                                  \
    do {                                                                                            \
        unsigned tag_ = ++g_scan_tag;                                                               \
        if (tag_ == 0) tag_ = ++g_scan_tag;                                                         \
        MARK();                                                                                     \
        MARK();                                                                                     \
        hipLaunchKernelGGL((k_scan<OUT, HS, SGV>), dim3(GRID), dim3(SGV * ((OUT + 63) / 64) * 64), 0, \
                           st, (const int*)(w.counts + NG), w.counts + 8 + LI, tag_, GL,             \
                           w.cbeg##LV, w.cend##LV, w.coff##LV, w.pst##LV, w.pen##LV, CELLS, w.bd,   \
                           LI, NEED, w.QVG, HOUT, w.sw, w.scan_err, wait_ticks);                    \
        MARK();                                                                                     \
    } while (0)
    // workgroups of the one-pass scans: one per group (at most one per kSG
    // chunks plus one per key); those past the group count exit at once
    const unsigned groups2 = (unsigned)(((size_t)E * kPatch / kCH + nk2 + 1) / kSG + nk2 + 1);
    const unsigned groups3 = (unsigned)(((size_t)nmax2 * kPatch / kCH + nk3 + 1) / kSG3 + nk3 + 1);
    // ---- L4: 24 -> 48, all records ----------------------------------------
    hipLaunchKernelGGL((k_qvg<SSLA_C1, SSLA_C2, true, kTMP>), dim3(gridP4), dim3(256), 0, st, E,
                       (const int*)nullptr, (const int*)nullptr, w.X0, w.pos2, pk.pp[0], w.QVG, w.trash);
    // [side] the s2 one-pass scan's ticket order, beside L4's projection
    hipLaunchKernelGGL(k_group_order, dim3(1), dim3(kScanThreads), 0, s3, (int)nk2, nv2, kSG, w.pst2,
                       w.pen2, w.ghist, w.gw, w.gstart, w.gbase, w.glist, w.counts + 6);
    HIPCHK(hipEventRecord(w.s2_groups, s3));
    MARK();
    HIPCHK(hipStreamWaitEvent(st, w.s2_groups, 0));
    SCAN1(SSLA_C2, SSLA_C2, kSG, 0, 2, 6, w.glist, all, Hc, G.C2, groups2);
    hipLaunchKernelGGL((k_outt<SSLA_C1, SSLA_C2, 2, 1, 3, SSLA_C2>), dim3(grid1(E, 32)), dim3(64), 0,
                       st, E, (const int*)nullptr, (const int*)nullptr, w.X0, w.pos2, Hc, pk.po[0],
                       L[0].ln_gamma, L[0].ln_beta, w.X1);
    MARK();
    // ---- [side] the s3 record order, tdrop_s3, s3 pair and chunk tables ---
    // (enqueued after L4's launches: the host needs a few microseconds per
    // launch, and L4 keeps the device busy meanwhile)
    hipLaunchKernelGGL(k_keys3a, dim3(grid1(nk3, 256)), dim3(256), 0, s3, nk3, G, w.n2, w.bd,
                       w.t3, w.n3);
    hipLaunchKernelGGL(k_keyscan<false>, dim3(1), dim3(kScanThreads), 0, s3, (int)nk3, w.t3, w.st3,
                       w.en3, (int*)nullptr, (int*)nullptr, w.n3, w.off3, w.counts + 1,
                       KeyHist{});
    hipLaunchKernelGGL(k_place3, dim3(grid1(nmax2, 256)), dim3(256), 0, s3, (const int*)(w.counts + 0),
                       w.list2, w.bd, G, w.cell2, w.sidx, V2, w.st2, w.en2, w.old2, w.st3, K3, V3,
                       w.key3g);
    hipLaunchKernelGGL(k_tdrop3, dim3(grid1(nmax2, 256)), dim3(256), 0, s3, (const int*)(w.counts + 0),
                       K3, V3, nk3, G.C3, w.st3, w.off3, w.bd, G.window, w.owner,
                       have_head ? 1 : 0, w.pass3, w.list3, w.last3, w.cnt3);
    hipLaunchKernelGGL(k_keys3b, dim3(grid1(nk3, 256)), dim3(256), 0, s3, nk3, G, w.t3, w.bd,
                       w.pen3);
    hipLaunchKernelGGL(k_keyscan<false>, dim3(1), dim3(kScanThreads), 0, s3, (int)nk3, w.pen3, w.pst3,
                       w.pen3, w.coff3, w.counts + 3, (const int*)nullptr, (int*)nullptr,
                       (int*)nullptr, KeyHist{});
    hipLaunchKernelGGL(k_chunks, dim3(grid1(nk3, 4)), dim3(256), 0, s3, nk3, w.pst3, w.pen3,
                       w.coff3, w.ckey3, w.cbeg3, w.cend3, w.ghist3, w.gw3);
    hipLaunchKernelGGL(k_group_order, dim3(1), dim3(kScanThreads), 0, s3, (int)nk3, nv3, kSG3, w.pst3,
                       w.pen3, w.ghist3, w.gw3, w.gstart3, w.gbase3, w.glist3, w.counts + 7);
    hipLaunchKernelGGL(k_pair_rank, dim3(grid1(nmax2, 256)), dim3(256), 0, s3, E,
                       (const int*)(w.counts + 0), K3, V3, nk3, G.C3, G.W3, G.H3, w.st3, w.en3,
                       w.pst3, w.pos3, w.pneed3, w.pass3);
    HIPCHK(hipEventRecord(w.s3_ordered, s3));
    HIPCHK(hipGetLastError());
    // ---- L5: 48 -> 48, state for all records, output for pass2 ---------------
    hipLaunchKernelGGL((k_qvg<SSLA_C2, SSLA_C2, true, kTMP>), dim3(gridP5), dim3(256), 0, st, E,
                       (const int*)nullptr, (const int*)nullptr, w.X1, w.pos2, pk.pp[1], w.QVG, w.trash);
    MARK();
    SCAN1(SSLA_C2, SSLA_C2, kSG, 1, 2, 6, w.glist, w.pneed2, Hc, G.C2, groups2);
    hipLaunchKernelGGL((k_outt<SSLA_C2, SSLA_C2, kOutRT5, kOutKS5, 1, SSLA_C2>), dim3(grid1(nmax2, 16 * kOutRT5)),
                       dim3(64 * kOutKS5), 0,
                       st, E, (const int*)(w.counts + 0), w.list2, w.X1, w.pos2, Hc, pk.po[1],
                       L[1].ln_gamma, L[1].ln_beta, w.X2);
    MARK();
    // ---- L6: 48 -> 96, pass2 records ------------------------------------------
    HIPCHK(hipStreamWaitEvent(st, w.s3_ordered, 0));
    hipLaunchKernelGGL((k_qvg<SSLA_C2, SSLA_C3, false, kTM, 2>), dim3(tiles2 * 2), dim3(256), 0, st, E,
                       (const int*)(w.counts + 0), w.list2, w.X2, w.pos3, pk.pp[2], w.QVG, w.trash);
    MARK();
    SCAN1(SSLA_C3, 2 * SSLA_C3, kSG3, 2, 3, 7, w.glist3, all, w.QVG, G.C3, groups3);
    hipLaunchKernelGGL((k_outt<SSLA_C2, SSLA_C3, kOutRT6, kOutKS6>), dim3(grid1(nmax2, 16 * kOutRT6)),
                       dim3(64 * kOutKS6), 0, st, E,
                       (const int*)(w.counts + 0), w.list2, w.X2, w.pos3, w.QVG, pk.po[2],
                       L[2].ln_gamma, L[2].ln_beta, w.X3);
    MARK();
    // ---- L7: 96 -> 96, state for pass2, output for pass3 ----------------------
    hipLaunchKernelGGL((k_qvg<SSLA_C3, SSLA_C3, false, kTM, 4>), dim3(tiles2 * 4), dim3(256), 0, st, E,
                       (const int*)(w.counts + 0), w.list2, w.X3, w.pos3, pk.pp[3], w.QVG, w.trash);
    MARK();
    SCAN1(SSLA_C3, 2 * SSLA_C3, kSG3, 3, 3, 7, w.glist3, w.pneed3, w.QVG, G.C3, groups3);
    hipLaunchKernelGGL((k_outt<SSLA_C3, SSLA_C3, kOutRT7, kOutKS7>), dim3(grid1(nmax3, 16 * kOutRT7)),
                       dim3(64 * kOutKS7), 0, st, E,
                       (const int*)(w.counts + 1), w.list3, w.X3, w.pos3, w.QVG, pk.po[3],
                       L[3].ln_gamma, L[3].ln_beta, w.X4);
    MARK();
    HIPCHK(hipGetLastError());
    // ---- head ------------------------------------------------------------------
    if (have_head) {
        const HeadPtrs hp = head_ptrs(cfg);
        if (head == kHeadYolox)
            hipLaunchKernelGGL(k_head, dim3(tiles3), dim3(256), 0, st, (const int*)(w.counts + 1),
                               w.list3, w.X4, hp, w.H7);
        else
            hipLaunchKernelGGL(k_head_linear, dim3(tiles3), dim3(256), 0, st,
                               (const int*)(w.counts + 1), w.list3, w.X4, hp, w.H7);
        hipLaunchKernelGGL(k_pred_write, dim3(grid1(nmax3, 256)), dim3(256), 0, st,
                           (const int*)(w.counts + 1), w.list3, w.owner, w.key3g, w.last3,
                           w.cnt3, w.bd, G, w.H7);
    }
    MARK();
    hipLaunchKernelGGL(k_emit, dim3(grid1(E, kEmitRec)), dim3(256), 0, st, E, w.bd, nb, w.cell2, w.owner,
                       w.pass2, w.pass3, w.X4, w.H7, have_head ? 1 : 0);
    HIPCHK(hipGetLastError());
    MARK();
#undef MARK
#undef SCAN1
    end.finish();
    if (phase_ms) {
        // this call's events join the pending ones (read below when sync is
        // set, else by a later call with sync)
        if (w.pending.size() >= kMaxPending) {
            const int rc = flush_pending(w, 1);
            if (rc) return rc;
        }
        Workspace::Pending p;
        for (int k = 0; k <= SSLA_DRAIN_PHASES; ++k) {
            p.ev[k] = ev[k];
            ev[k] = nullptr;
        }
        p.phase_ms = phase_ms;
        p.pmask = pmask;
        w.pending.push_back(p);
    }
    if (sync) {
        HIPCHK(hipStreamSynchronize(st));
        if (__atomic_exchange_n(w.scan_err, 0, __ATOMIC_RELAXED)) {
            set_error("drain: a wait of the one-pass scan ran out (results are invalid)");
            return SSLA_ERR_HIP;
        }
        // every earlier call finished before this one's kernels started
        const int rc = flush_pending(w, w.pending.size());
        if (rc) return rc;
    }
    return SSLA_OK;
}

}  // namespace ssla
