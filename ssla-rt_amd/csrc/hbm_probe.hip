// hbm_probe.hip -- measured HBM ceilings for the roofline report.
//
// The published MI355X figure (8 TB/s) is the sum of read and write
// capacity; a kernel that mostly writes cannot reach it.  These probes time,
// on the calling device, the traffic patterns the drain's kernels make:
//   0  streaming writes (16-byte stores over 1 GiB),
//   1  a streaming copy (read + write, bytes of both counted),
//   2  576-byte rows (the L4 pair-row width) at a random permutation of
//      1.8 M positions, each row written as 16-float segments the way an
//      MFMA 16x16 output tile leaves a wave (lane l: row 4*(l/16)+r,
//      column l%16).
// No counterpart in the reference.  Built as libssla_probe.so, apart from the
// drain library, and loaded by bench.py only.  Entry point:
//   int ssla_probe_hbm_ceiling(double* gbs, int n)   0, or -1 (n < 3) /
//       -2 (HIP failure; ssla_probe_last_error() names the call)
#include <hip/hip_runtime.h>

#include <algorithm>
#include <cstdint>
#include <numeric>
#include <random>
#include <string>
#include <vector>

namespace {

std::string g_err;

typedef float f4 __attribute__((ext_vector_type(4)));

__global__ void k_probe_write(f4* __restrict__ p, size_t n4) {
    for (size_t i = blockIdx.x * (size_t)blockDim.x + threadIdx.x; i < n4;
         i += (size_t)gridDim.x * blockDim.x)
        p[i] = f4{1.f, 2.f, 3.f, 4.f};
}

__global__ void k_probe_copy(const f4* __restrict__ a, f4* __restrict__ b, size_t n4) {
    for (size_t i = blockIdx.x * (size_t)blockDim.x + threadIdx.x; i < n4;
         i += (size_t)gridDim.x * blockDim.x)
        b[i] = a[i];
}

constexpr int kRowF = 144;   // floats per row

__global__ void k_probe_rows(float* __restrict__ out, const int* __restrict__ perm, int nrows) {
    const int lane = threadIdx.x & 63, wv = threadIdx.x >> 6;
    const int r0 = (blockIdx.x * 4 + wv) * 16;
    if (r0 >= nrows) return;
    for (int ct = 0; ct < kRowF / 16; ++ct)
        for (int r = 0; r < 4; ++r) {
            const int row = r0 + 4 * (lane >> 4) + r;
            if (row < nrows) out[(size_t)perm[row] * kRowF + ct * 16 + (lane & 15)] = (float)row;
        }
}

#define PCHK(call)                                                            \
    do {                                                                      \
        hipError_t e_ = (call);                                               \
        if (e_ != hipSuccess) {                                               \
            g_err = std::string(#call) + ": " + hipGetErrorString(e_);       \
            rc = -2;                                                          \
            goto done;                                                        \
        }                                                                     \
    } while (0)

}  // namespace

extern "C" const char* ssla_probe_last_error(void) { return g_err.c_str(); }

extern "C" int ssla_probe_hbm_ceiling(double* gbs, int n) {
    if (!gbs || n < 3) {
        g_err = "hbm_ceiling: need 3 slots";
        return -1;
    }
    int rc = 0;
    const size_t bytes = 1ull << 30;
    const int nrows = 1800000;           // 1.8 M x 576 B = 1.04 GB < 1 GiB buffer
    f4 *a = nullptr, *b = nullptr;
    int* perm = nullptr;
    hipEvent_t e0 = nullptr, e1 = nullptr;
    std::vector<int> hp(nrows);
    std::iota(hp.begin(), hp.end(), 0);
    std::mt19937 rng(1);
    std::shuffle(hp.begin(), hp.end(), rng);
    static_assert((size_t)1800000 * kRowF * sizeof(float) <= (1ull << 30), "rows fit the buffer");
    PCHK(hipMalloc(&a, bytes));
    PCHK(hipMalloc(&b, bytes));
    PCHK(hipMalloc(&perm, sizeof(int) * nrows));
    PCHK(hipMemcpy(perm, hp.data(), sizeof(int) * nrows, hipMemcpyHostToDevice));
    PCHK(hipEventCreate(&e0));
    PCHK(hipEventCreate(&e1));
    for (int k = 0; k < 3; ++k) {
        const double moved = k == 0 ? (double)bytes : k == 1 ? 2.0 * bytes : (double)nrows * kRowF * 4;
        for (int rep = 0; rep < 11; ++rep) {      // one warm-up, ten timed
            if (rep == 1) PCHK(hipEventRecord(e0, nullptr));
            if (k == 0)
                hipLaunchKernelGGL(k_probe_write, dim3(4096), dim3(256), 0, nullptr, a, bytes / 16);
            else if (k == 1)
                hipLaunchKernelGGL(k_probe_copy, dim3(4096), dim3(256), 0, nullptr, a, b, bytes / 16);
            else
                hipLaunchKernelGGL(k_probe_rows, dim3((nrows / 16 + 3) / 4), dim3(256), 0, nullptr,
                                   (float*)a, perm, nrows);
        }
        PCHK(hipGetLastError());
        PCHK(hipEventRecord(e1, nullptr));
        PCHK(hipEventSynchronize(e1));
        float ms = 0.f;
        PCHK(hipEventElapsedTime(&ms, e0, e1));
        gbs[k] = moved / (ms / 10.0 * 1e-3) / 1e9;
    }
done:
    if (e0) (void)hipEventDestroy(e0);
    if (e1) (void)hipEventDestroy(e1);
    if (a) (void)hipFree(a);
    if (b) (void)hipFree(b);
    if (perm) (void)hipFree(perm);
    return rc;
}
