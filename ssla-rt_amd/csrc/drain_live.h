// drain_live.h -- internal interface of the batch-mode and persistent live
// drains (drain_live.hip) used by the C ABI (api.cpp).
#pragma once

#include <hip/hip_runtime.h>

#include <string>

#include "ssla_hip.h"

namespace ssla {

constexpr int kLiveBatchMax = 32;   // records per in-kernel batch, at most
constexpr int kGroupMin = 3, kGroupMax = 6;   // workgroups per block of a group drain

void set_error(const std::string& msg);

// The [ping, pong] words of block blk's clock anchors when they were
// allocated by ssla_hip_timing_alloc, else null.
unsigned long long* timing_clock_sync(const HybridS2S3Config* cfg, int blk);

// Drains pre-filled rings in batches of `batch` records (ring order), one
// workgroup per block; batch_clks[b] (optional) receives a (t_pop, t_done)
// wall-clock pair per batch; phase_us (optional, needs sync) accumulates the
// in-kernel phase profile (SSLA_BATCH_PHASES slots).
int batch_drain(const HybridS2S3Config* cfg, const HybridInputRec* const* rings, const int* ns,
                HybridS2S3OutputSlot* const* outs, float* const* head_outs,
                unsigned long long* const* batch_clks, int batch, hipStream_t st, bool sync,
                double* phase_us);

// The batch drain with the device memory it needs beyond its inputs and
// outputs in a static per-device array (noalloc_scratch_bytes() bytes,
// up to SSLA_MAX_BLOCKS blocks): allocates nothing.  Asynchronous on st.
int batch_drain_noalloc(const HybridS2S3Config* cfg, const HybridInputRec* const* rings,
                        const int* ns, HybridS2S3OutputSlot* const* outs,
                        float* const* head_outs, int batch, hipStream_t st);
size_t noalloc_scratch_bytes();

struct LiveSession;

// group 1: one workgroup per block (k_live); kGroupMin..kGroupMax: that
// many workgroups per block, each owning channel slices (k_group); stages 2
// (with a group): two such groups per block in a pipeline, L4-L5 and L6-head.
int live_start(const HybridS2S3Config* cfg, HybridInputRec* const* rings,
               unsigned long long ring_mask, unsigned long long* const* tails, int* stop_flag,
               unsigned long long* const* events_done, unsigned int spin_ns, int max_batch,
               unsigned int idle_timeout_ms, double* phase_us, int group, int stages,
               LiveSession** out);

// The batch drain with `group` workgroups per block (kGroupMin..kGroupMax);
// synchronous on st.
int batch_drain_group(const HybridS2S3Config* cfg, const HybridInputRec* const* rings, const int* ns,
                      HybridS2S3OutputSlot* const* outs, float* const* head_outs, int batch,
                      int group, hipStream_t st, double* phase_us);

// Waits until the kernel has exited (after the caller set *stop_flag) and
// frees the session; *status_out: 0 stopped by flag, 2 ring overrun,
// 3 idle timeout.
int live_wait(LiveSession* s, int timeout_ms, int* status_out);

}  // namespace ssla
