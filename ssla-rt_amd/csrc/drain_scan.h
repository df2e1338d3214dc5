// drain_scan.h -- internal interface between the C ABI (api.cpp) and the
// whole-ring drain (drain_scan.hip).
#pragma once

#include <hip/hip_runtime.h>

#include <string>

#include "ssla_hip.h"

namespace ssla {

// Records `msg` as the calling thread's last error (ssla_hip_last_error).
void set_error(const std::string& msg);

// Whole-ring drain of every block of cfg; see ssla_hip_drain_n.  Returns an
// SSLA_* status.  Launches on `st`; waits for completion when `sync`.
// phase_ms (host, SSLA_DRAIN_PHASES floats, needs sync) accumulates the
// HIP-event time of the phases in phase_mask (bit k = phase k; 0 = all).
int scan_drain(const HybridS2S3Config* cfg, const HybridInputRec* const* rings,
               const int* ns, HybridS2S3OutputSlot* const* outs,
               float* const* head_outs, hipStream_t st, bool sync,
               float* phase_ms, unsigned long long phase_mask);

// Sizes the whole-ring workspace for calls of up to max_records records over
// cfg's blocks and grid (ssla_hip_drain_reserve).
int drain_reserve(const HybridS2S3Config* cfg, int max_records);

// Zeroes nbytes at p (16-byte aligned device memory) with a kernel on st,
// without waiting.
int zero_async(void* p, size_t nbytes, hipStream_t st);

}  // namespace ssla
