/*
 * stage01_capi.h -- C ABI of libstage01_capi.so: SSLA-S stages 0 + 1 on host
 * CPU shards without a GPU (the CPU reference path of the producer).
 *
 * Signatures and stats slots are those of src/lib_stage01_capi.cpp:156-343:
 * N shard threads with halo routing; the owner runs stage 0, tdrop_0, stage 1,
 * tdrop_1; halo shards run stage 0 for state.  Latency samples are taken per
 * owner event from submission to shard completion.
 */
#ifndef STAGE01_CAPI_H
#define STAGE01_CAPI_H

#ifdef __cplusplus
extern "C" {
#endif

typedef struct S0Handle S0Handle;

/* lib_stage01_capi.cpp:167-209; NULL on failure */
S0Handle* s0_init(const char* weights_dir, int n_shards, int halo, int base_core,
                  int sample_cap);
/* lib_stage01_capi.cpp:214-251: events [t_us, x, y, p] x n */
int  s0_submit_batch(S0Handle* h, const float* events_packed, int n);
/* lib_stage01_capi.cpp:272-316: 16 slots, the first 14 of s01g_snapshot_stats */
void s0_snapshot_stats(S0Handle* h, double* out);
void s0_reset_stats(S0Handle* h);
void s0_shutdown(S0Handle* h);

#ifdef __cplusplus
}
#endif

#endif /* STAGE01_CAPI_H */
