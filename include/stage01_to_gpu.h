/*
 * stage01_to_gpu.h -- C ABI of libstage01_to_gpu.so: SSLA-S stages 0 + 1 on
 * host CPU shards feeding the drain's rings.
 *
 * Signatures and semantics are those of the reference producer
 * (src/lib_stage01_to_gpu.cpp:341-755; ctypes declarations
 * orin/orin/hybrid_common.py:474-524), so its Python driver binds unchanged:
 *   - N shard threads (pinned to base_core + k when base_core >= 0), each with
 *     a private stage-0/1 state; events are routed to x-strips of width
 *     ceil(W / N) with `halo` extra columns each side; the owner shard runs
 *     stage 0 and, if tdrop_0 passes, stage 1; halo shards run stage 0 state
 *     only (tdrop checked first so dropped work runs state-only,
 *     lib_stage01_to_gpu.cpp:230-311);
 *   - a record that passes tdrop_1 is published to every attached ring whose
 *     s2 box contains its s2 (x, y): slot = fetch_add(head), fields, t_push_ns,
 *     then a release store of seq_done = slot + 1 (no back-pressure);
 *   - s01g_init* return NULL on failure (message on stderr); every other
 *     call is a no-op on a NULL handle; submit_batch needs exactly one
 *     submitting thread.
 */
#ifndef STAGE01_TO_GPU_H
#define STAGE01_TO_GPU_H

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

typedef struct S01gHandle S01gHandle;

/* lib_stage01_to_gpu.cpp:348-352 (shard ring capacity 65536) */
S01gHandle* s01g_init(const char* weights_dir, int n_shards, int halo,
                      int base_core, int sample_cap);
/* lib_stage01_to_gpu.cpp:354-421; shard_ring_cap is rounded up to 2^k */
S01gHandle* s01g_init_full(const char* weights_dir, int n_shards, int halo,
                           int base_core, int sample_cap,
                           unsigned int shard_ring_cap);
/* lib_stage01_to_gpu.cpp:437-466: two rings, x ranges [lo, hi), full y */
void s01g_attach_gpu_rings(S01gHandle* h,
                           void* ring_buf_0, void* ring_head_0,
                           void* ring_buf_1, void* ring_head_1,
                           unsigned long long ring_mask, int W2, int H2,
                           int proc_lo_0, int proc_hi_0,
                           int proc_lo_1, int proc_hi_1);
/* lib_stage01_to_gpu.cpp:477-502: n <= 16 rings with s2 boxes */
void s01g_attach_gpu_rings_multi(S01gHandle* h, int n_blocks,
                                 void* const* ring_bufs, void* const* ring_heads,
                                 unsigned long long ring_mask, int W2, int H2,
                                 const int* proc_x_los, const int* proc_x_his,
                                 const int* proc_y_los, const int* proc_y_his);
/* lib_stage01_to_gpu.cpp:504-538: events [t_us, x, y, p] x n; returns the
 * number accepted (events outside the sensor are counted as oob) */
int  s01g_submit_batch(S01gHandle* h, const float* events_packed, int n);
/* No counterpart in the reference (its rings overwrite unread slots and the
 * drain reports the overrun): optional back-pressure.  tails[b] (n entries,
 * n <= the attached ring count; NULL or n = 0 turns it off) is ring b's
 * consumer tail, e.g. the drain's tails in fine-grained memory.  A
 * publisher that claims slot s waits until s - tail <= mask, at most
 * timeout_ns, then writes anyway.  Call after attaching the rings (an
 * attach turns it off). */
void s01g_set_ring_tails(S01gHandle* h, int n, const unsigned long long* const* tails,
                         unsigned long long timeout_ns);
/* lib_stage01_to_gpu.cpp:540-611: 32 slots
 *   0 owner events, 1 halo events, 2 pass stage 0, 3 oob, 4 seconds since
 *   init/reset, 5 shard-ring occupancy, 6..11 owner latency p50 p90 p99
 *   p99.9 max mean (us, arrival -> shard done), 12 latency samples,
 *   13 pass stage 1, 14/15 records pushed to ring 0/1, 16..21 segment time
 *   sums (ns: preprocess, s0, tdrop0, s1, tdrop1, push), 22..27 segment
 *   counts, 28 back-pressure waits, 29 their total ns, 30 waits that
 *   timed out (the slot was overwritten), 31 reserved */
void s01g_snapshot_stats(S01gHandle* h, double* out);
void s01g_reset_stats(S01gHandle* h);
void s01g_shutdown(S01gHandle* h);
/* lib_stage01_to_gpu.cpp:624-706: paced synthetic source, uniform over the
 * sensor, polarity one random bit */
void s01g_start_synthetic(S01gHandle* h, double rate_mev, int pin_core,
                          unsigned long long seed);
void s01g_stop_synthetic(S01gHandle* h);
unsigned long long s01g_synthetic_n_pushed(S01gHandle* h);

/* No counterpart in the reference: the paced synthetic source with moving
 * Gaussian blobs (sigma_px, 0.5-2 px/ms, reflecting) plus bg_frac uniform
 * background, polarity +-1 -- the live-pipeline benchmark distribution. */
void s01g_start_synthetic_blobs(S01gHandle* h, double rate_mev, int pin_core,
                                unsigned long long seed, int n_blobs,
                                double sigma_px, double bg_frac);

/* No counterpart in the reference: replays pre-built ring records (post
 * stage 1, one array per ring, owned by the caller until stop) into n rings
 * at a paced aggregate rate, round-robin across rings, with the same publish
 * protocol and t_emit_ns = t_push_ns = publish time -- the source of the
 * multi-stream live benchmark.  NULL on bad arguments. */
typedef struct S01gReplay S01gReplay;
S01gReplay* s01g_replay_start(int n_rings, void* const* ring_bufs,
                              void* const* ring_heads, unsigned long long ring_mask,
                              const void* const* records, const int* counts,
                              double rate_rec_s, int pin_core);
/* Same, paced by the records' own times: the rings are merged in record-time
 * order (t in us) and a record goes out (t - t_first) / speed us after the
 * start, so copies of one record in several rings go out together. */
S01gReplay* s01g_replay_start_timed(int n_rings, void* const* ring_bufs,
                                    void* const* ring_heads, unsigned long long ring_mask,
                                    const void* const* records, const int* counts,
                                    double speed, int pin_core);
int  s01g_replay_done(S01gReplay* r);                 /* 1 when all are published */
unsigned long long s01g_replay_published(S01gReplay* r);
void s01g_replay_stop(S01gReplay* r);                 /* joins and frees */

#ifdef __cplusplus
}
#endif

#endif /* STAGE01_TO_GPU_H */
