/*
 * ssla_hip.h -- C ABI of libssla_hip.so, the MI355X (gfx950) drain of the
 * SSLA-S s2 + s3 + YOLOX-head path.
 *
 * Conventions for every entry point:
 *   - plain C types and pointers only; no exceptions cross the boundary;
 *   - int-returning calls return SSLA_OK (0) or a negative SSLA_ERR_* code,
 *     and ssla_hip_last_error() then holds a message (per thread);
 *   - "device pointer" means any pointer a gfx950 kernel may dereference:
 *     memory from ssla_hip_malloc_device (HBM) or ssla_hip_malloc_host
 *     (fine-grained, coherent, pinned host memory).
 *
 * Each entry cites the reference interface it replaces.  The reference
 * drives its CUDA kernels through cuda-python; a HIP build cannot be driven
 * that way, so the launches become host C functions with the same argument
 * meaning, plus the allocation helpers the reference took from cuda-python.
 */
#ifndef SSLA_HIP_H
#define SSLA_HIP_H

#include <stddef.h>

#include "ssla_abi.h"

#ifdef __cplusplus
extern "C" {
#endif

#define SSLA_OK          0
#define SSLA_ERR_ARG    (-1)   /* bad argument or shape */
#define SSLA_ERR_HIP    (-2)   /* HIP runtime failure */
#define SSLA_ERR_IO     (-3)   /* file missing / unreadable */
#define SSLA_ERR_FORMAT (-4)   /* weight directory does not follow the schema */
#define SSLA_ERR_STATE  (-5)   /* call out of order */

/* Last error message of the calling thread ("" when none). */
const char* ssla_hip_last_error(void);

/* Writes {sizeof HybridInputRec, sizeof HybridS2S3Config, offsetof preds,
 * sizeof HybridS2S3OutputSlot, sizeof GpuTimingSlot, sizeof HybridStrip,
 * sizeof LayerWeightsS2S3} into out[0..6] (cap >= 7).  Needs no GPU; lets
 * ctypes mirrors check themselves (hybrid_common.py:30-123 asserts). */
int ssla_hip_abi_layout(long long* out, int cap);

/* ---- memory helpers --------------------------------------------------
 * Replace orin/orin/cuda_util.py:39-48 (alloc_managed) and :59-76
 * (alloc_pinned).  Host memory is hipHostMalloc'd fine-grained and
 * coherent so the host may write rings / flags while a kernel polls them. */
int ssla_hip_malloc_device(size_t nbytes, void** out);
int ssla_hip_malloc_host(size_t nbytes, void** out);
int ssla_hip_free_device(void* p);
int ssla_hip_free_host(void* p);
/* Synchronous copy in any direction (hipMemcpyDefault). */
int ssla_hip_memcpy(void* dst, const void* src, size_t nbytes);
int ssla_hip_memset(void* dst, int value, size_t nbytes);
int ssla_hip_device_synchronize(void);
/* Non-blocking HIP streams at default priority for the drain entry points
 * (the reference's harness made them with cuda-python, cuda_util.py). */
int ssla_hip_stream_create(void** out);
int ssla_hip_stream_destroy(void* stream);
int ssla_hip_stream_synchronize(void* stream);

/* ---- weight directory (tools/make_ssla_stub.py schema) ----------------
 * Host-only readers (no GPU): replace vendor/src/weights_loader.cpp:162-252
 * (load_meta) and :255-350 (load_weights_npz).  weights.npz must be stored
 * (uncompressed) '<f4' C-order; ZIP64 entries are accepted.
 * ssla_hip_npz_read copies tensor `key` into out (cap floats) and returns
 * its element count, writing up to 4 dims into shape/ndim when non-NULL. */
long long ssla_hip_npz_read(const char* weights_dir, const char* key,
                            float* out, long long cap,
                            long long* shape, int* ndim);
/* out[0..3] = height, width, num_classes, ssla_tdrop_window */
int ssla_hip_meta_read(const char* weights_dir, int* out);

typedef struct SslaHipModel SslaHipModel;

typedef struct SslaHipModelInfo {
    int height, width;      /* sensor grid of meta.json */
    int num_classes;
    int tdrop_window;
    int H2, W2, H3, W3;     /* s2 / s3 grids (height/4, width/4, /8) */
    int has_head;           /* 2-branch YOLOX head present */
} SslaHipModelInfo;

/* Loads layers/4..7 and head level 0 of a weight directory into HBM in the
 * device layouts of ssla_abi.h (fused q/v/g and gather-o weights, head BN
 * folded).  Replaces multi_block.build_n_block_random_layers(npz=...)
 * (orin/orin/multi_block.py:128-210) and hybrid_common.
 * load_two_layer_head_weights (orin/orin/hybrid_common.py:352-409). */
int  ssla_hip_model_load(const char* weights_dir, SslaHipModel** out);
int  ssla_hip_model_info(const SslaHipModel* m, SslaHipModelInfo* out);
void ssla_hip_model_free(SslaHipModel* m);

/* ---- configuration and per-instance state -----------------------------
 * ssla_hip_config_bind replaces hybrid_common.build_config
 * (hybrid_common.py:214-271) / multi_block.build_n_block_config
 * (multi_block.py:288-340) for weight-directory models: it zeroes *cfg,
 * sets grid dims, tdrop window and head_out_dim, points every block's
 * layers[] and the head at the model, and gives every block the whole grid
 * as its owned strip (one ownership domain per block).  Buffers of
 * hidden/tdrop/preds/version/timing stay NULL until allocated.
 * ssla_hip_state_alloc allocates zeroed hidden state and tdrop counters for
 * block `blk` in HBM (multi_block.py:180-181, alloc_tdrop_n_block :213-226);
 * ssla_hip_preds_alloc allocates zeroed fine-grained host preds/version for
 * the block's owned s3 box (alloc_predictions_n_block :229-252). */
int  ssla_hip_config_bind(const SslaHipModel* m, int n_blocks,
                          HybridS2S3Config* cfg);
int  ssla_hip_state_alloc(HybridS2S3Config* cfg, int blk);
int  ssla_hip_state_reset(const HybridS2S3Config* cfg, int blk);
/* Same, enqueued on `stream` (hipStream_t or NULL) without waiting. */
int  ssla_hip_state_reset_async(const HybridS2S3Config* cfg, int blk,
                                void* stream);
void ssla_hip_state_free(HybridS2S3Config* cfg, int blk);
int  ssla_hip_preds_alloc(HybridS2S3Config* cfg, int blk);
void ssla_hip_preds_free(HybridS2S3Config* cfg, int blk);

/* ---- drain ----------------------------------------------------------
 * Processes ns[b] pre-filled records of rings[b] for every block b <
 * cfg->n_blocks, with the per-block hidden state and tdrop counters of
 * cfg, exactly as if the records were processed one at a time in ring
 * order: L4, L5, tdrop_s2 at the s2 cell, L6, L7, tdrop_s3 at the s3 cell,
 * then (when head weights and preds are set) the YOLOX head for owned
 * pass-3 records, last write per s3 cell winning.
 * Replaces the kernels k_ssla_s2s3_celled_drain_n_multi
 * (orin/kernels/ssla_s2_s3_head_celled.cuh:1108-1255) and
 * k_ssla_s2s3_celled_drain_n (:914-1095).
 *   cfg        host pointer; its pointer members are device pointers
 *   rings[b]   device pointer to ns[b] records (x, y in s2 coordinates)
 *   outs[b]    NULL or device pointer to ns[b] output slots: pass2/pass3 as
 *              1/0 for owned records and -1 for halo records; s3_feat holds
 *              the L7 output for pass-3 records and zeros otherwise
 *   batch_clks NULL: the whole ring is drained at once (fastest).  Non-NULL:
 *              records are taken in in-kernel batches of 8, one workgroup
 *              per block, and batch_clks[b] (NULL or device memory, 2 u64
 *              per batch) receives (t_pop, t_done) wall-clock ticks of each
 *              batch (ssla_hip_wall_clock_khz gives the rate).
 * Records outside the s2 grid leave all state untouched and report
 * pass2 = pass3 = -2.  Synchronous.  Weights must be shared by all blocks. */
int ssla_hip_drain_n(const HybridS2S3Config* cfg,
                     const HybridInputRec* const* rings, const int* ns,
                     HybridS2S3OutputSlot* const* outs,
                     unsigned long long* const* batch_clks);

/* Two-ring form of the same call (the reference's P1 entry signature). */
int ssla_hip_drain_n2(const HybridS2S3Config* cfg,
                      const HybridInputRec* ring0, const HybridInputRec* ring1,
                      int n0, int n1,
                      HybridS2S3OutputSlot* out0, HybridS2S3OutputSlot* out1);

#define SSLA_DRAIN_PHASES 23
/* Phase order of SslaHipDrainOpts.phase_ms (one kernel launch each, except
 * 0, 21): 0 ordering (decode, sorts, tdrop decisions, chunk tables); per
 * layer a projection of v, g, the recurrence in three slots, then the
 * contraction (q, q*h, goW, residual, LayerNorm): L4 1-5, L5 6-10, L6
 * 11-15, L7 16-20; 21 head and prediction grid, 22 output slots.  The
 * recurrence of every layer is one launch, in the third of its slots; the
 * first holds L4's wait for its ticket order (built beside L4's
 * projection) and is empty for L5-L7, and the second is empty. */

#define SSLA_BATCH_PHASES 32
/* Slots of the in-kernel batch profile (batch-mode and live drains), summed
 * over blocks: microseconds of 0 batch load, 1 tdrop s2, 2 s2 pairs,
 * 3-6 L4 (projection, recurrence, contraction, LayerNorm), 7-10 L5,
 * 11 pool + tdrop s3, 12 s3 pairs, 13-16 L6, 17-20 L7, 21 head hidden,
 * 22 head outputs, 23 prediction grid, 24 outputs / publish; then counts:
 * 25 batches, 26 records; then, for group drains only, 27-30 the exchange
 * waits of L4-L7 (slots 5, 9, 15, 19 then hold the contraction up to the
 * member's own partial sums); 31 unused. */

typedef struct SslaHipDrainOpts {
    void*         stream;      /* hipStream_t; NULL = default stream */
    int           sync;        /* nonzero: wait for completion */
    int           batch;       /* 0: whole-ring drain; 1..32: in-kernel
                                  batches of this many records */
    float* const* head_outs;   /* NULL or [n_blocks] device pointers to
                                  (ns[b], 7) raw head outputs, written for
                                  owned pass-3 records, zeros otherwise */
    float*        phase_ms;    /* NULL or host float[SSLA_DRAIN_PHASES]:
                                  adds the GPU time of each phase, measured
                                  with HIP events on `stream`.  With sync
                                  = 0 the times are added when a later
                                  whole-ring call with sync set returns
                                  (keep the array alive until then), so
                                  timed calls can be queued back to back */
    double*       batch_phase_us; /* NULL or host double[SSLA_BATCH_PHASES]:
                                  batch mode only (needs sync); adds the
                                  in-kernel wall-clock profile */
    int           group;       /* batch mode: 0 or 1 = one workgroup per
                                  block; 3..6 = that many workgroups per
                                  block, each owning 16-channel slices of
                                  every layer (see ssla_hip_persistent_start);
                                  runs synchronously */
    unsigned long long phase_mask; /* with phase_ms: time only the phases
                                  whose bit is set (bit k = phase k); 0 =
                                  all.  Each timed phase boundary costs a
                                  few microseconds of queue time */
} SslaHipDrainOpts;

int ssla_hip_drain_n_ex(const HybridS2S3Config* cfg,
                        const HybridInputRec* const* rings, const int* ns,
                        HybridS2S3OutputSlot* const* outs,
                        const SslaHipDrainOpts* opts);

/* The batch-mode drain (ssla_hip_drain_n_ex with opts->batch = batch) for
 * callers that cannot allocate device memory: code under HIP graph
 * capture, tight serving loops, harnesses that forbid hipMalloc.  No
 * counterpart in the reference.  It makes no hipMalloc / hipFree /
 * allocating call: the memory its kernel needs beyond the caller's inputs
 * and outputs (each block's pair rows, the fragment-order weight copy, the
 * block table; 7.8 MiB) is a static array of the library, one per
 * device, held until the process ends.  Limits: cfg->n_blocks <= 16,
 * 1 <= batch <= 32 (SSLA_ERR_ARG beyond).  All calls on one device share
 * that array: calls that overlap on one device (other streams or threads)
 * race and must be ordered by the caller.  The first call on a device
 * looks up the array's device address; make it before any graph capture.
 * head_outs as in SslaHipDrainOpts.  Enqueued on `stream` (hipStream_t or
 * NULL); waits for completion when sync is nonzero.  Results equal
 * ssla_hip_drain_n_ex's with the same batch. */
int ssla_hip_drain_batch_noalloc(const HybridS2S3Config* cfg,
                                 const HybridInputRec* const* rings, const int* ns,
                                 HybridS2S3OutputSlot* const* outs,
                                 float* const* head_outs, int batch,
                                 void* stream, int sync);

/* The whole-ring drain keeps one workspace per process (device memory
 * sized for the largest call so far; about 9 KB per record).  A call with
 * more records than it holds regrows it, which waits for the previous
 * drain call to finish and frees and allocates device memory.  Call this
 * once up front -- in particular before ssla_hip_persistent_start, while no
 * other kernel of the caller's runs -- to size it for calls of up to
 * max_records records in total over cfg's blocks and grid.  No counterpart
 * in the reference (its drain kernel works in shared memory only).
 *
 * Every drain call rebuilds its fragment-order copy of the layer weights
 * (reordered for the matrix cores) from cfg's weight pointers, so weights
 * rewritten in place, by any means, between calls are the ones used. */
int ssla_hip_drain_reserve(const HybridS2S3Config* cfg, int max_records);

/* Ticks per millisecond of the constant-rate GPU clock used by batch_clks
 * and GpuTimingSlot (s_memrealtime). */
int ssla_hip_wall_clock_khz(int* out);

/* Timing ring of block blk: `capacity` (power of two) GpuTimingSlot in HBM,
 * timing_mask = capacity - 1, and kernel_start_clk / kernel_end_clk anchors
 * in fine-grained host memory (hybrid_common.py:274-310).  All zeroed.
 * The anchors are words 0 and 1 of four: while the live kernel runs, a
 * host that writes a new value into word 2 (kernel_start_clk[blk][2]) gets,
 * within a poll, word 3 = (GPU wall clock << 8) | (that value & 0xff),
 * read after the kernel saw the new value -- a clock reading the host can
 * bracket between two of its own. */
int  ssla_hip_timing_alloc(HybridS2S3Config* cfg, int blk, unsigned int capacity);
void ssla_hip_timing_free(HybridS2S3Config* cfg, int blk);

/* ---- persistent live drain --------------------------------------------
 * Replaces k_ssla_s2s3_celled_persistent_multi
 * (orin/kernels/ssla_s2_s3_head_celled.cuh:1547-1784) and its launch in
 * orin/hybrid_runner_multi.py:514-523.  One workgroup per block polls
 * rings[b] (capacity ring_mask + 1, a power of two, in fine-grained host
 * memory): slot t is ready when its seq_done == t + 1.  Ready records are
 * processed in ring order in batches of up to opts->max_batch; the head
 * writes preds / version (last write per cell wins); GpuTimingSlot entries
 * are written when cfg->timing[b] is set; *tails[b] and *events_done[b]
 * advance (system-scope release) after each batch.  spin_ns is the idle
 * sleep between polls.  The kernel returns when *stop_flag becomes
 * nonzero, when a producer laps the ring (status 2), or after
 * opts->idle_timeout_ms without a ready record (status 3).
 * With opts->group = G in 3..6, each block is drained by G workgroups
 * instead of one: member k owns the 16-channel slices k, k + G, ... of
 * every layer (projection, recurrence, its part of the contraction), and
 * the members exchange partial pre-LayerNorm sums through device memory
 * once per layer.  Results are those of one workgroup up to fp32 summation
 * order; each block's weights stream through G compute units.  All
 * n_blocks x G workgroups must fit on the device at once (SSLA_ERR_ARG
 * otherwise); a member whose wait for another runs out (2 s inside a
 * batch) ends the kernel with status 4.  With opts->stages = 2 each block
 * has two such groups in a pipeline (n_blocks x G x 2 workgroups): the
 * first loads a batch and runs tdrop_s2, L4 and L5, then hands the batch
 * (through device memory) to the second, which runs tdrop_s3, L6, L7, the
 * head and the predictions while the first takes the next batch.  The
 * ring tail, events_done and the timing slots advance once the second
 * group has finished a batch.
 * The kernel runs on its own non-blocking stream; do not call
 * ssla_hip_device_synchronize while it runs. */
typedef struct SslaHipLive SslaHipLive;

typedef struct SslaHipLiveOpts {
    int          max_batch;        /* 1..32; default 32 */
    unsigned int idle_timeout_ms;  /* default 30000 */
    double*      phase_us;         /* NULL or host double[SSLA_BATCH_PHASES]:
                                      filled (added to) by persistent_wait
                                      (member 0's profile with groups) */
    int          group;            /* 0 or 1: one workgroup per block;
                                      3..6: workgroups per block */
    int          stages;           /* 0 or 1: each group runs every layer of
                                      a batch; 2 (with group 3..6): a second
                                      group of as many workgroups runs L6, L7
                                      and the head of batch k while the first
                                      runs L4 and L5 of batch k + 1 */
} SslaHipLiveOpts;

int ssla_hip_persistent_start(const HybridS2S3Config* cfg,
                              HybridInputRec* const* rings,
                              unsigned long long ring_mask,
                              unsigned long long* const* tails,
                              int* stop_flag,
                              unsigned long long* const* events_done,
                              unsigned int spin_ns,
                              const SslaHipLiveOpts* opts,
                              SslaHipLive** out);

/* Two-ring form of ssla_hip_persistent_start: the signature of the
 * reference's legacy live kernel k_ssla_s2s3_celled_persistent(cfg, ring0,
 * ring1, ring_mask, tail0, tail1, stop_flag, events_done0, events_done1,
 * spin_ns) (orin/kernels/ssla_s2_s3_head_celled.cuh:1271-1281, launched
 * with a grid of 2 by orin/hybrid_runner.py:334-393).  cfg->n_blocks must be
 * 2 (block b drains ring b).  As in that kernel, each block is one
 * workgroup taking records in batches of up to 8; the idle timeout is the
 * default 30 s.  Stop it with *stop_flag and ssla_hip_persistent_wait. */
int ssla_hip_persistent_start2(const HybridS2S3Config* cfg,
                               HybridInputRec* ring0, HybridInputRec* ring1,
                               unsigned long long ring_mask,
                               unsigned long long* tail0, unsigned long long* tail1,
                               int* stop_flag,
                               unsigned long long* events_done0,
                               unsigned long long* events_done1,
                               unsigned int spin_ns, SslaHipLive** out);

/* Waits (up to timeout_ms, < 0 = forever) for the kernel to return after
 * the caller set *stop_flag, then frees the session.  *status: 0 stopped
 * by the flag, 2 ring overrun, 3 idle timeout, 4 a group member's wait
 * ran out.  Returns SSLA_ERR_STATE if
 * the kernel is still running at the timeout (the session stays valid). */
int ssla_hip_persistent_wait(SslaHipLive* h, int timeout_ms, int* status);

/* ---- prediction grid: host-side consumer ------------------------------
 * Host code only: these calls make no HIP call and need no GPU.
 *
 * Each owned s3 cell of block b holds SSLA_HEAD_OUT raw head floats
 * [tx, ty, log_w, log_h, obj, cls0, cls1] in cfg->preds[b] and a version
 * word in cfg->version[b] that counts the pass-3 records the head has
 * written to the cell (0 = never written; the reference adds 1 per write,
 * orin/kernels/ssla_s2_s3_head_celled.cuh:900,1498,1750).  While the device
 * writes a cell it holds SSLA_PRED_BUSY in the word, and the values are
 * stored between two system-scope fences, so a reader that sees the same
 * word (busy bit clear) before and after copying a cell has a whole cell.
 * Counts wrap at 2^31. */
#define SSLA_PRED_BUSY 0x80000000u

/* Copies n_cells cells (cols floats + version each) torn-free: a cell is
 * read up to max_tries times (>= 1), about 1 us apart.  Returns the number of cells that
 * stayed busy or kept changing (their version_out has SSLA_PRED_BUSY set
 * and preds_out holds the last copy), or a negative SSLA_ERR_*.  Replaces
 * the direct reads of the pinned views (orin/hybrid_runner_multi.py:648-656,
 * orin/orin/multi_block.py:229-253). */
int ssla_hip_preds_snapshot(const float* preds, const unsigned* version, int n_cells, int cols,
                            float* preds_out, unsigned* version_out, int max_tries);

/* decode_yolox_cell's transform (vendor/openeva/heads/async_yolox.h:189-196)
 * on n_cells raw rows of cols (>= 5) floats: cell i sits at grid
 * (gx0 + i % grid_w, gy0 + i / grid_w) and becomes
 * [(tx+gx)*stride_w, (ty+gy)*stride_h, exp(log_w)*stride_w,
 *  exp(log_h)*stride_h, obj, cls...] (logits stay raw). */
int ssla_hip_decode_cells(const float* raw, int n_cells, int cols, int grid_w, int gx0, int gy0,
                          int stride_w, int stride_h, float* out);

/* The whole s3 grid as the CPU pipeline's DetectionOutput holds it
 * (src/ssla_kernels.cpp:934-966): out is (H3*W3, SSLA_HEAD_OUT), row
 * gy*W3 + gx, decoded as ssla_hip_decode_cells.  Cells of every block's
 * owned box with version > 0 come from a torn-free read of cfg->preds[b];
 * every other cell holds zero_row (the head's raw output for an all-zero
 * feature, ssla_hip_model_head_row), as the CPU pipeline prepopulates them
 * (src/ssla_kernels.cpp:966-987).  Returns the number of torn cells (left at
 * zero_row) or a negative SSLA_ERR_*. */
int ssla_hip_grid_decode(const HybridS2S3Config* cfg, const float* zero_row, int stride_w,
                         int stride_h, int max_tries, float* out);

/* The live demo's box collection for one block
 * (orin/hybrid_runner_multi.py:163-207), in fp32: over the s3w*s3h raw rows
 * (row-major over the block's owned s3 box at (s3x_lo, s3y_lo)),
 * obj = sigmoid(raw[4]); cells with obj >= obj_thresh give the box
 *   cx = s3x*8 + 4 + tx*8, cy = s3y*8 + 4 + ty*8,
 *   w = clip(exp(log_w)*8, 2, W_full), h = clip(exp(log_h)*8, 2, H_full),
 *   [(cx - w/2)*scale, (cy - h/2)*scale, w*scale, h*scale]
 * and score obj, in cell order.  *max_seen is raised to the largest obj
 * seen (the caller initialises it).  Returns the number of cells kept
 * (boxes past max_boxes are counted, not written). */
int ssla_hip_collect_boxes(const float* raw, int s3w, int s3h, int s3x_lo, int s3y_lo, float scale,
                           float obj_thresh, int W_full, int H_full, float* boxes_xywh,
                           float* scores, int max_boxes, float* max_seen);

/* Host-side YOLOX head on one 96-channel s3 feature: out[0..6] = raw
 * [reg4, obj, cls2] with BatchNorm folded as the device head has it.  With
 * an all-zero feature this is the row the CPU pipeline prepopulates
 * (src/ssla_kernels.cpp:966-987).  SSLA_ERR_STATE if the model has no head. */
int ssla_hip_model_head_row(const SslaHipModel* m, const float* feat, float* out);
/* The same from a weight directory's head (needs no GPU). */
int ssla_hip_head_row(const char* weights_dir, const float* feat, float* out);

/* ---- OEVA head-grid dumps (include/oracle.h:10-18) --------------------
 * Little-endian file: uint32 magic 0x4F455641 ("OEVA"), uint32 version 1,
 * uint32 num_anchors, uint32 cols, uint32 num_checkpoints, then per
 * checkpoint uint64 event_idx and float[num_anchors * cols]. */
#define SSLA_OEVA_MAGIC   0x4F455641u
#define SSLA_OEVA_VERSION 1u

/* Writes n_cp checkpoints (preds: n_cp * num_anchors * cols floats) in one
 * go; OracleRecorder::save (include/oracle.h:57-77). */
int ssla_hip_oeva_write(const char* path, unsigned num_anchors, unsigned cols, unsigned n_cp,
                        const unsigned long long* event_idx, const float* preds);
/* out3 = {num_anchors, cols, num_checkpoints}.  SSLA_ERR_IO when the file
 * cannot be opened, SSLA_ERR_FORMAT on a short header or a bad
 * magic/version (include/oracle.h:103-116). */
int ssla_hip_oeva_header(const char* path, unsigned* out3);
/* Reads every checkpoint (cap_cp >= num_checkpoints); a truncated body
 * leaves the checkpoints past the short read zero-filled, as
 * include/oracle.h:117-121 does. */
int ssla_hip_oeva_read(const char* path, unsigned long long* event_idx, float* preds,
                       unsigned cap_cp);

typedef struct SslaHipOevaDiff {
    int    ok;                /* shapes, checkpoint counts and indices agree */
    size_t n_cp;
    double max_abs_delta;
    size_t n_mismatched_cp;   /* checkpoints with any |delta| > tol_abs */
} SslaHipOevaDiff;

/* deploy::diff_dumps (include/oracle.h:90-150): ok = 0 on a shape or count
 * mismatch (nothing compared) or at the first checkpoint whose event_idx
 * differs (comparison stops there); NaN deltas are passed over. */
int ssla_hip_oeva_diff(const char* path_a, const char* path_b, double tol_abs,
                       SslaHipOevaDiff* out);

#ifdef __cplusplus
}
#endif

#endif /* SSLA_HIP_H */
