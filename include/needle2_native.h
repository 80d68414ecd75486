/*
 * libneedle2_native.so - gfx950 (MI355X) implementation of OpenNeedle's
 * quantized-matmul hot path behind the reference's C ABI.
 *
 * Section 1 is the reference's ctypes boundary; each declaration cites the
 * reference definition it replaces. Section 2 lists additive exports (no
 * counterpart in the reference). All entry points are synchronous unless they
 * take a stream argument; pointers in section 1 are host pointers.
 *
 * Conventions (the reference's, needle2/native.py:165-279, cq.cpp:342-371):
 *  - *_create returns NULL on failure; the reason is in needle2_gpu_error().
 *  - void entry points have no error channel in the reference; on failure
 *    this library fills the output with NaN and sets needle2_gpu_error().
 *  - int entry points return 0 on success and -1 on failure.
 *  - Calls on one handle must be serialized (needle2/native.py:313);
 *    different handles may be used concurrently (each owns a HIP stream).
 */
#ifndef NEEDLE2_NATIVE_H
#define NEEDLE2_NATIVE_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* ======================= 1. Reference ABI (drop-in) ===================== */

/* needle2/csrc/cq.cpp:343-349 */
const char *needle2_native_features(void);

/* needle2/csrc/cq.cpp:350-352. Uploads packed codes ([out][padded*bits/8],
 * LSB-first), fp16 norms ([out][padded/group]) and the codebook (16/8/4/3
 * floats) to device memory; the host buffers are not retained.
 * bits: 2, 3, 4 or 5 (ternary crumbs); group: power of two >= 8. Returns NULL
 * (reason in needle2_gpu_error) for a codebook that is not finite and strictly
 * increasing, a norm that is not finite or is negative, or a ternary crumb 2:
 * the inputs the reference's loader refuses (needle2/native.py:190-202). */
void *needle2_cq_create(const uint8_t *packed, const uint16_t *norms, int out, int in, int bits, int group,
                        const float *codebook);
/* needle2/csrc/cq.cpp:353 */
void needle2_cq_destroy(void *handle);
/* needle2/csrc/cq.cpp:354-356. x: [batch][in], y: [batch][out]. threads is ignored.
 * Bit-identical to the reference's portable (non-NEON) build for every bit width. */
void needle2_cq_linear(void *handle, const float *x, float *y, int batch, int threads);
/* needle2/csrc/cq.cpp:357-359. Every mode runs the GPU GEMV (same tolerance contract). */
void needle2_cq_linear_lookup(void *handle, const float *x, float *y, int batch, int threads, int mode);
/* needle2/csrc/cq.cpp:287-292, 360-366. One x for count matrices; ys[i] receives matrix i's output.
 * Matrices of one input length and group share one copy and one transform of x (one GEMV launch per
 * storage geometry); otherwise each runs alone. Every mode runs the GPU GEMV. */
void needle2_cq_linear_many(void *const *handles, int count, const float *x, float *const *ys, int threads,
                            int mode);
/* needle2/csrc/cq.cpp:367-370. y: [count][in] = FWHT(cb[code]*norm) of each row. */
void needle2_cq_rows(void *handle, const int64_t *ids, float *y, int count);

/* needle2/csrc/sdot.cpp:350. Always 1: the int8 path runs on the GPU. */
int needle2_sdot_supported(void);
/* needle2/csrc/sdot.cpp:351-354. NULL unless bits is 2 or 4 and 64 <= group <= 131072. */
void *needle2_sdot_create(const uint8_t *packed, const uint16_t *norms, int out, int in, int bits, int group,
                          const float *codebook);
/* needle2/csrc/sdot.cpp:355 */
void needle2_sdot_destroy(void *handle);
/* needle2/csrc/sdot.cpp:356-359. Bit-exact with the reference's int8 arithmetic. */
void needle2_sdot_linear(void *handle, const float *x, float *y, int batch, int threads);

/* needle2/csrc/engine.cpp:1499-1548: the single-sequence engine, on the GPU.
 * config is the reference's EngineConfig (engine.cpp:15-19), tensors its
 * TensorDesc table (engine.cpp:14) with CQ entries pointing at this library's
 * CQ handles (borrowed) and dense entries at host fp32 data (copied at
 * creation); dfa is the reference's DFAStateDesc (engine.cpp:326-338).
 * threads and set_lookup's mode are ignored (one GPU path per matrix).
 * set_sdot switches the 2/4-bit CQ matrices of groups 64..131072 to the int8
 * path on any host (the reference needs an ARM64 CPU with DotProd); prefill
 * runs chunks of 32 tokens (or the window) through the same per-token
 * arithmetic. For a window model the device KV ring holds chunk - 1 slots more
 * than the reference's (window + prefix), and kv_storage_bytes counts them.
 * Failures return NULL / -1 with the message in needle2_engine_error(). */
const char *needle2_engine_error(void);
void *needle2_engine_create(const void *config, const void *tensors, int count, int threads, int activation_bits);
void needle2_engine_destroy(void *engine);
void needle2_engine_set_lookup(void *engine, int mode);
int needle2_engine_set_sdot(void *engine);
void needle2_engine_reset(void *engine, int prefix);
int needle2_engine_cache_prefix(void *engine);
int needle2_engine_reset_to_prefix(void *engine);
int needle2_engine_step(void *engine, int token, float *logits, float *hidden);
int needle2_engine_prefill(void *engine, const int *tokens, int num_tokens, int last_only, float *logits,
                           float *hidden);
int needle2_engine_step_candidates(void *engine, int token, const int *candidates, int num_candidates,
                                   float *candidate_logits, float *hidden);
int needle2_engine_project_candidates(void *engine, const int *candidates, int num_candidates,
                                      float *candidate_logits);
int needle2_engine_decode_loop(void *engine, int first_token, int max_new_tokens, const void *dfa,
                               int *output_tokens, int *out_generated_count);
int needle2_engine_import(void *engine, int pos, int prefix, const int *ids, const int *positions, int count,
                          const float *k, const float *v);
int needle2_engine_set_int8_kv(void *engine, int enable);
size_t needle2_engine_kv_storage_bytes(void *engine);

/* ======================= 2. Additive gfx950 exports ===================== */

/* Thread-local message of the last failed call on this thread ("" after a
 * successful one). */
const char *needle2_gpu_error(void);

/* needle2_sdot_create with groups down to 8 (CQ4) or 16 (CQ2). Same
 * arithmetic; the reference cannot run these groups (its ABI rejects them). */
void *needle2_gpu_sdot_create(const uint8_t *packed, const uint16_t *norms, int out, int in, int bits, int group,
                              const float *codebook);

/* needle2_cq_create / needle2_gpu_sdot_create from device-resident packed
 * codes and norms in the reference's layouts (needle2/native.py:189-197 passes
 * host pointers): the relayout kernels are enqueued on `stream` and the call
 * returns without waiting, so a model's matrices can be built from one bulk
 * copy of its archive. The inputs must stay valid, and the handle unused on
 * other streams, until `stream` has run them. */
void *needle2_gpu_cq_create_device(const uint8_t *d_packed, const uint16_t *d_norms, int out, int in, int bits,
                                   int group, const float *codebook, void *stream);
void *needle2_gpu_sdot_create_device(const uint8_t *d_packed, const uint16_t *d_norms, int out, int in, int bits,
                                     int group, const float *codebook, void *stream);

/* Device-resident variants: d_x [batch][in] and d_y [batch][out] are device
 * pointers; work is enqueued on `stream` (hipStream_t, NULL = the handle's
 * stream) and the call returns without waiting. */
int needle2_gpu_cq_linear_device(void *handle, const float *d_x, float *d_y, int batch, void *stream);
int needle2_gpu_sdot_linear_device(void *sdot_handle, const float *d_x, float *d_y, int batch, void *stream);

/* The int32 group dots of the int8 product (the accumulators of SdotCQ::dot_group,
 * needle2/csrc/sdot.cpp:108-137): d_dots[b][row][g] = sum over group g of
 * centroid(code) * q(x_b), from the kernels needle2_gpu_sdot_linear_device runs
 * for this batch on a large matrix (batch 1: the row kernel; 2 .. 8: the
 * 4x4x4 batch-tile MFMA kernel; 9 or more: the 16x16x32 batch-tile MFMA
 * kernel where a group holds whole code chunks, else the 4x4x4 one). Groups
 * of 8 .. 256. */
int needle2_gpu_sdot_dots_device(void *sdot_handle, const float *d_x, int32_t *d_dots, int batch, void *stream);

/* No counterpart in the reference: needle2_gpu_sdot_linear_device for callers
 * that cannot allocate (work captured into a HIP graph, serving loops that
 * forbid allocation). The same kernels, with the quantized activations and
 * scales in a static 4 MiB device array the library holds per GPU until the
 * process ends; nothing is allocated. stream NULL: the null stream. Returns -1
 * when batch * (P + 8 * groups) bytes exceed 4 MiB, where P is the input
 * padded to whole groups and then rounded up to a multiple of 256 (each of the
 * two parts rounded up to 256 bytes), or for groups above 16384. All calls on one GPU share the
 * array: calls that overlap in time on one GPU race. */
int needle2_gpu_sdot_linear_device_noalloc(void *sdot_handle, const float *d_x, float *d_y, int batch, void *stream);

/* Candidate rows (replaces the CQ and SDOT branches of
 * Engine::project_candidates, needle2/csrc/engine.cpp:1302-1349, behind
 * needle2_engine_project_candidates, engine.cpp:1530): y[i] = row ids[i] of
 * the product of one input vector x[in], bit-identical to that row of
 * needle2_cq_linear / needle2_sdot_linear; order and duplicates are kept.
 * Host-pointer forms return -1 with "candidates must be nonempty" (count < 1)
 * or "candidate outside vocabulary" (an id outside [0, out)), as the
 * reference does. Device forms: d_ids int32 on the device, an id outside
 * [0, out) yields NaN. */
int needle2_gpu_cq_candidates(void *handle, const float *x, const int32_t *ids, int count, float *y);
int needle2_gpu_cq_candidates_device(void *handle, const float *d_x, const int32_t *d_ids, int count, float *d_y,
                                     void *stream);
int needle2_gpu_sdot_candidates(void *sdot_handle, const float *x, const int32_t *ids, int count, float *y);
int needle2_gpu_sdot_candidates_device(void *sdot_handle, const float *d_x, const int32_t *d_ids, int count,
                                       float *d_y, void *stream);

/* Prefill GEMM (replaces the per-token-pair CQ loops of Engine::linear_batch /
 * attention_projections_batch, needle2/csrc/engine.cpp:607-750, for prompt
 * chunks): d_y[m][out] = FWHT-domain product of d_x[m][in] (device fp32) on
 * fp16 MFMA with fp32 accumulation; activations and cb*norm weights are
 * rounded to fp16 (agreement with needle2_cq_linear about 1e-3 normwise).
 * Every storage width: 2-bit and ternary codes are widened to 4-bit codes in
 * device memory on the first call (kept with the handle). The _timed form (a timing aid, no reference
 * counterpart) records two events around `repeat` back-to-back launches of
 * the GEMM kernel after one activation transform. */
int needle2_gpu_cq_gemm_device(void *cq_handle, const float *d_x, float *d_y, int m, void *stream);
int needle2_gpu_cq_gemm_timed(void *cq_handle, const float *d_x, float *d_y, int m, void *stream, void *gemm_start,
                              void *gemm_stop, int repeat);

/* Plans: `count` handles of one geometry (in, bits, group, codebook), matrix
 * i reading d_x[i] ([batch][in]) and writing d_y[i] ([batch][out_i]); one
 * GEMV launch covers all of them. */
void *needle2_gpu_cq_plan_create(void *const *handles, int count, const float *const *d_x, float *const *d_y,
                                 int batch);
void *needle2_gpu_sdot_plan_create(void *const *sdot_handles, int count, const float *const *d_x,
                                   float *const *d_y, int batch);
int needle2_gpu_plan_run(void *plan, void *stream);
/* needle2_gpu_plan_run, recording gemv_start/gemv_stop (hipEvent_t) on the
 * stream immediately before and after the GEMV launch. */
int needle2_gpu_plan_run_timed(void *plan, void *stream, void *gemv_start, void *gemv_stop);
/* Chained int8 plans (no counterpart in the reference, whose CPU layer runs
 * each projection on its own; Engine::attention_projections_batch,
 * needle2/csrc/engine.cpp:671-750, quantizes each input in turn): with
 * `prepared` non-zero the run uses the prepared input a chained call of its
 * producer left in its staging since its last run (and prepares its input
 * itself when none did); with `next` not NULL (a one-matrix int8 plan whose
 * input buffer is this plan's output) the run also leaves next's input
 * prepared, in the GEMV epilogue for groups of 32 on decode-sized matrices,
 * else by next's prepare launch, unless next's GEMV prepares its own input
 * (batch 1). Outputs are the bits of unchained runs; one stream per chain. */
int needle2_gpu_plan_run_chained(void *plan, void *next, int prepared, void *stream);
void needle2_gpu_plan_destroy(void *plan);

/* Device memory, streams and events (HIP runtime of this library). */
void *needle2_gpu_malloc(size_t bytes);
void needle2_gpu_free(void *ptr);
int needle2_gpu_memcpy(void *dst, const void *src, size_t bytes, int kind); /* 0 H2D, 1 D2H, 2 D2D */
int needle2_gpu_memset(void *dst, int value, size_t bytes);
/* Streaming copy kernel (16 B per lane per step; bytes rounded down to 16), the
 * reference point for scaling hardware byte counters to HBM bytes. */
int needle2_gpu_copy_kernel(void *dst, const void *src, size_t bytes, void *stream);
/* Hardware calibration (no counterpart in the reference: the measured limits
 * the kernels are compared against). calib_launch: microseconds per launch of
 * an empty kernel issued `launches` times back to back on `stream` (the
 * dependent-launch floor). calib_lds: LDS read bytes per shader clock per CU
 * for `width`-byte reads (4, 8, 16; every lane its own column) and the shader
 * clock of the run. calib_stream: microseconds per pass reading one third of
 * the `bytes` of d_src (the thirds in turn, so no pass finds the previous one
 * in the last-level cache; at least 3 * 512 * 48 KiB): pattern 0 / 1 the
 * GEMVs' walk (512 workgroups, each reading its own contiguous tile front to
 * back, tiles of whole 48 KiB multiples) with plain / non-temporal loads, 2 /
 * 3 grid-stride streaming with plain / non-temporal loads. */
int needle2_gpu_calib_launch(int launches, float *us_per_launch, void *stream);
int needle2_gpu_calib_lds(int width, float *bytes_per_clk_per_cu, float *shader_ghz, void *stream);
int needle2_gpu_calib_stream(const void *d_src, size_t bytes, int pattern, float *us, void *stream);
int needle2_gpu_synchronize(void);
void *needle2_gpu_stream_create(void);
void needle2_gpu_stream_destroy(void *stream);
int needle2_gpu_stream_synchronize(void *stream);
void *needle2_gpu_event_create(void); /* timing event: recorded without a system-scope fence */
void needle2_gpu_event_destroy(void *event);
int needle2_gpu_event_record(void *event, void *stream);
float needle2_gpu_event_elapsed(void *start, void *stop); /* ms; waits for stop */
int needle2_gpu_device_info(char *buf, int len);         /* "name;arch;cus;hbm_bytes;clock_khz" */
/* HIP graphs (no counterpart in the reference, which has no device): capture
 * what is issued to `stream` between begin and end, instantiate, replay with
 * one launch. Entry points used inside must have run once before the capture
 * and must not read host memory: plan_run, attention, kv_store_device. */
int needle2_gpu_graph_begin(void *stream);
void *needle2_gpu_graph_end(void *stream);                /* instantiated graph, or NULL */
int needle2_gpu_graph_launch(void *graph, void *stream);
void needle2_gpu_graph_destroy(void *graph);

/* ---- int8 KV cache and batched decode attention ----------------------------
 * Replaces the int8 branch of the reference Engine's cache and attention,
 * which it exposes only through needle2_engine_set_int8_kv and
 * needle2_engine_kv_storage_bytes (needle2/native.py:418-433):
 *   allocation      needle2/csrc/engine.cpp:433-449 (reset)
 *   quantize/store  needle2/csrc/engine.cpp:1005-1021
 *   attention       needle2/csrc/engine.cpp:898-967 (with 56-74, 137-147, 816-897)
 * Here one handle holds `seqs` sequences, so one call serves a whole decode
 * batch. Layout on the device is private; kv_import / kv_export move host
 * rows in the reference's layout ([slots][kvheads][head_dim] int8 and
 * [slots][kvheads] fp32 scales). head_dim: 32, 64 or 128; query heads per
 * kv head: 1, 2, 4 or 8. All return 0 / -1 (message in needle2_gpu_error). */
void *needle2_gpu_kv_create(int layers, int capacity, int kvheads, int head_dim, int seqs);
void needle2_gpu_kv_destroy(void *kv);
size_t needle2_gpu_kv_storage_bytes(void *kv);   /* engine.cpp kv_storage_bytes (int8 cache) */
/* d_k, d_v: device fp32 [seqs][count][kvheads][head_dim]; token i of
 * sequence s goes to slot (seq_first_slot ? seq_first_slot[s] : first_slot) + i
 * (seq_first_slot is a host array). */
int needle2_gpu_kv_store(void *kv, int layer, const float *d_k, const float *d_v, int count, int first_slot,
                         const int *seq_first_slot, void *stream);
/* The same with the first slots in device memory (d_first_slot[seqs]); no
 * host copy or wait, so it can be captured in a graph. Rows whose slot falls
 * outside [0, capacity) are skipped. */
int needle2_gpu_kv_store_device(void *kv, int layer, const float *d_k, const float *d_v, int count,
                                const int *d_first_slot, void *stream);
/* d_q, d_out: device fp32 [seqs][heads][head_dim]. Sequence s attends slots
 * d_slots[j] (device, >= length entries; NULL: j) for j < d_lengths[s]
 * (device; NULL: length), never more than `length`; listed slots outside
 * [0, capacity) are skipped. splits: slot-range pieces (0: automatic). */
int needle2_gpu_attention(void *kv, int layer, const float *d_q, float *d_out, int heads, int length,
                          const int *d_slots, const int *d_lengths, int splits, void *stream);
/* needle2_gpu_attention that first stores the step's new token of every
 * sequence (d_new_k / d_new_v [seqs][kvheads][head_dim] fp32 at slot
 * d_new_slot[s]: needle2_gpu_kv_store_device with count 1; all three NULL:
 * no store) and also leaves d_out prepared as the input of `next` (NULL, or
 * a one-matrix int8 plan of batch seqs reading d_out, e.g. the O projection)
 * for needle2_gpu_plan_run_chained(next, ..., prepared = 1). Both in the
 * attention launch where its shapes allow. Counterpart of the store-then-
 * attend order of Engine::step (needle2/csrc/engine.cpp:1005-1021, 898-967),
 * whose next linear quantizes the attention output itself. */
int needle2_gpu_attention_chained(void *kv, int layer, const float *d_q, float *d_out, int heads, int length,
                                  const int *d_slots, const int *d_lengths, int splits, const float *d_new_k,
                                  const float *d_new_v, const int *d_new_slot, void *next, void *stream);
int needle2_gpu_kv_import(void *kv, int layer, int seq, const int8_t *k, const int8_t *v, const float *k_scales,
                          const float *v_scales, int first_slot, int count);
int needle2_gpu_kv_export(void *kv, int layer, int seq, int8_t *k, int8_t *v, float *k_scales, float *v_scales,
                          int first_slot, int count);

#ifdef __cplusplus
}
#endif

#endif /* NEEDLE2_NATIVE_H */
