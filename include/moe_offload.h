/*
 * moe_offload.h -- C ABI of libmoeoffload.so, the MI355X (gfx950) expert-offload
 * MoE path.
 *
 * Conventions for every entry point:
 *   - arguments are plain pointers and sizes; device pointers are HBM
 *     addresses, "host" pointers are page-locked host memory;
 *   - kernels are enqueued on `stream` (a hipStream_t; NULL = the null
 *     stream) and never synchronise, never allocate and never record a
 *     memset, so every call can sit inside a captured hipGraph;
 *   - every quantity that changes from call to call at replay time (expert
 *     ids, miss counts, the LRU step) is read from device memory by the
 *     kernel, never baked into a launch argument;
 *   - the return value is 0 on success, MOE_EINVAL (-1) when a precondition
 *     fails (nothing is enqueued), or the positive hipError_t of a failed
 *     launch; moe_last_error() then describes the failure (thread-local);
 *   - a call with zero tokens does nothing and may pass NULL for its
 *     per-token arrays (moe_permute / moe_unique_inverse still write their
 *     per-expert outputs: all experts empty).
 */
#ifndef MOE_OFFLOAD_H
#define MOE_OFFLOAD_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define MOE_OK 0
#define MOE_EINVAL (-1)

/* dtype codes for arguments that accept more than one element type */
#define MOE_I32 0
#define MOE_I64 1
#define MOE_F32 2
#define MOE_BF16 3

/* ------------------------------------------------------------------ misc */

/* Text of the last failure on this thread ("" if none). */
const char* moe_last_error(void);

/* Library version string, and the path of the HIP runtime library this
 * library resolved its HIP symbols from (to check it shares the caller's
 * runtime). */
const char* moe_version(void);
const char* moe_hip_runtime_path(void);

/* Device self-check of the activation quantiser's e4m3 encoding.  The
 * kernels quantise with the conversion unit (v_cvt_pk_fp8_f32 after a clamp
 * to +-448, NaN kept as sign | 0x7f); this compares that, for the float bit
 * patterns first .. first + count - 1 (1 <= count <= 2^30), with the
 * branch-free software encoder that the CPU tests pin against the oracle's
 * round-to-nearest-even e4m3fn (oracle/fp8.py), and adds the number of
 * mismatching patterns to *mismatches (device uint64, not cleared here).
 * No counterpart in the reference, whose activations are quantised by
 * torch's float8_e4m3fn cast inside fp8_moe_forward (bin/offload.py:239). */
int moe_e4m3_check(uint32_t first, uint32_t count, uint64_t* mismatches, void* stream);

/* Device self-check of the expert kernels' SiLU(gate) * up: out[i] =
 * g[i] * rcp(1 + 2^(-g[i] log2 e)) * u[i] on the hardware exp2 and
 * reciprocal, the float32 formula the decode and grouped kernels apply to
 * h, for n <= 2^30 device floats (n == 0 does nothing).  No counterpart in
 * the reference, whose SiLU runs inside fp8_moe_forward
 * (bin/devcache.py:275-277). */
int moe_silu_check(const float* g, const float* u, float* out, uint32_t n, void* stream);

/* HBM read floor: every 16-byte word of src[0, bytes) (bytes a multiple of
 * 16, src 16-byte aligned) is read once with nontemporal loads by
 * `workgroups` workgroups of 256 threads (1..65535), four loads in flight
 * per lane; nothing is written unless the XOR of a lane's words equals a
 * fixed constant (then to sink[0], device uint32).  No counterpart in the
 * reference: it measures the read-only floor that the decode GEMV and the
 * HBM roofline are judged against. */
int moe_stream_read(const void* src, int64_t bytes, int32_t workgroups, uint32_t* sink,
                    void* stream);

/* y[t] = x[t] W^T in bf16 for 1..128 tokens: W [out_features, in_features]
 * bf16 (nn.Linear layout, in_features a multiple of 8), x [tokens,
 * in_features], y [tokens, out_features]; each output the f32 sum of its
 * row's products rounded once to bf16 (up to 4 tokens: per lane in slice
 * order, then a fixed lane tree; 5 to 128 tokens: on the matrix cores,
 * with in_features a multiple of 64, out_features of 16 and no x_add).
 * x_add (nullable, x's shape, up to 4 tokens): the product is of
 * bf16(x + x_add) instead, each element's float sum rounded once to bf16
 * (a residual add folded into the loads).  rows_per_wave (up to 4
 * tokens): 1, 2 or 4 rows per wave, 0 for the default (1); the outputs do
 * not depend on it.  x, x_add and w 16-byte aligned.  No counterpart in the reference: the
 * decode benchmark's stand-in for the non-expert compute of a layer (one
 * [2048, 2048] matrix) runs on it, one pass over the weights. */
int moe_linear_bf16(const void* x, const void* x_add, const void* w, int32_t tokens,
                    int32_t in_features, int32_t out_features, void* y,
                    int32_t rows_per_wave, void* stream);

/* Measurement: the calling thread's next moe_route_fetch_ffn or
 * moe_fetch_ffn call records `start` and `stop` (hipEvent_t, created by the
 * caller) around its fetch + gate/up launch alone, through
 * hipExtLaunchKernel, so hipEventElapsedTime gives that kernel's own
 * duration.  The next such call disarms them, whether or not it launches;
 * NULL, NULL disarms.  Not for stream capture.  No counterpart in the
 * reference: it times the decode step's dominant kernel for its roofline. */
int moe_time_fused_launch(void* start, void* stop);

/* ------------------------------------------------------------- host pool */

/* Page-locked, device-mapped host allocation for an expert pool.
 * flags: 0 = coherent (hipHostMallocMapped), 1 = non-coherent
 * (hipHostMallocMapped | hipHostMallocNonCoherent).
 * Replaces the per-layer Tensor.pin_memory() of pin_experts
 * (bin/offload.py:664-699) with one region per pool. */
int moe_host_alloc(void** host_ptr, size_t bytes, int flags);
int moe_host_free(void* host_ptr);

/* Device-side address of page-locked host memory (hipHostGetDevicePointer).
 * Replaces device_ptr_of (csrc/fetch_experts.cu:40-47). Fails with
 * MOE_EINVAL for memory the runtime does not know as page-locked (the
 * reference's "expected a contiguous page-locked CPU tensor"). */
int moe_device_ptr_of(const void* host_ptr, void** dev_ptr);

/* ------------------------------------------------------------ slot table */

/* Initialise one layer's slot table: slot_of[0..n_experts) = -1,
 * slot_expert[0..cap) = -1, slot_stamp[c] = -(cap - c), step = 0.
 * Replaces the table set-up of init_dev_cache (bin/devcache.py:146-152). */
int moe_slots_init(int32_t* slot_of, int32_t n_experts, int32_t* slot_expert,
                   int64_t* slot_stamp, int32_t cap, int64_t* step, void* stream);

/* Resolve k expert ids to cache slots on the device, queueing misses.
 * Replaces _resolve_slots (bin/devcache.py:45-98) with identical decisions:
 * step += 1; a hit stamps its slot; a miss takes the slot with the smallest
 * stamp (lowest index on a tie), evicting its expert.  Outputs
 * out_slot[k], fetch_slot[<=k], fetch_expert[<=k], nmiss[1].
 * ids_dtype: MOE_I32 or MOE_I64.  stats (nullable) is int64[2]
 * {hits, misses} accumulated on the device -- the reference keeps no such
 * counter (bin/devcache.py:274).  Constraints: 1 <= cap <= 4096,
 * n_experts >= 1, k <= cap (more ids than slots would give one slot to two
 * ids of the call; the reference's callers never pass more than 8 ids,
 * bin/devcache.py:232-233); ids must lie in [0, n_experts) (an out-of-range
 * id is ignored and reported as slot -1). */
int moe_resolve_slots(const void* ids, int32_t ids_dtype, int32_t k,
                      int32_t* slot_of, int32_t n_experts,
                      int32_t* slot_expert, int64_t* slot_stamp, int32_t cap,
                      int64_t* step, int32_t* out_slot, int32_t* fetch_slot,
                      int32_t* fetch_expert, int32_t* nmiss, int64_t* stats,
                      void* stream);

/* ----------------------------------------------------------------- fetch */

/* One (host buffer, cache buffer) pair moved on a miss: record j of the
 * host buffer (src + j * bytes) is copied to slot s of the cache buffer
 * (dst + s * bytes).  Mirrors _copy_pairs (bin/devcache.py:170-181). */
typedef struct moe_fetch_pair {
  const void* src;   /* device-side address of the page-locked host buffer */
  void* dst;         /* HBM cache buffer */
  int64_t bytes;     /* bytes per expert record in this buffer */
  int64_t tile_k;    /* 0: a byte copy.  K > 0: each record of this buffer is
                        a row-major [bytes / K, K] e4m3 matrix (K % 128 == 0,
                        bytes / K a multiple of 16) written to the cache in
                        MFMA tile order (MOE_LAYOUT_TILES) */
} moe_fetch_pair;

/* Copy the queued misses host -> HBM with a zero-copy gather kernel.
 * Job j < min(*nmiss, max_jobs) copies expert fetch_expert[j] into slot
 * fetch_slot[j] for every pair; *nmiss is read on the device at run time,
 * so later jobs cost nothing.  The grid is blocks_per_job * min(max_jobs, 8)
 * workgroups of 128 threads over which the queued records are dealt in
 * 8 KiB pieces (default 3 per job: ~192 KiB of host reads in flight, about
 * the link's bandwidth-delay product; more outstanding reads measured
 * slower).  A tile-order pair's pieces are 16 rows x up to 512 bytes,
 * transposed through LDS into one contiguous 8 KiB run of the slot.
 * Replaces fetch_experts/fetch_kernel (csrc/fetch_experts.cu:49-94) and the
 * four per-buffer launches of _cpp_fetch (bin/devcache.py:197-220) with one
 * launch.  fetch_expert and fetch_slot hold max_jobs entries (each
 * workgroup reads its first job before the count is known; entries at or
 * past *nmiss are read, never used).  Preconditions: 1 <= npairs <= 4;
 * each pair's src, dst and bytes are 4-byte aligned (16-byte aligned pairs
 * take the 16-byte path), and a pair with tile_k > 0 is 16-byte aligned
 * with records under 64 GiB; 1 <= max_jobs <= 65535;
 * 1 <= blocks_per_job <= 4096. */
int moe_fetch(const moe_fetch_pair* pairs, int32_t npairs,
              const int32_t* fetch_expert, const int32_t* fetch_slot,
              const int32_t* nmiss, int32_t max_jobs, int32_t blocks_per_job,
              void* stream);

/* ---------------------------------------------------------------- router */

/* Router: logits = x . W^T (+ bias), softmax, top_k, renormalise.
 * x [tokens, hidden] bf16, w [n_experts, hidden] bf16, bias [n_experts]
 * f32 or NULL.  Writes ids [tokens, top_k] (ids_dtype MOE_I32/MOE_I64),
 * weights [tokens, top_k] (w_dtype MOE_F32/MOE_BF16), and the f32 logits
 * [tokens, n_experts] to `logits` (caller-provided, also the workspace).
 * Each logit is the float64-accumulated sum of exact bf16 x bf16 products
 * rounded once to logit_dtype: MOE_BF16 (the output of upstream's bf16
 * nn.Linear gate, round to nearest even) or MOE_F32; the bias is then added
 * in float32.  Selection is by descending logit, ties to the lower index;
 * weights are the softmax over the selected logits.
 * Replaces upstream's gate + softmax + topk + norm_topk_prob
 * (moe.py:217-220 per notes/01-static-findings.md:133-138).
 * Constraints: hidden % 8 == 0, 1 <= top_k <= 32, top_k <= n_experts <= 4096. */
int moe_router_topk(const void* x, const void* w, const float* bias,
                    int32_t logit_dtype, int32_t tokens, int32_t hidden, int32_t n_experts,
                    int32_t top_k, float* logits, void* ids, int32_t ids_dtype,
                    void* weights, int32_t w_dtype, void* stream);

/* Decode-step fusion of the router and the slot-table resolve for ONE token:
 * moe_router_topk (ids int32 [top_k], weights f32 [top_k], logits f32
 * [n_experts]) followed by moe_resolve_slots on those ids, in two launches
 * instead of three.  Outputs and table updates are exactly those of the two
 * entry points called in sequence, and top_k <= cap as there.  It has no
 * single counterpart in the
 * reference: it fuses the router (moe.py:217-220) with _resolve_slots
 * (bin/devcache.py:45-98) as they occur back to back in the decode step
 * (bin/devcache.py:230-239). */
int moe_route_resolve(const void* x, const void* w, const float* bias,
                      int32_t logit_dtype, int32_t hidden, int32_t n_experts, int32_t top_k,
                      float* logits, int32_t* ids, float* weights,
                      int32_t* slot_of, int32_t* slot_expert,
                      int64_t* slot_stamp, int32_t cap, int64_t* step,
                      int32_t* out_slot, int32_t* fetch_slot,
                      int32_t* fetch_expert, int32_t* nmiss, int64_t* stats,
                      void* stream);

/* Decode-step fusion of the router, the slot-table resolve AND the fetch of
 * the misses for ONE token, in two launches instead of four: the logits
 * (which also count the step), then one launch on the fetch's grid whose
 * every workgroup makes the resolve's decisions and copies its share of the
 * misses, workgroup 0 writing the outputs.  Decisions, outputs (ids,
 * weights, out_slot, fetch lists, nmiss, stats) and cache contents are those
 * of moe_route_resolve followed by moe_fetch(pairs, npairs, fetch_expert,
 * fetch_slot, nmiss, top_k, blocks_per_job).
 * The slot table is double-buffered: slot_of [2, n_experts], slot_expert
 * [2, cap] and slot_stamp [2, cap], with buffer 0 set up by moe_slots_init
 * (step 0); after a call that leaves *step = s the table is buffer s & 1
 * (the call reads buffer (s - 1) & 1 and writes the other, so no workgroup
 * reads what another writes).
 * No counterpart in the reference: it fuses the router (moe.py:217-220),
 * _resolve_slots (bin/devcache.py:45-98) and the fetch
 * (csrc/fetch_experts.cu:49-94) as they occur back to back in the decode
 * step (bin/devcache.py:230-255).  Constraints: those of moe_route_resolve
 * and moe_fetch, with n_experts <= 1024 and cap <= 1024. */
int moe_route_fetch(const void* x, const void* w, const float* bias, int32_t logit_dtype,
                    int32_t hidden, int32_t n_experts, int32_t top_k, float* logits,
                    int32_t* ids, float* weights, int32_t* slot_of, int32_t* slot_expert,
                    int64_t* slot_stamp, int32_t cap, int64_t* step, int32_t* out_slot,
                    int32_t* fetch_slot, int32_t* fetch_expert, int32_t* nmiss, int64_t* stats,
                    const moe_fetch_pair* pairs, int32_t npairs, int32_t blocks_per_job,
                    void* stream);

/* The decode step's whole MoE layer of one token from packed records:
 * moe_route_fetch's router, slot resolve and miss fetch followed by
 * moe_fp8_moe_forward_ex's expert FFN on the cache slots, in three launches
 * instead of four, with the same outputs bit for bit.  The workgroups that
 * fetch a miss's gate and up rows run that expert's gate/up MFMAs on the
 * bytes as they arrive, and the hits' gate/up runs beside the fetch in the
 * same launch; the down projection (with the routing weights, the residual
 * and the bf16 output) is the last launch.  Records: w13 [2*inter, hidden] |
 * w2 [hidden, inter], both in MFMA tile order (MOE_LAYOUT_TILES), | s13
 * [2*inter/128, hidden/128] | s2 [hidden/128, inter/128] f32, record_bytes
 * apart (>= their sum, a multiple of 256) in `pool` (the device address of
 * the page-locked host pool, n_experts records) and in `cache` (cap slots),
 * both 256-byte aligned.  out [hidden] bf16 = bf16(residual + bf16(MoE(x)))
 * (residual nullable, may be x), the workspace 256-byte aligned with
 * top_k * inter floats rounded up to 256 bytes plus 256 bytes (the
 * fetch's piece counter, which the logits launch zeroes;
 * moe_fp8_moe_workspace(1, top_k, cap, hidden, inter) bytes always
 * suffice).  With `shared` (nullable) the call is the MoE block
 * of moe_fp8_moe_block_forward: the shared expert's gate/up rows ride in the
 * fetch launch and its down rows in the down launch, out = bf16(residual +
 * bf16(routed + sigmoid-gated shared)), and the workspace holds
 * moe_fp8_moe_block_workspace(1, top_k, cap, hidden, inter, shared->inter)
 * bytes.  The table arguments are moe_route_fetch's (double-buffered).
 * Constraints: hidden a multiple of 512 up to 8192, inter a multiple of 128
 * up to 2048, 1 <= top_k <= min(16, n_experts) <= cap <= 1024, n_experts <=
 * 1024.  Replaces, for the decode step, the router top-k + _resolve_slots +
 * fetch_experts + fp8_moe_forward sequence of bin/devcache.py:230-277; no
 * single counterpart. */
int moe_route_fetch_ffn(const void* x, const void* w, const float* bias, int32_t logit_dtype,
                        int32_t hidden, int32_t n_experts, int32_t top_k, float* logits,
                        int32_t* ids, float* weights, int32_t* slot_of, int32_t* slot_expert,
                        int64_t* slot_stamp, int32_t cap, int64_t* step, int32_t* out_slot,
                        int32_t* fetch_slot, int32_t* fetch_expert, int32_t* nmiss,
                        int64_t* stats, const void* pool, void* cache, int64_t record_bytes,
                        int32_t inter, int32_t blocks_per_job,
                        const struct moe_shared_expert* shared, const void* residual, void* out,
                        void* workspace, size_t workspace_bytes, void* stream);

/* moe_route_fetch_ffn with no cache policy: every routed expert is a miss,
 * fetched on every call into cache slot k, its place in the top-k (0-hit
 * decode; the cache holds cap >= top_k slots).  There is no slot table;
 * out_slot[k] = k, the miss list is fetch_expert = ids and fetch_slot[k] = k
 * with *nmiss = top_k, and stats (nullable) gains top_k misses.  The three
 * launches, the other arguments and the outputs are moe_route_fetch_ffn's:
 * with every pick a miss, the step's output, ids, weights and slot bytes
 * equal moe_router_topk + moe_fetch of ids into slots 0..top_k-1 +
 * moe_fp8_moe_forward_ex (or moe_fp8_moe_block_forward with `shared`) bit
 * for bit.  Replaces the uncached offloaded_forward's router top-k,
 * per-expert host-to-device copies and fp8_moe_forward
 * (bin/offload.py:137-239) for one decode token; no single counterpart. */
int moe_route_fetch_ffn_uncached(const void* x, const void* w, const float* bias,
                                 int32_t logit_dtype, int32_t hidden, int32_t n_experts,
                                 int32_t top_k, float* logits, int32_t* ids, float* weights,
                                 int32_t cap, int32_t* out_slot, int32_t* fetch_slot,
                                 int32_t* fetch_expert, int32_t* nmiss, int64_t* stats,
                                 const void* pool, void* cache, int64_t record_bytes,
                                 int32_t inter, int32_t blocks_per_job,
                                 const struct moe_shared_expert* shared, const void* residual,
                                 void* out, void* workspace, size_t workspace_bytes,
                                 void* stream);

/* The drop-in's fetch and expert FFN of one token: moe_fetch of the four
 * buffers (pairs in the order w13, w2, s13, s2, as the reference's
 * _cpp_fetch copies them, w13 and w2 with tile_k set so the cache holds
 * them in tile order) followed by moe_fp8_moe_forward_ex(x, slots, weights,
 * w13, s13, w2, s2, strides) on the cache, in two launches instead of three,
 * with the same outputs bit for bit.  The workgroups that fetch a miss's
 * gate and up rows run its gate/up MFMAs on each piece while it sits
 * transposed in LDS; the hits' gate/up runs beside the fetch.  slots
 * [top_k] int32 are the resolve's out_slot (every slot below n_slots), the
 * miss list its fetch_slot/fetch_expert/nmiss (max_jobs entries, top_k <=
 * max_jobs <= 32), weights [top_k] w_dtype MOE_F32/MOE_BF16, out [hidden]
 * bf16 = bf16(residual + bf16(MoE(x))) (residual nullable), the workspace
 * top_k * inter floats.  Constraints: those of moe_route_fetch_ffn on
 * hidden, inter and top_k; the w13/s13 and w2/s2 pairs fill the cache
 * buffers w13/s13 and w2/s2 (dense); strides->layout MOE_LAYOUT_TILES.
 * A slot that two picks share (an expert repeated in the row) is fetched
 * once and both picks read its activations.  Replaces fetch_experts +
 * fp8_moe_forward in dev_cached_forward (bin/devcache.py:270-277); no
 * single counterpart. */
int moe_fetch_ffn(const moe_fetch_pair* pairs, int32_t npairs, const int32_t* fetch_expert,
                  const int32_t* fetch_slot, const int32_t* nmiss, int32_t max_jobs,
                  int32_t blocks_per_job, const void* x, const int32_t* slots,
                  const void* weights, int32_t w_dtype, int32_t top_k, const void* w13,
                  const float* s13, const void* w2, const float* s2, int32_t n_slots,
                  int32_t hidden, int32_t inter, const struct moe_expert_strides* strides,
                  const void* residual, void* out, void* workspace, size_t workspace_bytes,
                  void* stream);

/* A slot table in the reference's single-buffer form (bin/devcache.py:146-
 * 152: slot_of [n_experts] int32, slot_expert [cap] int32, stamp [cap]
 * int64, step [1] int64) and staging of the same sizes for its next state:
 * the launch that resolves a call writes the next state there, because all
 * its workgroups read the table, and the launch after it copies it in. */
typedef struct moe_slot_table {
  int32_t* slot_of;
  int32_t* slot_expert;
  int64_t* stamp;
  int64_t* step;
  int32_t n_experts;
  int32_t cap;
  int32_t* next_slot_of;
  int32_t* next_slot_expert;
  int64_t* next_stamp;
  int64_t* next_step;
} moe_slot_table;

/* The drop-in's whole decode call in two launches: moe_resolve_slots on the
 * reference's table for ids [top_k] (ids_dtype MOE_I32/MOE_I64), then
 * moe_fetch_ffn.  Every workgroup of the first launch makes the call's slot
 * decisions from the table (the decisions of moe_resolve_slots, bit for
 * bit), workgroup 0 writes out_slot [top_k], the miss list (fetch_slot,
 * fetch_expert [top_k], nmiss), the hit/miss counters `stats` (nullable)
 * and the table's next state into the staging; the misses are fetched and
 * every pick's gate/up formed as in moe_fetch_ffn; the down launch forms
 * the output and copies the staging into the table, so the table holds the
 * call's decisions when the call's work is done, as after
 * moe_resolve_slots.  Constraints: those of moe_fetch_ffn with n_slots =
 * table->cap and max_jobs = top_k; 1 <= n_experts <= 1024, top_k <= cap <=
 * 1024.  Replaces _resolve_slots + fetch_experts + fp8_moe_forward in
 * dev_cached_forward (bin/devcache.py:230-277); no single counterpart. */
int moe_resolve_fetch_ffn(const void* ids, int32_t ids_dtype, int32_t top_k,
                          const moe_slot_table* table, int32_t* out_slot, int32_t* fetch_slot,
                          int32_t* fetch_expert, int32_t* nmiss, int64_t* stats,
                          const moe_fetch_pair* pairs, int32_t npairs, int32_t blocks_per_job,
                          const void* x, const void* weights, int32_t w_dtype, const void* w13,
                          const float* s13, const void* w2, const float* s2, int32_t hidden,
                          int32_t inter, const struct moe_expert_strides* strides,
                          const void* residual, void* out, void* workspace,
                          size_t workspace_bytes, void* stream);

/* ------------------------------------------------------- expert compute */

/* Workspace bytes moe_fp8_moe_forward needs for this shape. */
size_t moe_fp8_moe_workspace(int32_t tokens, int32_t top_k, int32_t n_experts,
                             int32_t hidden, int32_t inter);

/* W8A8 block-FP8 MoE forward, the counterpart of upstream
 * fp8_moe_forward(x, topk_ids, topk_weights, w13, s13, w2, s2) as called at
 * bin/devcache.py:275-277 and bin/offload.py:239.
 *   x        [tokens, hidden] bf16
 *   ids      [tokens, top_k]  MOE_I32/MOE_I64, index into the expert axis
 *   weights  [tokens, top_k]  MOE_F32/MOE_BF16
 *   w13      [n_experts, 2*inter, hidden] e4m3fn (gate rows, then up rows)
 *   s13      [n_experts, 2*inter/128, hidden/128] f32 scale_inv
 *   w2       [n_experts, hidden, inter] e4m3fn
 *   s2       [n_experts, hidden/128, inter/128] f32 scale_inv
 *   out      [tokens, hidden] bf16
 * Activations are quantised per token per 128 columns (scale amax/448).
 * Dispatch: decode-sized calls use the per-pair GEMV kernels, larger ones the
 * permuted grouped GEMM; both give bit-identical rows.
 * Constraints: hidden % 128 == 0, inter % 128 == 0, 1 <= top_k <= 16. */
int moe_fp8_moe_forward(const void* x, const void* ids, int32_t ids_dtype,
                        const void* weights, int32_t w_dtype, int32_t tokens,
                        int32_t top_k, const void* w13, const float* s13,
                        const void* w2, const float* s2, int32_t n_experts,
                        int32_t hidden, int32_t inter, void* out,
                        void* workspace, size_t workspace_bytes, void* stream);

/* Byte order of each expert's e4m3 matrices w13 [2*inter, hidden] and w2
 * [hidden, inter] (the scales are row-major in both):
 *   MOE_LAYOUT_ROWS   row-major, the checkpoint's nn.Linear layout (what
 *                     upstream fp8_moe_forward takes);
 *   MOE_LAYOUT_TILES  MFMA operand order: an [R, K] matrix is R/16 row
 *                     groups, each K/128 tiles of 2048 bytes in K order;
 *                     byte (16g + r, 128b + 32q + 16h + i) of the matrix
 *                     (r < 16, q < 4, h < 2, i < 16) sits at
 *                     (g*K/128 + b)*2048 + h*1024 + (16q + r)*16 + i.
 *                     A wave's 16-byte load of an MFMA A operand then reads
 *                     1 KiB contiguous (8 whole 128-byte lines) instead of
 *                     16 half lines; the packed host records use it.
 * Both orders give bit-identical results. */
#define MOE_LAYOUT_ROWS 0
#define MOE_LAYOUT_TILES 1

/* Distance between consecutive experts of each weight buffer, in elements
 * of that buffer (e4m3 bytes for w13/w2, floats for s13/s2).  Dense
 * [n, ...] buffers use the product of the trailing dimensions; a packed
 * record pool (w13|w2|s13|s2 per record) uses the record size.  `layout`
 * is MOE_LAYOUT_ROWS or MOE_LAYOUT_TILES (NULL strides: dense, rows). */
typedef struct moe_expert_strides {
  int64_t w13;
  int64_t s13;
  int64_t w2;
  int64_t s2;
  int64_t layout;
} moe_expert_strides;

/* moe_fp8_moe_forward with explicit expert strides (NULL = dense), an
 * optional bf16 residual [tokens, hidden] added to the bf16 result the way a
 * bf16 tensor add would (out = bf16(residual + bf16(sum_k w*y)); NULL =
 * none; it may be x itself, not out), and a kernel choice: mode 0 automatic
 * (per-pair GEMV up to 16 tokens, grouped beyond), 1 per-pair GEMV, 2
 * grouped, 3 per-pair GEMV with bf16 activations.  Modes 0-2 quantise the
 * activations (x, and SiLU(gate) * up) per 128 columns to e4m3 and give
 * bit-identical rows.  Mode 3 keeps them in bf16 (x as given, SiLU(gate) *
 * up rounded to bf16) and multiplies them with the e4m3 weights converted
 * exactly to bf16, accumulating in float32: the numerics of the
 * dequantise-then-matmul path (bin/offload.py's CPU experts), at any token
 * count the GEMV takes (pairs <= 65535: each pair reads its expert's weights,
 * where the grouped e4m3 path of a prefill-sized call reads each expert
 * once); with moe_fp8_moe_block_forward its shared expert runs in its own
 * two launches after the routed call. */
int moe_fp8_moe_forward_ex(const void* x, const void* ids, int32_t ids_dtype,
                           const void* weights, int32_t w_dtype,
                           int32_t tokens, int32_t top_k, const void* w13,
                           const float* s13, const void* w2, const float* s2,
                           int32_t n_experts, int32_t hidden, int32_t inter,
                           const moe_expert_strides* strides,
                           const void* residual, void* out,
                           void* workspace, size_t workspace_bytes,
                           int32_t mode, void* stream);

/* The router and the expert FFN of 1..16 tokens over resident experts, in
 * three launches instead of four: the router's logits (x . w_gate^T as in
 * moe_router_topk, + bias) into logits [tokens, n_experts], then the
 * per-pair GEMV gate/up launch, each of whose waves takes the top-k of its
 * token's logits itself (writing ids [tokens, top_k] int32 and weights
 * [tokens, top_k] float32), then the down launch.  ids, weights, logits and
 * out equal moe_router_topk followed by moe_fp8_moe_forward_ex (mode 1,
 * int32 ids, float32 weights) bit for bit.  No counterpart in the
 * reference: it fuses the router's top-k (moe.py:217-220) into
 * fp8_moe_forward (bin/devcache.py:275-277) for the all-resident decode.
 * Constraints: those of both, with 1 <= top_k <= min(16, n_experts),
 * n_experts <= 1024, w_gate 16-byte aligned. */
int moe_router_fp8_moe_forward(const void* x, const void* w_gate, const float* bias,
                               int32_t logit_dtype, int32_t tokens, int32_t hidden,
                               int32_t n_experts,
                               int32_t top_k, float* logits, int32_t* ids, float* weights,
                               const void* w13, const float* s13, const void* w2,
                               const float* s2, int32_t inter,
                               const moe_expert_strides* strides, const void* residual,
                               void* out, void* workspace, size_t workspace_bytes,
                               void* stream);

/* Bytes of the per-GPU scratch array behind moe_fp8_moe_forward_noalloc. */
#define MOE_NOALLOC_SCRATCH_BYTES ((size_t)16 << 20)

/* moe_fp8_moe_forward_ex without a workspace argument and without any
 * allocation: the workspace is a 16 MiB device array inside the library
 * (MOE_NOALLOC_SCRATCH_BYTES), one copy per GPU, held until the process
 * ends.  No counterpart in the reference: it is for callers that cannot
 * allocate (code under hipGraph capture, tight serving loops, harnesses
 * that forbid hipMalloc).  Calls whose moe_fp8_moe_workspace exceeds the
 * array are refused with MOE_EINVAL (decode, and batches up to about 160
 * tokens at top-8 of 256 with hidden 2048 and inter 512, fit).  Every call
 * on one GPU shares that GPU's array: calls that overlap on one GPU (two
 * streams or threads) race.  `stream` must belong to the current device,
 * on which the first call looks the array's address up.  Outputs are those
 * of moe_fp8_moe_forward_ex with the same arguments, bit for bit. */
int moe_fp8_moe_forward_noalloc(const void* x, const void* ids, int32_t ids_dtype,
                                const void* weights, int32_t w_dtype,
                                int32_t tokens, int32_t top_k, const void* w13,
                                const float* s13, const void* w2, const float* s2,
                                int32_t n_experts, int32_t hidden, int32_t inter,
                                const moe_expert_strides* strides,
                                const void* residual, void* out, int32_t mode,
                                void* stream);

/* ------------------------------------------------------ permute/unpermute */

/* Stable token->expert grouping of ids [tokens, top_k]:
 * counts[n_experts], offsets[n_experts + 1] (exclusive scan),
 * sorted_pairs[tokens*top_k] (pair p = t*top_k + k, sorted by expert, stable)
 * and pair_pos[tokens*top_k] (the inverse).  The counterpart of the
 * reference's torch.unique(return_inverse) remap (bin/offload.py:157-158,
 * 447-448) and of the sort inside upstream fp8_moe_forward.
 * Constraints: n_experts <= 4096, tokens*top_k <= 1<<24. */
int moe_permute(const void* ids, int32_t ids_dtype, int32_t tokens,
                int32_t top_k, int32_t n_experts, int32_t* counts,
                int32_t* offsets, int32_t* sorted_pairs, int32_t* pair_pos,
                void* stream);

/* out[t] = sum over k of weights[t,k] * y[pair_pos[t*top_k+k]], accumulated
 * in k order as acc = fma(w, y, acc) in float32, rounded to bf16 (the
 * combine of the decode path, so both give identical rows).
 * y [tokens*top_k, hidden] f32. */
int moe_unpermute(const float* y, const int32_t* pair_pos, const void* weights,
                  int32_t w_dtype, int32_t tokens, int32_t top_k,
                  int32_t hidden, void* out, void* stream);

/* Distinct experts of ids in ascending order and the renumbering of every
 * pair into that list (torch.unique(sorted, return_inverse), the remap of
 * bin/offload.py:157-158): n_unique[1], uniq[<=n_experts],
 * inverse[tokens*top_k] int32.  Needs counts/offsets from moe_permute.
 * Also writes rank_of[n_experts] (position in uniq, -1 when absent). */
int moe_unique_inverse(const void* ids, int32_t ids_dtype, int32_t tokens,
                       int32_t top_k, int32_t n_experts, const int32_t* counts,
                       int32_t* n_unique, int32_t* uniq, int32_t* rank_of,
                       int32_t* inverse, void* stream);

/* Hybrid prefill gather plan.  The distinct experts uniq[0..*n_unique) of a
 * multi-token call (from moe_unique_inverse) are split between the device
 * cache and the host pool: expert e = uniq[i] with 0 <= slot_of[e] < cap is
 * queued as (cache_src = slot_of[e], cache_dst = i), every other expert as
 * (host_expert = e, host_dst = i), both lists in uniq order; counts go to
 * n_host[1] and n_cache[1].  Two moe_fetch launches then fill gather slot i
 * from the cache slot (device to device) or from the host record.  The table
 * is only read -- no insert, no stamp -- so prefill never evicts the decode
 * working set.  cap == 0 (slot_of may be NULL) sends every expert to the
 * host list.  stats (nullable) int64[2] accumulates {cache copies, host
 * copies}.  Replaces the host loop of the reference's hybrid gather
 * (bin/offload.py:195-224), which needs slot_of.cpu() and a per-expert copy.
 * Lists need n_experts entries each; 1 <= n_experts <= 4096. */
int moe_gather_plan(const int32_t* uniq, const int32_t* n_unique,
                    const int32_t* slot_of, int32_t n_experts, int32_t cap,
                    int32_t* host_expert, int32_t* host_dst, int32_t* n_host,
                    int32_t* cache_src, int32_t* cache_dst, int32_t* n_cache,
                    int64_t* stats, void* stream);

/* Shared expert of the MoE block, first half.  The model gates a dense bf16
 * expert that every token passes through with a sigmoid and adds it to the
 * routed experts' output (notes/drama3-config.json:215-216
 * shared_expert_gate, shared_expert_intermediate_size 512;
 * notes/01-static-findings.md:80-82; checkpoint tensors
 * layers.N.mlp.shared_expert.{gate,up,down}_proj.weight and
 * layers.N.mlp.shared_expert_gate.weight [1, H], bf16).  The module itself
 * is upstream's and not in the reference; this is its conventional form.
 *   x [tokens, hidden], w_gate / w_up [inter, hidden], w_sgate [hidden]: bf16
 *   act [tokens, inter] bf16 = bf16(silu(bf16(x w_gate^T))) * bf16(x w_up^T)
 *   sig [tokens] f32 = bf16(sigmoid(bf16(x w_sgate^T)))  (bf16 values)
 * Each product rounds to bf16 as the model's bf16 modules do.  hidden and
 * inter positive multiples of 128; x and weights 16-byte aligned. */
int moe_shared_gate_up(const void* x, const void* w_gate, const void* w_up,
                       const void* w_sgate, int32_t tokens, int32_t hidden,
                       int32_t inter, void* act, float* sig, void* stream);

/* Shared expert, second half, and the block's sums:
 *   d   = bf16(act w_down^T)                 w_down [hidden, inter] bf16
 *   v   = bf16(sig * d)
 *   v   = bf16(routed + v)      if routed   (the routed experts' bf16 output)
 *   out = bf16(residual + v)    if residual
 * out [tokens, hidden] bf16 may alias routed or residual. */
int moe_shared_down(const void* act, const float* sig, const void* w_down,
                    int32_t tokens, int32_t hidden, int32_t inter,
                    const void* routed, const void* residual, void* out,
                    void* stream);

/* Decode-step finiteness guard: *flag = 1 if every one of the n elements of
 * x (dtype MOE_F32 or MOE_BF16, 16-byte aligned) is finite, else 0; the
 * device-side counterpart of the decode graph's
 * `finite.copy_(torch.isfinite(logits).all())` (generate.py:376-377 as
 * quoted in notes/botnotes/lm-head-inf-sentinel.md:18-28).  One workgroup
 * writes the flag, so nothing has to be cleared before a graph replay. */
int moe_all_finite(const void* x, int32_t dtype, int64_t n, int32_t* flag,
                   void* stream);

/* ------------------------------------------------------------------------
 * Entropy-coded records.  The reference stores host records raw
 * (bin/offload.py:603, 3,146,496 B per expert) and the decode step is bound
 * by moving them (its fetch, csrc/fetch_experts.cu:49-94).  A coded pool
 * holds the same records with the fp8 bytes' exponent nibble Huffman-coded
 * (blocks of 8192 bytes; sign and mantissa raw; the bytes after the fp8
 * part raw), about 84 % of the size for block-scaled weights, and
 * moe_fetch_coded decodes it on the GPU into cache slots identical to those
 * moe_fetch fills from the raw pool.  Format: codec.hip.  No counterpart in
 * the reference; an opt-in host pool format.
 * ---------------------------------------------------------------------- */

/* Counts of the 16 exponent values over the first fp8_bytes of each of the
 * n_records records (host memory) into hist[16]. */
int moe_codec_histogram(const void* records, int64_t n_records,
                        int64_t record_bytes, int64_t fp8_bytes,
                        uint64_t* hist, int32_t threads);

/* Largest coded size of one record (bytes), or -1 if fp8_bytes is not a
 * positive multiple of 8192. */
int64_t moe_codec_bound(int64_t record_bytes, int64_t fp8_bytes);

/* Code n_records records into dst (host): code_lengths[16] are the exponent
 * code lengths (1..6 bits, a prefix code).  Writes rec_offset[n + 1] (each
 * record's byte offset in dst, 256-aligned; the last is the total) and
 * blk_offset[n][nblk + 1] (each block's offset within its record; the last
 * is the raw tail's).  Returns the bytes used, or MOE_EINVAL. */
int64_t moe_codec_encode(const void* records, int64_t n_records,
                         int64_t record_bytes, int64_t fp8_bytes,
                         const uint8_t* code_lengths, void* dst,
                         int64_t dst_capacity, int64_t* rec_offset,
                         uint32_t* blk_offset, int32_t threads);

/* The decoder's 4096-entry table for code_lengths (at most 6 bits each):
 * entry p = first symbol | second symbol << 4 | total length << 8 of the two
 * codes that the stream bits p (least significant first) start with. */
int moe_codec_table(const uint8_t* code_lengths, uint16_t* lut);

/* moe_fetch for a coded pool: job j < min(*nmiss, max_jobs) decodes coded
 * record fetch_expert[j] into cache slot fetch_slot[j] (slot_bytes apart);
 * the lists hold max_jobs entries, as for moe_fetch.
 * pool: device address of the page-locked coded pool (256-byte aligned);
 * rec_offset, blk_offset, lut: device copies of moe_codec_encode's and
 * moe_codec_table's outputs.  Job lists are read on the device, so a
 * captured call serves new misses on every replay.  workgroups: grid size
 * (4 waves each, one 8192-byte block per wave at a time; 24-32 measured
 * best on MI355X). */
int moe_fetch_coded(const void* pool, const int64_t* rec_offset,
                    const uint32_t* blk_offset, int64_t record_bytes,
                    int64_t fp8_bytes, const uint16_t* lut,
                    const int32_t* fetch_expert, const int32_t* fetch_slot,
                    const int32_t* nmiss, int32_t max_jobs, void* cache,
                    int64_t slot_bytes, int32_t workgroups, void* stream);

/* moe_route_fetch for a coded pool: the router's logits (which count the
 * step), then one launch whose every workgroup makes the route (top-k and
 * slot resolve on the double-buffered table, workgroup 0 writing ids,
 * weights, out_slot, the fetch lists, nmiss, stats and the next buffer) and
 * decodes its share of the misses' coded records into their slots.
 * Outputs and cache contents are those of moe_route_resolve on the same
 * table followed by moe_fetch_coded(..., fetch_expert, fetch_slot, nmiss,
 * top_k, ...).  The table and the step as for moe_route_fetch; the pool,
 * offsets, table and grid as for moe_fetch_coded.
 * No counterpart in the reference: it fuses the router (moe.py:217-220),
 * _resolve_slots (bin/devcache.py:45-98) and the fetch of the misses
 * (csrc/fetch_experts.cu:49-94) for the coded pool format.  Constraints:
 * those of moe_route_fetch and moe_fetch_coded. */
int moe_route_fetch_coded(const void* x, const void* w, const float* bias,
                          int32_t logit_dtype, int32_t hidden, int32_t n_experts,
                          int32_t top_k, float* logits, int32_t* ids, float* weights,
                          int32_t* slot_of, int32_t* slot_expert, int64_t* slot_stamp,
                          int32_t cap, int64_t* step, int32_t* out_slot,
                          int32_t* fetch_slot, int32_t* fetch_expert, int32_t* nmiss,
                          int64_t* stats, const void* pool, const int64_t* rec_offset,
                          const uint32_t* blk_offset, int64_t record_bytes,
                          int64_t fp8_bytes, const uint16_t* lut, void* cache,
                          int64_t slot_bytes, int32_t workgroups, void* stream);

/* The MoE block's shared expert as one argument: bf16 weights w_gate and
 * w_up [inter, hidden], w_down [hidden, inter], w_sgate [hidden], all
 * 16-byte aligned. */
typedef struct moe_shared_expert {
  const void* w_gate;
  const void* w_up;
  const void* w_down;
  const void* w_sgate;
  int32_t inter;
} moe_shared_expert;

/* Workspace of moe_fp8_moe_block_forward: moe_fp8_moe_workspace's plus the
 * shared expert's act and gate scratch. */
size_t moe_fp8_moe_block_workspace(int32_t tokens, int32_t top_k,
                                   int32_t n_experts, int32_t hidden,
                                   int32_t inter, int32_t shared_inter);

/* The whole MoE block in one call:
 *   out = bf16(residual + bf16(routed + bf16(sig * shared_down)))
 * with routed the bf16 result of moe_fp8_moe_forward_ex on the same
 * arguments and the shared terms those of moe_shared_gate_up/_down, bit for
 * bit.  On the per-pair GEMV path with at most 2 tokens (decode) the shared
 * expert is carried by the two routed launches: extra workgroups of the
 * gate/up launch and one extra wave per workgroup of the down launch.  Any
 * other call runs the routed experts, then the two shared-expert kernels
 * on its output.  No counterpart in the reference: upstream's MoE block
 * calls the expert forward (bin/devcache.py:275-277) and the shared expert
 * separately. */
int moe_fp8_moe_block_forward(const void* x, const void* ids, int32_t ids_dtype,
                              const void* weights, int32_t w_dtype, int32_t tokens,
                              int32_t top_k, const void* w13, const float* s13,
                              const void* w2, const float* s2, int32_t n_experts,
                              int32_t hidden, int32_t inter,
                              const moe_expert_strides* strides,
                              const moe_shared_expert* shared, const void* residual,
                              void* out, void* workspace, size_t workspace_bytes,
                              int32_t mode, void* stream);

#ifdef __cplusplus
}
#endif

#endif /* MOE_OFFLOAD_H */
