/*
 * ferry_amd -- C ABI of the MI355X-native per-GPU MoE hot path of FERRY.
 *
 * Every entry point takes raw device pointers, int64 sizes and a hipStream_t (passed as
 * void*), returns 0 on success and a non-zero status on error; ferry_last_error() then
 * returns a thread-local message.  Apart from the H2D engine handle (which owns one HIP
 * stream and per-slot events) the library allocates no memory: scratch space is passed in
 * by the caller.  All index arrays are int64 like the reference's (torch.long) tensors.
 *
 * The replaced reference interfaces are cited per entry point (paths are relative to the
 * FERRY repository).
 */
#ifndef FERRY_AMD_H
#define FERRY_AMD_H

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* Thread-local description of the last failure of any entry point. */
const char* ferry_last_error(void);
/* ABI version of this library (bumped on any signature change). */
int32_t ferry_abi_version(void);

/*
 * Per-launch kernel timing (a measurement aid with no reference counterpart): when enabled,
 * every kernel launch of the library is bracketed by its own start/stop HIP events.
 * ferry_timing_enable clears the log; ferry_timing_summary sums the launches of one kernel;
 * ferry_timing_mark returns the current log position and ferry_timing_range sums the launches
 * between two positions.  The sums wait for the launches they cover.
 */
int ferry_timing_enable(int32_t enable);
int ferry_timing_summary(const char* kernel, int64_t* launches, double* total_ms);
int64_t ferry_timing_mark(void);
int ferry_timing_range(int64_t begin, int64_t end, double* total_ms);
/* time in ms that the launches at log positions [begin, end) overlap the window between the
 * caller's timing events t0 and t1 (hipEvent_t): the compute that ran while copies were in
 * flight, when t0 / t1 bracket the copies */
int ferry_timing_overlap(int64_t begin, int64_t end, void* t0, void* t1, double* total_ms);

/* A plain read of `bytes` (a multiple of 16) of device memory at `data` (16-byte aligned) on
 * `stream`: the HBM read ceiling that memory-bound kernels are measured against (a measurement
 * aid with no reference counterpart).  Each wavefront of the launch reads 8 KiB and stores the
 * XOR of its 16-byte words at sink + 16 * w (device memory, 16-byte aligned, at least
 * ferry_hbm_read_sink_bytes(bytes) bytes): the XOR of those records is the XOR of the range. */
int64_t ferry_hbm_read_sink_bytes(int64_t bytes);
int ferry_hbm_read(const void* data, int64_t bytes, void* sink, int64_t sink_bytes, void* stream);

enum { FERRY_BF16 = 0, FERRY_F32 = 1 };

/*
 * Router: fp32 softmax over each row of logits[T, E], top-k, optional renormalisation of the
 * k weights, multiplication by `scale`, cast to bf16.
 * Replaces ferry/model.py:141-146 (Qwen3 hook: softmax(dtype=fp32), topk(k) sorted,
 * w /= w.sum(), .to(bf16)) and the greedy DeepSeek-V2 gate whose outputs reach
 * ferry/model.py:151-157 (softmax, topk(sorted=False), * routed_scaling_factor, .to(bf16)).
 * Selection reproduces torch's CPU topk exactly, ties included.  probs_out (nullable)
 * receives the fp32 probabilities [T, E]; tie_rows (nullable, one int32 counter) counts
 * rows that took the exact tie-resolution path.
 */
int ferry_router_topk(const void* logits, int32_t logits_dtype, int64_t tokens, int64_t experts,
                      int64_t topk, int32_t renorm, float scale, int32_t sorted,
                      int64_t* idx_out, void* w_out_bf16, float* probs_out, int32_t* tie_rows,
                      void* stream);

/*
 * Dispatch layout at world = 1.  Replaces ferry/layout.py:12-94 (build_layout +
 * device_layout: sorted packet IDs, per-expert counts, exclusive prefix, stable
 * (rows, cols) counting sort) and the packet-weight reorder of pack_dispatch
 * (ferry/csrc/expert_ops.cpp:57-60).  Outputs, all device memory:
 *   send_ids[T,k]   int64  expert IDs of each token, ascending
 *   w_sorted[T,k]   bf16   routing weight of send_ids[t,j]
 *   starts[E+1]     int64  exclusive prefix of the per-expert counts
 *   rows[T*k]       int64  token of each (expert, rank) entry, ascending token per expert
 *   cols[T*k]       int64  position of that expert in the token's sorted ID list
 *   pair_pos[T*k]   int32  inverse map: pair_pos[t*k+j] = grouped position (nullable)
 * `workspace` must hold ferry_layout_workspace_bytes(T, k, E) bytes of device memory.  Every
 * token's IDs must be distinct and in [0, E); after the call the first 4 bytes of `workspace`
 * hold an int32 count of the tokens that break this (their entries are left out of the
 * permutation), for the caller to read when it wants the check.
 */
int64_t ferry_layout_workspace_bytes(int64_t tokens, int64_t topk, int64_t experts);
int ferry_layout(const int64_t* selected, const void* weights_bf16, int64_t tokens, int64_t topk,
                 int64_t experts, int64_t* send_ids, void* w_sorted_bf16, int64_t* starts,
                 int64_t* rows, int64_t* cols, int32_t* pair_pos, void* workspace,
                 int64_t workspace_bytes, void* stream);
/*
 * ferry_layout with no workspace argument and no allocation.  No counterpart in the reference:
 * it is for callers that cannot allocate device memory (code under HIP graph capture, tight
 * serving loops, harnesses that forbid hipMalloc).  The workspace is a static device buffer of
 * 262,400 bytes per GPU (256 + 128 * 512 * 4), held until the process ends, which bounds the
 * layout to ferry_layout_workspace_bytes(T, k, E) <= 262,400: at most 524,288 tokens with 128
 * experts, 131,072 with 512.  Larger calls fail with an error before any launch.  Every call on
 * one GPU shares that buffer, so calls that overlap on one GPU (on different streams, or from
 * different threads) race; calls ordered on one stream do not.  The device of the calling
 * thread must be the one `stream` belongs to.  Outputs and errors as ferry_layout; the
 * invalid-ID count stays in the static buffer.
 */
int ferry_layout_noalloc(const int64_t* selected, const void* weights_bf16, int64_t tokens,
                         int64_t topk, int64_t experts, int64_t* send_ids, void* w_sorted_bf16,
                         int64_t* starts, int64_t* rows, int64_t* cols, int32_t* pair_pos,
                         void* stream);

/*
 * Grouped SwiGLU over resident cache slots.  Replaces ferry/csrc/expert_ops.cpp:13-45
 * (execute_experts: per expert x = in[rows]; g = x Wg^T; u = x Wu^T; a = silu(g) * u;
 * y = a Wd^T; out = y * w[rows, cols]) and the silu_mul kernel of
 * ferry/csrc/expert_ops.cu:6-25.  cache[slot] = [gate I*H | up I*H | down H*I] bf16.
 * The experts computed are expert_list[0..n_list); slot_of[e] gives the cache slot of
 * expert e (host arrays, at most FERRY_MAX_EXPERTS entries).  x is bf16 [R, H];
 * w_sorted bf16 [R, k]; starts/rows/cols come from ferry_layout.  act is bf16 scratch of
 * [R*k, I] elements.  out_mode 0 writes bf16 rows out[rows[p]*k + cols[p]] (token-major,
 * the combine input); out_mode 1 writes row p of out (grouped order).
 * max_rows_per_expert must bound every n_e from above (R does for a layout from ferry_layout),
 * min_rows_per_expert from below (0 when unknown).  Experts with at most 64 rows run the
 * bandwidth-bound small-expert kernels (one launch per phase; their gate/up workgroups cover
 * 64 columns when max_rows_per_expert > 16, 16 otherwise), larger ones the tiled MFMA kernels;
 * a launch is skipped when the bounds show that no listed expert needs it (e.g.
 * min_rows_per_expert > 64).  list_rows (host, nullable) gives each list entry's row count:
 * list_rows[i] must equal n_e of expert_list[i] (within the two bounds).  The call then issues
 * the experts with 1-64 rows and then those with more as separate launches with exact bounds,
 * skips experts without rows, and gives the small experts' gate/up launch 64-column
 * workgroups for the experts with 17-64 rows (dispatched first) and 16-column ones for the
 * others.  The outputs are bit-identical to those of the same call without it; like the
 * bounds, the counts decide which launches run, so an entry below its expert's row count can
 * leave that expert uncomputed.
 * phases: 1 = gate/up projection + SwiGLU (writes act), 2 = down projection + routing weight
 * (reads act, writes out), 3 = both.  An expert's cache row (3 * H * I bf16) must be smaller
 * than 4 GiB.
 */
enum { FERRY_MAX_EXPERTS = 512 };
/* A call with phases = 3 whose experts all have at most 16 rows (decode, intermediate <= 2048)
 * runs both phases in one launch: an expert's down projection starts once its up projection is
 * stored, through arrival flags in a static device ring of 8 sets, one per call in turn.  Calls
 * on one GPU whose kernels run at the same time must number fewer than 8 (calls on one stream
 * never overlap); more would share a set and could leave outputs unwritten.
 * ferry_expert_ffn_sync_timeouts (a diagnostic with no counterpart in the reference) returns
 * how many waits of such launches on the current device gave up: each wait is bounded (about a
 * second), and the count stays 0 when workgroups are dispatched in index order, as the
 * hardware does.  A wait that gave up leaves its rows of `out` unwritten; ferry_history_update
 * copies the count where a caller reads its routing IDs, so that the caller can fail.
 * ferry_expert_ffn_set_sync_spin_limit (no counterpart in the reference) sets how often such a
 * wait polls before it gives up, for launches made after the call: limit < 0 restores the
 * default, 0 makes every wait give up at once (for tests of how a timeout is reported; every
 * workgroup still exits normally). */
int ferry_expert_ffn(const void* cache, int64_t cache_rows, int64_t hidden, int64_t inter,
                     const void* x, int64_t rows_in, int64_t topk, const void* w_sorted,
                     const int64_t* starts, const int64_t* rows, const int64_t* cols,
                     const int32_t* expert_list, int32_t n_list, const int32_t* slot_of,
                     int64_t experts, int64_t max_rows_per_expert,
                     int64_t min_rows_per_expert, const int32_t* list_rows, void* act, void* out,
                     int32_t out_mode, int32_t phases, void* stream);
int ferry_expert_ffn_sync_timeouts(int64_t* count);
int ferry_expert_ffn_set_sync_spin_limit(int64_t limit);

/*
 * Combine: out[t, :] = bf16( sum_{j<k} fp32(part[src(t, j), :]) ), j ascending (= ascending
 * expert ID).  src(t, j) = pair_pos[t*k+j] when pair_pos is non-null, else t*k+j.
 * Replaces ferry/csrc/expert_ops.cpp:75-92 (reduce_partials: fp32 index_add_ over experts in
 * ascending order, then bf16; scatter_returned: identity at world = 1).
 */
int ferry_combine(const void* part, const int32_t* pair_pos, int64_t tokens, int64_t topk,
                  int64_t hidden, void* out, void* stream);
/*
 * Combine plus a bf16 addend: out[t, :] = bf16( fp32(combine(t, :)) + fp32(addend[t, :]) ).
 * Replaces the DeepSeek-V2 block's `hidden_states + self.shared_experts(residuals)` (HF
 * transformers 4.57 DeepseekV2MoE, reached through ferry/model.py:150-157; the installed
 * analogue is transformers/models/deepseek_v2/modeling_deepseek_v2.py:130-137), fused into the
 * routed combine.  addend is bf16 [tokens, hidden].
 */
int ferry_combine_add(const void* part, const int32_t* pair_pos, int64_t tokens, int64_t topk,
                      int64_t hidden, const void* addend, void* out, void* stream);

/*
 * Dispatch packets (the reference's exchange format).  Replaces ferry/csrc/expert_ops.cpp:88-104
 * (pack_dispatch) and :106-111 (unpack_dispatch), called from ferry/transport.py:22-29.
 * Packet row i (2H + 3k bytes) = [hidden[send_idx[i]] (bf16 H) | packet weights (bf16 k) |
 * uint8(send_ids[i])], where packet weight j = bf16(sum of fp32(weights[t, q]) over the q with
 * selected[t, q] == send_ids[i, j]) for t = send_idx[i], times (send_ids[i, j] >= 0).
 * selected / weights are the router outputs [tokens, topk_selected]; send_idx [packets] and
 * send_ids [packets, topk] come from the layout; a packet whose send_idx is outside
 * [0, tokens) is left unwritten.  unpack_dispatch splits packet rows back into
 * hidden_out bf16 [packets, H] and weights_out bf16 [packets, topk].
 */
int ferry_pack_dispatch(const void* hidden, int64_t tokens, int64_t hidden_size,
                        const int64_t* selected, const void* weights_bf16, int64_t topk_selected,
                        const int64_t* send_idx, const int64_t* send_ids, int64_t packets,
                        int64_t topk, int64_t experts, void* payload, void* stream);
int ferry_unpack_dispatch(const void* payload, int64_t packets, int64_t hidden_size, int64_t topk,
                          void* hidden_out, void* weights_out, void* stream);

/*
 * Selection-frequency history on the device.  Replaces ferry/metadata.py:15-38 (GateHistory
 * update/scores over one-hot rows built by RouteGather.collect, ferry/metadata.py:67-83).
 * State per layer (device memory, caller-owned, zero-initialised):
 *   ring[L, W, k] int32, counts[L, E] int32, meta[L, 2] int32 (count, head).
 * Update with the last min(T, W) tokens of selected[T, k]; then scores_out[E] =
 * float32(count_e / max(1, n)).  ids_out (nullable, needs E <= 255) receives selected as
 * uint8 [T*k] (the D2H payload of the host planner), with 0xFF for an ID outside [0, E).
 * ffn_timeouts_out (nullable; no counterpart in the reference) receives the device's count of
 * fused decode FFN workgroups that gave up waiting (ferry_expert_ffn_sync_timeouts), as the
 * stream's earlier kernels left it: a caller that reads its routing IDs from host memory reads
 * this word with them and can fail the layer call instead of using unwritten rows.
 * ready_out (nullable, needs ids_out; no counterpart in the reference) receives ready_value in
 * each of its ferry_history_ready_words(T, k) int32 words, each with a system-scope release
 * after the launch's other writes of that word's workgroup: a caller whose outputs are in
 * coherent host memory can poll the words (ferry_h2d_wait_ready) instead of waiting for an
 * event behind the launch.
 */
int ferry_history_update(const int64_t* selected, int64_t tokens, int64_t topk, int64_t experts,
                         int64_t window, int64_t layer, int32_t* ring, int32_t* counts,
                         int32_t* meta, float* scores_out, uint8_t* ids_out,
                         int32_t* ffn_timeouts_out, int32_t* ready_out, int32_t ready_value,
                         void* stream);
/* Number of int32 ready words a ferry_history_update call with ids_out writes: one per
 * workgroup, 1 + ceil(tokens * topk / 4096); -1 for bad sizes. */
int64_t ferry_history_ready_words(int64_t tokens, int64_t topk);

/*
 * Host planner at world = 1.  Replaces ferry/policy.py:130-194 (plan_layer with
 * FERRY/RANDOM at world = 1, the quota check of ferry/quota.py:63) and :109-127
 * (_choose_slot).  State arrays are host memory owned by the caller:
 *   slots[cap], owner[L*E], last[L*E] int64; scores[L*E] float32.
 * Returns the number of misses m (fetches_out receives m rows of (0, key, slot) in ascending
 * expert order), or -1 with ferry_last_error() set when the misses exceed the admission
 * capacity, or -3 (state untouched) when an expert ID is outside [0, E) or repeated within a
 * token.  destinations_out (nullable) receives owner[layer*E + selected[t,j]].
 */
int64_t ferry_plan_layer(int64_t event, int64_t layer, const int64_t* selected, int64_t tokens,
                         int64_t topk, const float* gate_scores, int64_t* slots, int64_t cap,
                         int64_t* owner, int64_t* last, float* scores, int64_t experts,
                         int64_t* fetches_out, int64_t* destinations_out);
int64_t ferry_choose_slot(int64_t layer, const uint8_t* active, const int64_t* slots,
                          int64_t cap, const int64_t* last, const float* scores, int64_t experts);
/* ferry/policy.py:197-205 */
void ferry_layer_slots(const int64_t* slots, int64_t cap, int64_t layer, int64_t experts,
                       int64_t* lookup);

/*
 * H2D expert fetch engine.  Replaces the H2DEngine class of ferry/csrc/expert_ops.cpp:94-142.
 * The engine copies pool rows (pinned host memory) into cache slots on its own stream; a copy
 * into a slot first waits (GPU-side) for the last compute that read the slot.
 */
typedef struct ferry_h2d ferry_h2d;
int ferry_h2d_create(void* cache, int64_t cache_rows, const void* pool, int64_t pool_rows,
                     int64_t row_bytes, int32_t device, ferry_h2d** out);
int ferry_h2d_destroy(ferry_h2d* h);
/* expert_ops.cpp:107-117 */
int ferry_h2d_fetch(ferry_h2d* h, const int64_t* slots, const int64_t* keys, int64_t n);
/* expert_ops.cpp:119-122: host blocks until the slots' copies are done */
int ferry_h2d_wait_host(ferry_h2d* h, const int64_t* slots, int64_t n);
/* GPU-side variant: `stream` waits for the slots' copies without blocking the host */
int ferry_h2d_wait_stream(ferry_h2d* h, const int64_t* slots, int64_t n, void* stream);
/* expert_ops.cpp:124-128 */
int ferry_h2d_mark_used(ferry_h2d* h, const int64_t* slots, int64_t n, void* stream);
/* mark_used and an event in one record (no counterpart in the reference, which records one
 * event per mark_used): the slots count as read by the work enqueued on `stream` so far, and
 * *event_out is that one event, recorded with a system-scope release so that the host can wait
 * on it (ferry_h2d_event_synchronize) before reading what the stream's kernels wrote to host
 * memory.  A caller that reads the routing IDs back this way marks the slots of its previous
 * call without a second event on its stream.  n may be 0.  The engine owns the event; it stays
 * valid until the next ferry_h2d_mark_used_record call on the engine. */
int ferry_h2d_mark_used_record(ferry_h2d* h, const int64_t* slots, int64_t n, void* stream,
                               void** event_out);
int ferry_h2d_event_synchronize(ferry_h2d* h, void* event);
/* The host's wait for a kernel's host-memory results without the event's completion latency
 * (no counterpart in the reference, which synchronises its stream): spins until all n int32
 * words at `words` (coherent host memory) hold `value`.  The words must be written, after the
 * kernel's other writes, by a kernel queued on `event`'s stream after every read that `event`
 * marks -- as ferry_history_update's ready words are when it is called before
 * ferry_h2d_mark_used_record -- and `event` must be the engine's latest
 * ferry_h2d_mark_used_record event.  Those reads are then complete, so later copies into the
 * slots it marks do not wait for the event itself.  Queries the event every 1024 rounds:
 * returns 3 (error set) if the stream passed the event and the words still do not hold
 * `value`. */
int ferry_h2d_wait_ready(ferry_h2d* h, void* event, const int32_t* words, int64_t n,
                         int32_t value);
/* expert_ops.cpp:130-133 */
int ferry_h2d_synchronize(ferry_h2d* h);
/* The state of a new engine on the same streams and buffers (runtime.py:51-62 builds a new
 * H2DEngine on reset): waits for all of the engine's work and for every read of a slot marked
 * on a caller's stream (mark_used, mark_used_record), then forgets every slot's copies and
 * reads and zeroes the copy counter; DMA mode, the engine's own kernel stream, no deferred
 * unpack.  Reads that were never marked are the caller's to finish.  Keeping the streams keeps their hardware queues: a new engine's streams can land on
 * the queue of the caller's compute stream and serialise with it. */
int ferry_h2d_reset(ferry_h2d* h);
/* expert_ops.cpp:135 */
int64_t ferry_h2d_copies(const ferry_h2d* h);
/* The last fetch call's groups of rows that become ready together (no counterpart in the
 * reference, which waits for all of a call's copies at once): with a packed pool in DMA mode
 * its sub-batches, each unpacked as soon as its copies land, otherwise one group.  Writes the
 * groups' ends (positions in the call's slot list, exclusive, ascending) into ends[0..max) and
 * returns the number of groups (0 after an empty call or a reset; -1 on bad arguments).  A
 * caller can wait for and compute each group's experts while the later groups still copy. */
int64_t ferry_h2d_groups(const ferry_h2d* h, int64_t* ends, int64_t max_groups);
/* the engine's copy stream (for event timing by the caller): after a fetch call its queue ends
 * with the call's copies -- the first DMA lane, which the others join, or, with a packed pool
 * attached, the stream that runs the unpacks */
void* ferry_h2d_stream(ferry_h2d* h);
/* How the engine copies (no counterpart in the reference, whose engine always issues one
 * cudaMemcpyAsync per row).  FERRY_H2D_DMA (the default): hipMemcpyAsync on two DMA streams,
 * each taking half of the call's bytes.  FERRY_H2D_KERNEL: one launch of a copy kernel per
 * fetch call that reads the pool through its device mapping (possible when the pool has one
 * and rows are 16-byte multiples).
 * Both write the same bytes, and a copy into a slot is ordered after the earlier copies into
 * that slot, of either kind, that are still in flight.  ferry_h2d_set_kernel_stream picks the stream that kernel-mode
 * copies run on (initially the engine's own, ferry_h2d_stream; null is HIP's null stream):
 * with the caller's compute stream, the
 * kernels that read the fetched rows follow the copy on one queue, with no cross-queue wait.
 * The copy kernel slows HBM-bound kernels that run beside it (its host reads hold memory
 * resources for the link's latency), so callers use it where little compute overlaps the copy.
 */
enum { FERRY_H2D_DMA = 0, FERRY_H2D_KERNEL = 1 };
int ferry_h2d_set_engine(ferry_h2d* h, int32_t kind);
/* Deferred last unpack (no counterpart in the reference; packed pools in DMA mode): with `on`,
 * the unpack of a fetch call's last sub-batch is not queued on the engine's unpack stream but
 * by the first ferry_h2d_wait_stream that names one of its slots, on the waiting stream, right
 * after its wait for the copies -- the reader then follows the last copies with one cross-queue
 * wait instead of two.  Any other engine call (fetch, wait_host, synchronize, ...) first queues
 * a pending deferred unpack on the unpack stream.  Off by default. */
int ferry_h2d_set_defer_last(ferry_h2d* h, int32_t on);
int32_t ferry_h2d_engine(const ferry_h2d* h);
int ferry_h2d_set_kernel_stream(ferry_h2d* h, void* stream);
/* Lossless packing of the pool for the host link (no counterpart in the reference, whose
 * engine copies raw bf16 rows).  ferry_pack_pool copies every pool row into pinned host memory,
 * in a packed form where it shrinks: per value one byte sign | mantissa and a 2-bit exponent
 * code against the row's 3 most populated exponents; the escapes' exponents follow as 2-bit
 * codes against the next 3, theirs as 4-bit codes against a window of 15, and the rest in an
 * (index, exponent) list (about 10.7 bits per value for weights that span few binades); a row
 * that would not shrink is copied raw.  Rows hold a multiple of 32 values.  It reads the pool
 * (pinned or pageable host memory, not changed afterwards) on `threads` host threads; the
 * packed pool then stands alone.  An engine made from it (ferry_h2d_create_packed) or given it
 * (ferry_h2d_use_packed, an engine of the same pinned pool; null detaches it) fetches in DMA
 * mode: packed rows go into `ring_rows` device staging buffers it allocates, and an unpack
 * kernel writes the slots -- the slot bytes are exactly the pool row's.  A call is fetched in
 * sub-batches of about 4 MiB, each unpacked on a stream of its own while the DMA lanes copy the
 * next.  In kernel mode (ferry_h2d_set_engine) the unpack kernel reads the packed rows over the
 * link through the packed pool's device mapping, with no staging.  A packed pool outlives the
 * engines that use it. */
typedef struct ferry_packed_pool ferry_packed_pool;
int ferry_pack_pool(const void* pool, int64_t rows, int64_t row_bytes, int32_t threads,
                    ferry_packed_pool** out);
int ferry_packed_pool_stats(const ferry_packed_pool* pp, int64_t* packed_bytes,
                            int64_t* packed_rows);
int ferry_packed_pool_destroy(ferry_packed_pool* pp);
int ferry_h2d_use_packed(ferry_h2d* h, const ferry_packed_pool* pp, int64_t ring_rows);
int ferry_h2d_create_packed(void* cache, int64_t cache_rows, const ferry_packed_pool* pp,
                            int32_t device, int64_t ring_rows, ferry_h2d** out);
/* The packing of one row of n bf16 values (n a multiple of 32) into dst (cap bytes; null to
 * query the size): 0, or 1 when the row would not shrink (dst untouched); *bytes_out is the
 * packed size.  For tests and tools; the engine packs its pool itself. */
int ferry_pack_row(const void* src, int64_t n, void* dst, int64_t cap, int64_t* bytes_out);

/*
 * Plan one layer call and enqueue its fetch in one host call: the steps of ferry/runtime.py:64-89
 * between the routing read-back and the expert computation (policy.plan_layer of
 * ferry/policy.py:130-194, then H2DEngine.fetch of ferry/h2d.py / expert_ops.cpp:94-142).
 * ids are the routing IDs as uint8 [tokens*topk] and gate_scores the layer's float32 scores,
 * e.g. straight from the mapped staging buffer that ferry_history_update writes; the other
 * arguments are those of ferry_plan_layer, plus demand_out (nullable: int64 [experts], each
 * expert's (token, expert) pair count in this call, as the planner counts them anyway) and the
 * fetch engine (nullable: plan only).
 * Returns the number of misses m (fetches_out rows as in ferry_plan_layer, their copies queued),
 * -1 when the misses exceed the admission capacity, -2 when the fetch fails, -3 when an ID is
 * outside [0, E) (0xFF from ferry_history_update) or repeated within a token; errors set
 * ferry_last_error().
 */
int64_t ferry_plan_fetch(int64_t event, int64_t layer, const uint8_t* ids, int64_t tokens,
                         int64_t topk, const float* gate_scores, int64_t* slots, int64_t cap,
                         int64_t* owner, int64_t* last, float* scores, int64_t experts,
                         int64_t* fetches_out, int64_t* destinations_out, int64_t* demand_out,
                         ferry_h2d* h2d);

#ifdef __cplusplus
}
#endif

#endif /* FERRY_AMD_H */
