/*
 * lrmoe.h -- C ABI of liblrmoe.so, the MI355X (gfx950) kernels for the MoE
 * expert-layer hot path of the Qwen3.6-35B-A3B runner.
 *
 * Conventions (every entry point):
 *   - plain device pointers and sizes, no framework types;
 *   - bf16 tensors are passed as uint16_t bit patterns, row-major, contiguous;
 *   - `stream` is a hipStream_t (NULL = the null stream); work is enqueued on
 *     it and the call returns without a host synchronisation, so calls can be
 *     captured into a HIP graph and replayed;
 *   - the return value is 0 on success, a negative LRMOE_E_* code for misuse
 *     detected on the host (nothing is launched), or a positive hipError_t;
 *   - the library never allocates: scratch comes from a caller-provided
 *     `workspace` of at least lrmoe_workspace_bytes(tokens) bytes, zeroed once
 *     by the caller after allocation (its counters reset themselves), and used
 *     on one device by one stream at a time (calls that overlap on one
 *     workspace race);
 *   - route problems found on the device (an expert id outside [0, 256) or a
 *     token routed twice to one expert) set bits in the int32 status word at
 *     byte offset LRMOE_WS_STATUS_OFFSET of the workspace; the affected call
 *     then writes zeros (plus the residual, where one is given) instead of
 *     reading out of bounds;
 *   - the decode layer and chain (lrmoe_moe_layer and lrmoe_moe_experts at
 *     tokens <= 16, lrmoe_moe_chain) run one
 *     persistent workgroup per CU whose workgroups wait for each other's
 *     results, so all of them must be resident at once: a kernel running
 *     concurrently on another stream of the same device can keep some of
 *     them off the GPU.  Every such wait is bounded (50 ms); on expiry the
 *     call still ends, sets LRMOE_STATUS_TIMEOUT in the status word, and
 *     its outputs are invalid.  Callers that share the device with other
 *     streams read the status word after such calls;
 *   - the prefill expert stage (tokens > 16) is one launch whose workgroups
 *     claim work items from counters, down items after the gate/up items
 *     they read; a claimed gate/up item never waits, so its waits end
 *     whether or not every workgroup is resident, and they are bounded in
 *     the same way.
 *
 * Fixed model shape: hidden 2048, 256 routed experts, top-8, expert
 * intermediate 512, one shared expert with intermediate 512.  A routed
 * expert's weights are gate_up [1024, 2048] (gate rows 0-511, up rows
 * 512-1023) and down [2048, 512]; `expert_ptrs` is a device array of 256
 * (gate_up, down) address pairs, so the expert banks can live anywhere in HBM
 * (e.g. 40 layers x 256 experts in one allocation, the "packed pair" layout).
 */
#ifndef LRMOE_H
#define LRMOE_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define LRMOE_HIDDEN 2048
#define LRMOE_INNER 512
#define LRMOE_EXPERTS 256
#define LRMOE_TOPK 8

#define LRMOE_OK 0
#define LRMOE_E_ARG (-1)        /* null pointer, bad size or shape */
#define LRMOE_E_WORKSPACE (-2)  /* workspace smaller than lrmoe_workspace_bytes(tokens) */
#define LRMOE_E_DEVICE (-3)     /* current device is not gfx950 */

#define LRMOE_WS_STATUS_OFFSET 4  /* int32 route status word in the workspace */
#define LRMOE_STATUS_BAD_EXPERT 1
#define LRMOE_STATUS_REPEATED_EXPERT 2
#define LRMOE_STATUS_CODEC_ROW 4
#define LRMOE_STATUS_TIMEOUT 8  /* a bounded cross-workgroup wait expired: the call's outputs are invalid */

/* Library version string.  No reference counterpart. */
const char *lrmoe_version(void);

/* Human-readable text for a return code.  Replaces the status checks of
 * edge35b/native_bf16_gather.py:25-29 (_checked) and packed_ada.py:10-12. */
const char *lrmoe_error_string(int code);

/* 0 when the current HIP device is gfx950, else LRMOE_E_DEVICE (or a
 * hipError_t).  Replaces the capability gate of
 * edge35b/native_bf16_gather.py:37-38 and packed_ada.py:17-18. */
int lrmoe_device_check(void);

/* Bytes of workspace a call with `tokens` tokens needs.  No reference
 * counterpart (the reference allocates per call, e.g. block_experts.py:123-134). */
size_t lrmoe_workspace_bytes(int tokens);

/* Router: logits = bf16(x W^T) in a fixed fp32 reduction order, softmax over
 * 256 experts in fp32, top-8 by (logit desc, id asc), renormalised in fp32,
 * weights rounded to bf16; optionally RMSNorm (x*r)*(1+w) of `hidden` first
 * (norm_weight != NULL) and the shared-expert gate bf16(sigmoid(bf16(x.w))).
 * Exactly one of router_weight and logits_in is given: with logits_in
 * [tokens, 256] bf16 the GEMV is skipped and top-k runs on those logits.
 * Also leaves the route plan in the workspace.
 * Replaces Transformers Qwen3_5MoeTopKRouter.forward (modeling_qwen3_5_moe.py,
 * called from SparseMoeBlock.forward), whose outputs edge35b/expert_stream.py:383
 * (_Layer.forward) receives; RMSNorm replaces Qwen3_5MoeRMSNorm.forward. */
int lrmoe_route_topk(const uint16_t *hidden, int tokens, const uint16_t *router_weight,
                     const uint16_t *logits_in, const uint16_t *norm_weight, float eps, const uint16_t *shared_expert_gate,
                     uint16_t *logits_out, int64_t *indices_out, uint16_t *weights_out,
                     uint16_t *shared_gate_out, uint16_t *normed_out, void *workspace,
                     size_t workspace_bytes, void *stream);

/* Token-to-expert bucketing of indices [tokens, 8]: unique experts ascending
 * (expert[0..unique)), pair offsets (offset[0..unique]), pairs in (expert asc,
 * token asc) order (pair_token, pair_slot), and route_pair[t*8 + r] = pair of
 * token t's r-th route in ascending expert order.  unique and status are
 * single int32 device words.  Replaces edge35b/block_experts.py:102-121,
 * fused_experts.py:47-54 (T=1 schedule), pipeline.py:59-76 (_routes) and
 * packed_workers.cpp:102-113 (packed_plan), all of which run on the host after
 * a device-to-host read of the indices. */
int lrmoe_bucket(const int64_t *indices, int tokens, int32_t *expert, int32_t *offset,
                 int32_t *pair_token, int32_t *pair_slot, int32_t *route_pair, int32_t *unique,
                 int32_t *status, void *workspace, size_t workspace_bytes, void *stream);

/* Routed experts for given routes: out[t] = sum over t's routes in ascending
 * expert order of bf16(y * w), y = SwiGLU expert output with cpu_experts.c's
 * rounding points.  hidden [T,2048], indices [T,8] int64, weights [T,8] bf16.
 * Replaces the experts forward the reference patches
 * (edge35b/expert_stream.py:383-454 _Layer.forward, i.e. Transformers
 * Qwen3_5MoeExperts.forward) and its modes fused_experts.fused_forward
 * (fused_experts.py:40-70), block_experts.grouped_block (:89-139),
 * pipeline.routed_forward (:79-110) and cpu_route.cpu_forward (:23-69). */
int lrmoe_moe_experts(const uint16_t *hidden, int tokens, const int64_t *indices,
                      const uint16_t *weights, const int64_t *expert_ptrs, uint16_t *out,
                      void *workspace, size_t workspace_bytes, void *stream);

/* Whole sparse MoE block: router + top-k + bucketing, routed experts, ordered
 * combine, shared expert scaled by its sigmoid gate.  With norm_weight:
 * out = bf16(hidden + MoE(RMSNorm(hidden))) (the decoder layer's MLP half);
 * without: out = MoE(hidden).  Shared expert pointers may all be NULL.
 * Exactly one of router_weight and logits_in is given (see lrmoe_route_topk).
 * indices_out / weights_out may be NULL.  expert_codec (may be NULL; 16-byte
 * aligned) is a device table [257][LRMOE_CODEC_TABLE_COLUMNS] int64, row 256
 * the shared expert (whose packed gate_up is gate_proj then up_proj): four
 * tile-codec addresses (packed gate_up, packed down, gate_up bases, down
 * bases, as written by lrmoe_codec_pack), then 48 bytes of raw flags: byte
 * i < 32 for gate_up item i, byte 32 + i for down item i, bit w set when a
 * tile that wave w of the item reads has base 255 (gate_up item i, wave w:
 * tiles 2(w%4), 2(w%4)+1 of gate_proj and up_proj rows 16i + 8(w/4) .. +7;
 * down item i, wave w: both tiles of rows 128i + 16w .. +15).  For 8 <=
 * tokens <= 16 an expert whose four addresses are non-zero is read from its
 * codec form, tile by tile, with the raw row's tile where a tile's base is
 * 255; fewer tokens read the raw rows (too few items per workgroup for the
 * codec to pay).  Results are identical to the raw rows' either way.  The
 * raw pointers stay required.
 * Replaces Transformers
 * Qwen3_5MoeSparseMoeBlock.forward + the residual add of
 * Qwen3_5MoeDecoderLayer.forward, as driven by edge35b/expert_stream.py:457-526
 * (patch_experts). */
int lrmoe_moe_layer(const uint16_t *hidden, int tokens, const uint16_t *router_weight,
                    const uint16_t *logits_in, const int64_t *expert_ptrs, const int64_t *expert_codec,
                    const uint16_t *shared_gate_proj,
                    const uint16_t *shared_up_proj, const uint16_t *shared_down_proj,
                    const uint16_t *shared_expert_gate, const uint16_t *norm_weight, float eps,
                    uint16_t *out, int64_t *indices_out, uint16_t *weights_out, void *workspace,
                    size_t workspace_bytes, void *stream);

/* lrmoe_moe_layer for decode sizes (1 <= tokens <= LRMOE_STATIC_MAX_TOKENS)
 * without a workspace: no counterpart in the reference.  For callers that
 * cannot allocate (code under HIP graph capture, tight serving loops,
 * harnesses that forbid hipMalloc).  Same arguments and results as
 * lrmoe_moe_layer, minus the workspace; the route status word (the
 * LRMOE_STATUS_* bits of that call) goes to *status_out when status_out (a
 * device int32) is given.  Its scratch (3 MiB: counters and tagged rows) is
 * a static device array of the library, one per GPU, held until the process
 * ends, zero-filled when the library's code object is loaded; the first
 * call on a GPU looks up its address and, unless that call's stream is
 * capturing a graph, zeroes it again with a kernel on that stream (a first
 * call under capture records no clear).  Every call on a GPU shares that GPU's
 * array: calls that overlap on one GPU (two streams, or two host threads)
 * race, as calls sharing one workspace do.  Calls nothing that allocates.
 * Returns LRMOE_E_ARG for tokens > LRMOE_STATIC_MAX_TOKENS. */
#define LRMOE_STATIC_MAX_TOKENS 16
int lrmoe_moe_layer_static(const uint16_t *hidden, int tokens, const uint16_t *router_weight,
                           const uint16_t *logits_in, const int64_t *expert_ptrs, const int64_t *expert_codec,
                           const uint16_t *shared_gate_proj, const uint16_t *shared_up_proj,
                           const uint16_t *shared_down_proj, const uint16_t *shared_expert_gate,
                           const uint16_t *norm_weight, float eps, uint16_t *out, int64_t *indices_out,
                           uint16_t *weights_out, int32_t *status_out, void *stream);

/* Several MoE decode layers (tokens <= 16) chained in one persistent launch:
 * h_0 = hidden, h_{l+1} = MoE layer l applied to h_l exactly as
 * lrmoe_moe_layer with that layer's router and weights, out = h_layers
 * (out must not overlap hidden).  layer_table is a HOST array
 * [layers][LRMOE_CHAIN_PTRS] of device addresses per layer, in the order of
 * the LRMOE_CHAIN_* indices below: the router (required), the expert
 * address table (required), the shared expert's gate_proj, up_proj,
 * down_proj and shared_expert_gate (all four or none), the RMSNorm weight
 * (0 = no norm and no residual add), and the tile-codec table (0 = none;
 * see lrmoe_moe_layer's expert_codec).  The table is
 * copied into the launch, so it may be freed or changed once the call has
 * returned (also while a stream is captured).  layers <=
 * LRMOE_CHAIN_MAX_LAYERS; longer stacks take several calls.  indices_out /
 * weights_out may be NULL, else [layers][T][8].  Replaces the MoE halves of
 * the 40 Qwen3_5MoeDecoderLayer.forward calls of one decode step ([HF]
 * 834-875: the post-attention RMSNorm 801-818, Qwen3_5MoeSparseMoeBlock.forward
 * 787-798, the residual add 875), which the reference replays as one
 * captured graph per step (edge35b/packed_native.py:58-63). */
#define LRMOE_CODEC_TABLE_COLUMNS 10
#define LRMOE_CHAIN_PTRS 8
#define LRMOE_CHAIN_MAX_LAYERS 48
#define LRMOE_CHAIN_ROUTER 0
#define LRMOE_CHAIN_EXPERTS 1
#define LRMOE_CHAIN_SHARED_GATE_PROJ 2
#define LRMOE_CHAIN_SHARED_UP_PROJ 3
#define LRMOE_CHAIN_SHARED_DOWN_PROJ 4
#define LRMOE_CHAIN_SHARED_EXPERT_GATE 5
#define LRMOE_CHAIN_NORM 6
#define LRMOE_CHAIN_CODEC 7
int lrmoe_moe_chain(const uint16_t *hidden, int tokens, int layers, const int64_t *layer_table, float eps,
                    uint16_t *out, int64_t *indices_out, uint16_t *weights_out, void *workspace,
                    size_t workspace_bytes, void *stream);

/* Lossless BF16 tile codec (the format of the reference's tile packer,
 * edge35b/cpu_bf16_reads.h:16-52 pack_cpu_read_tiles, decoded by
 * bf16_gather_ada.cu:117-123; bytes reordered for the decode kernel's MFMA
 * lanes, see lightreason_amd/csrc/codec.hip).  w is [rows][cols] bf16 with
 * cols a multiple of 256; packed receives rows * cols / 256 tiles of 384
 * bytes and bases one byte per tile (255: the tile's exponent fields span
 * more than 8 values and it is not encoded).  *misfit (device, may be NULL)
 * is increased by the number of such tiles.  Replaces the packing that
 * edge35b/gpu_resident_experts.py:29 and cpu_read_packing.py:138 run on the
 * host. */
int lrmoe_codec_pack(const uint16_t *w, int64_t rows, int cols, uint8_t *packed, uint8_t *bases,
                     unsigned long long *misfit, void *stream);
/* Inverse of lrmoe_codec_pack (tiles with base 255 decode to 0xffff). */
int lrmoe_codec_unpack(const uint8_t *packed, const uint8_t *bases, int64_t rows, int cols, uint16_t *w,
                       void *stream);

/* BF16 row gather: for row < *count and bank b < banks, fill sizes[b] bytes
 * at destinations[b] + dst_ids[row]*sizes[b] from the descriptor
 * descriptors[(b*experts + src_ids[row])*3] = (address, base, escapes).
 * base < 0: a raw row, copied.  base >= 0: an escape-codec row of n =
 * sizes[b]/2 values (edge35b/bf16_expert_codec.py pack_row): n sign|fraction
 * bytes, n/2 bytes of 4-bit exponent deltas from base, then `escapes` sorted
 * int32 indices and their raw 16-bit values; it is decoded, and
 * LRMOE_STATUS_CODEC_ROW is or-ed into *status (may be NULL).  Grid
 * (stripes, banks, max_copies) of `threads` (64, 128, 192 or 256) threads;
 * keep_in_l2 = 0 streams the rows with nontemporal accesses, 1 uses cached
 * accesses (the reference geometries' "default" and "l2" policies).  Sizes
 * and addresses are multiples of 16 bytes.  Replaces
 * edge35b/bf16_gather_ada.cu:36-112 (gather_bf16, gather_bf16_l2) launched by
 * native_bf16_gather.py:71-77 (NativeBf16Gather.copy), and the staging copy
 * of scheduled_graph.py:14-26 (_stage). */
int lrmoe_gather(const int64_t *descriptors, const int64_t *destinations, const int64_t *sizes,
                 const int32_t *src_ids, const int32_t *dst_ids, const int64_t *count, int experts,
                 int banks, int max_copies, int stripes, int threads, int keep_in_l2, int32_t *status,
                 void *stream);

/* Tile-codec row gather, the launch protocol of lrmoe_gather: descriptors
 * [banks][experts][3] = (packed, bases, raw).  bases == 0: copy sizes[b]
 * bytes from raw.  Otherwise, per 512-byte tile t of the row, in the
 * reference's tile format and byte order (cpu_bf16_reads.h:16-52: value k's
 * low byte at byte k, its 4-bit code in nibble k of bytes 256..383): base
 * bases[t], 384 packed bytes at packed + 384t, decoded; base 255: the tile is
 * copied from raw + 512t.  With compact != 0, a descriptor whose raw is -1 is
 * a compact row: bases holds uint32 headers (raw tiles before t) << 8 | base
 * and tile t's bytes (512 for a raw tile) start at packed + 384t + 128 * (raw
 * tiles before t).  sizes[b] a multiple of 512.  Replaces
 * edge35b/bf16_gather_ada.cu:127-201 (gather_bf16_cpu_tiles, and
 * gather_bf16_resident with compact), launched by native_bf16_gather.py:71-77
 * with the "cpu-tiles" / "resident" policies. */
int lrmoe_gather_tiles(const int64_t *descriptors, const int64_t *destinations, const int64_t *sizes,
                       const int32_t *src_ids, const int32_t *dst_ids, const int64_t *count, int experts, int banks,
                       int max_copies, int stripes, int threads, int compact, void *stream);

/* Batched matvec with the _matvec protocol: for e < experts and r < N,
 * result[e*N + r] = bf16(sum_k W_e[r,k] x_e[k]), W_e = table[stride*e + column]
 * (rows skipped when that address is 0 and stride != 3), x_e = x when
 * shared_x else x + e*K.  K must be a multiple of 512.
 * Replaces edge35b/fused_experts.py:8-24 (_matvec), launched at
 * fused_experts.py:60,67, packed_hybrid.py:71-74, packed_native.py:49-52. */
int lrmoe_matvec(const int64_t *table, const uint16_t *x, uint16_t *result, int K, int N, int column,
                 int shared_x, int stride, int experts, void *stream);

/* Ordered combine over the 8 table rows: out[h] = bf16 running sum of
 * bf16(v_r[h] * router[table[stride*r + 2]]); v_r = hot[r] unless stride == 4,
 * cold != NULL and table[4r + 3] >= 0, then cold[table[4r + 3]].
 * Replaces edge35b/fused_experts.py:27-37 (_ordered_sum) and
 * packed_hybrid.py:13-27 (_combine). */
int lrmoe_ordered_sum(const int64_t *table, const uint16_t *hot, const uint16_t *cold,
                      const uint16_t *router, uint16_t *out, int stride, void *stream);

/* active[e*512 + r] = bf16(bf16(silu(bf16(g))) * bf16(u)) for the table rows
 * whose gate_up address (table[stride*e]) is non-zero.
 * Replaces edge35b/packed_ada.cu:13-40 (packed_gate_silu), loaded by
 * packed_ada.py:15-66 (load_gate). */
int lrmoe_gate_silu(const int64_t *table, const uint16_t *hidden, uint16_t *active, int stride,
                    int experts, void *stream);

/* Grouped projection with the _project protocol: for expert e < experts and
 * route row r < 16, Y[(e*16 + r)*out + c] = bf16(sum_k X[row][k] W[c][k]),
 * W = pointers[2e + down], row = e*16 + r (down) or routes[e*16 + r]
 * (otherwise); routes < 0 read zeros.  in and out must be multiples of 256
 * and 64.  Replaces edge35b/block_experts.py:12-28 (_project). */
int lrmoe_project(const int64_t *pointers, const int32_t *routes, const uint16_t *X, uint16_t *Y,
                  int in, int out, int down, int experts, void *stream);

/* active[r][c] = bf16(bf16(silu(g)) * u), g = gates[r][c], u = gates[r][512 + c]
 * for rows r < rows.  Replaces the torch act_fn(gate) * up between the two
 * _project launches (edge35b/block_experts.py:131-132, fused_experts.py:61-62). */
int lrmoe_swiglu_rows(const uint16_t *gates, uint16_t *active, int rows, void *stream);

/* The decoder layer's glue around its mixer, per token row of x
 * [tokens][2048] bf16: s = bf16(x + add) elementwise when add is given (the
 * residual add after the mixer, [HF] Qwen3_5MoeDecoderLayer.forward 866:
 * hidden = residual + mixer output), else s = x; sum_out (requires add)
 * receives s; with norm_weight [2048], norm_out receives RMSNorm(s) =
 * bf16(s rsqrt(mean(s^2) + eps) (1 + w)) (the input_layernorm before the
 * mixer, Qwen3_5MoeRMSNorm [HF] 801-818, in the canonical summation order of
 * the router and decode kernels, so the rows equal lrmoe_route_topk's
 * normed_out bit for bit).  norm_weight and norm_out come together; at least
 * one of sum_out, norm_out is given.  Every pointer 16-byte aligned.  No
 * reference counterpart as a kernel: the reference runs these as torch ops
 * inside the stock decoder layer. */
int lrmoe_add_rmsnorm(const uint16_t *x, const uint16_t *add, int tokens, const uint16_t *norm_weight, float eps,
                      uint16_t *sum_out, uint16_t *norm_out, void *stream);

/* Per-token ordered combine through inverse [tokens][8][3] = (expert, row,
 * slot): out[t][h] = bf16 running sum of bf16(v * router[t*8 + slot]),
 * v = X[(expert*16 + row)][h], or cold[row][h] when hybrid and expert < 0.
 * Replaces edge35b/block_experts.py:31-49 (_combine). */
int lrmoe_block_combine(const int32_t *inverse, const uint16_t *X, const uint16_t *cold,
                        const uint16_t *router, uint16_t *out, int tokens, int hybrid, void *stream);

/* Synthetic bf16 ~N(0, sigma) from a counter-based generator: element i is a
 * function of (seed, stream_id, first + i) only.  No reference counterpart
 * (the reference draws torch.randn weights, probe_experts.py:69). */
int lrmoe_fill_normal_bf16(uint16_t *out, int64_t count, uint64_t seed, uint64_t stream_id,
                           double sigma, int64_t first, void *stream);

/* Measurement support, no reference counterpart (the reference brackets
 * stages with CUDA events in Python, e.g. benchmark_packed_gather8.py:168-178).
 * lrmoe_timing_enable(mask, launches) brackets every launch of the stages in
 * `mask` (LRMOE_STAGE_* bits) with a pair of HIP events on its stream, room
 * for `launches` launches per stage; mask 0 turns timing off.  Do not enable
 * it while a stream is being captured.  lrmoe_timing_collect(stage, ...)
 * synchronises on those events and returns the summed milliseconds and the
 * launch count, then rewinds. */
#define LRMOE_STAGE_ROUTE 1
#define LRMOE_STAGE_GATE_UP 2      /* the prefill expert launch (gate/up and down items, tokens > 16) */
#define LRMOE_STAGE_DOWN 4         /* kept for the mask layout: no launch is timed under it */
#define LRMOE_STAGE_COMBINE 8
#define LRMOE_STAGE_GATHER 16
#define LRMOE_STAGE_LAYER 32       /* lrmoe_moe_layer / lrmoe_moe_chain decode kernel */
#define LRMOE_STAGE_DELTA_MIXER 64 /* lrmoe_delta_mixer (one launch) */
#define LRMOE_STAGE_DELTA_RULE 128 /* lrmoe_delta_rule */
#define LRMOE_STAGE_ATTENTION 256  /* lrmoe_attn_decode (first to last of its launches) */
int lrmoe_timing_enable(int mask, int launches);
int lrmoe_timing_collect(int stage, double *total_ms, int *launches);

/* Measurement support, no reference counterpart: the best time of `reps`
 * launches of a read-only stream kernel over `bytes` (a multiple of 16) at
 * the device address `src` (16-byte nontemporal loads, nothing written but
 * possibly the 4-byte device word `sink`), in *best_ms.  Synchronises on
 * the stream.  bytes / best_ms is the HBM read rate a weight-streaming
 * kernel can reach on this device. */
int lrmoe_read_bandwidth(const void *src, int64_t bytes, int reps, uint32_t *sink, double *best_ms, void *stream);

/* ---- Gated DeltaNet decode (the linear-attention mixer before each of the
 * 30 linear-attention layers' MoE) ------------------------------------------ */

/* The gated delta rule over a block of `tokens` tokens and `heads` heads,
 * the recurrence of edge35b/delta_decode.py:11-36 (_delta) with the calling
 * convention of :38-55 (_run): q, k [tokens][heads][key_width] bf16 (value
 * head h reads q/k head h; repeat grouped key heads before the call),
 * v [tokens][heads][value_width] bf16, G [tokens][heads] fp32 = exp(g),
 * beta [tokens][heads] bf16, initial [heads][key_width][value_width] fp32
 * (state_bf16 = 0) or bf16.  normalize != 0 applies l2norm to q and k first
 * (Transformers l2norm on bf16: every step rounded).  Per token and head:
 * state *= G; delta = (v - state^T k) beta; state += k delta^T;
 * out = bf16(state^T q / sqrt(key_width)); the state is rounded to its dtype
 * after every token.  record != 0: states [tokens][heads][kw][vw] receives
 * the state after every token; else states [heads][kw][vw] the final state
 * (states may equal initial then: updated in place).  key_width 64, 128 or
 * 256, value_width a multiple of 16; q, k 16-byte aligned (8 for width 64),
 * v and out 8-byte, initial and states 16-byte aligned. */
int lrmoe_delta_rule(const uint16_t *q, const uint16_t *k, const uint16_t *v, const float *G, const uint16_t *beta,
                     const void *initial, int state_bf16, int tokens, int heads, int key_width, int value_width,
                     int normalize, int record, uint16_t *out, void *states, void *stream);

/* Bytes of workspace lrmoe_delta_mixer needs for `tokens` tokens (1..16;
 * 0 outside that range).  No reference counterpart. */
#define LRMOE_DELTA_MAX_TOKENS 16
size_t lrmoe_delta_workspace_bytes(int tokens);

/* One cached step of the Gated DeltaNet mixer of the 35B model (hidden 2048,
 * 16 key heads and 32 value heads of width 128, conv kernel 4) for 1..16
 * tokens that follow the cached state: [HF] Qwen3_5MoeGatedDeltaNet.forward
 * 430-543 with cache_params holding a previous state, the short-block path
 * that edge35b/delta_decode.py:84-126 (fused_delta) routes through its
 * _delta kernel, and the single-token step that edge35b/packed_native.py:
 * 96-149 (mixer_graphs) replays.  Weights as the module holds them, bf16:
 * in_proj_qkv [8192][2048], in_proj_z [4096][2048], in_proj_b and in_proj_a
 * [32][2048], conv_weight [8192][4] (conv1d.weight without its middle
 * axis), A_log, dt_bias [32], norm_weight [128], out_proj [2048][4096].
 * conv_state [8192][4] bf16 and state [32][128][128] (fp32, or bf16 when
 * state_bf16) are updated in place.  conv_record [tokens][8192][4] and
 * state_record [tokens][32][128][128] (may be NULL) receive both states
 * after every token, for rolling back to an accepted prefix.  out
 * [tokens][2048] bf16.  Workspace of lrmoe_delta_workspace_bytes(tokens),
 * 256-byte aligned, zeroed once after allocation (its counters never need
 * a reset), used by one stream at a time.  One persistent launch of 256
 * workgroups, one per CU, which wait for flags that other workgroups set:
 * all must be resident (a device with fewer than 256 CUs gets
 * hipErrorNotSupported; a kernel running on another stream can keep some
 * off the GPU).  Waits are bounded (50 ms); on expiry the call still ends,
 * sets LRMOE_STATUS_TIMEOUT in the int32 status word at byte offset
 * LRMOE_DELTA_WS_STATUS_OFFSET of the workspace, and its outputs are
 * invalid.  Rounding points: those of the Transformers forward in bf16
 * (see lrmoe_delta_rule for the recurrence). */
#define LRMOE_DELTA_WS_STATUS_OFFSET 0
int lrmoe_delta_mixer(const uint16_t *hidden, int tokens, const uint16_t *in_proj_qkv, const uint16_t *in_proj_z,
                      const uint16_t *in_proj_b, const uint16_t *in_proj_a, const uint16_t *conv_weight,
                      const uint16_t *A_log, const uint16_t *dt_bias, const uint16_t *norm_weight, float eps,
                      const uint16_t *out_proj, uint16_t *conv_state, void *state, int state_bf16,
                      uint16_t *conv_record, void *state_record, uint16_t *out, void *workspace,
                      size_t workspace_bytes, void *stream);

/* The linear-attention half of a decoder layer in one call: [HF]
 * Qwen3_5MoeDecoderLayer.forward 834-875 runs residual -> input_layernorm
 * (Qwen3_5MoeRMSNorm 801-818) -> the mixer -> residual + mixer output as
 * three torch steps; here `residual` [tokens][2048] bf16 is the layer's
 * input, normed inside the mixer launch with input_norm [2048] (applied as
 * 1 + w) and input_eps, bit for bit as lrmoe_add_rmsnorm would write it;
 * out receives the mixer output as from lrmoe_delta_mixer on those normed
 * rows, and sum_out [tokens][2048] bf16(residual + out).  norm_out, when
 * not NULL, receives the normed rows.  sum_out may be residual itself.  No
 * reference counterpart as one call: it saves the two glue launches per
 * layer.  Other arguments, workspace and status as lrmoe_delta_mixer's. */
int lrmoe_delta_mixer_step(const uint16_t *residual, int tokens, const uint16_t *input_norm, float input_eps,
                           const uint16_t *in_proj_qkv, const uint16_t *in_proj_z, const uint16_t *in_proj_b,
                           const uint16_t *in_proj_a, const uint16_t *conv_weight, const uint16_t *A_log,
                           const uint16_t *dt_bias, const uint16_t *norm_weight, float eps, const uint16_t *out_proj,
                           uint16_t *conv_state, void *state, int state_bf16, uint16_t *conv_record,
                           void *state_record, uint16_t *out, uint16_t *sum_out, uint16_t *norm_out,
                           void *workspace, size_t workspace_bytes, void *stream);

/* ---- full-attention decode (the attention before each of the 10
 * full-attention layers' MoE) ----------------------------------------------- */

/* Bytes of workspace lrmoe_attn_decode needs for `tokens` tokens (1..16; 0
 * outside that range).  No reference counterpart. */
#define LRMOE_ATTN_MAX_TOKENS 16
size_t lrmoe_attn_workspace_bytes(int tokens);

/* One cached step of a full-attention layer of the 35B model (hidden 2048,
 * 16 query heads over 2 key/value heads of width 256, rotary width 64) for
 * 1..16 tokens after `length` cached positions: [HF]
 * Qwen3_5MoeAttention.forward with a key/value cache, which the reference
 * runs stock (edge35b/benchmark.py:141-146 and dflash_probe.py:122 decode
 * and verify through the Transformers model; edge35b/delta_decode.py:84-126
 * replaces only the linear-attention layers).  Weights as the module holds
 * them, bf16: q_proj [8192][2048] (per head 256 query rows, then 256 gate
 * rows), k_proj and v_proj [512][2048], o_proj [2048][4096], q_norm and
 * k_norm [256] (applied as 1 + w).  cos, sin [tokens][64] bf16: the
 * model's position embeddings for the new positions.  k_cache, v_cache
 * [2][capacity][256] bf16 hold the normed, rotated keys and the values of
 * positions 0 .. length - 1 and receive positions length .. length +
 * tokens - 1 (capacity >= length + tokens, at most 2^22).  Token t attends
 * to positions 0 .. length + t (causal within the block).  out
 * [tokens][2048] bf16 (the module's output, before the residual).
 * Workspace of lrmoe_attn_workspace_bytes(tokens), 256-byte aligned, used by
 * one stream at a time.  Rounding points: those of the Transformers forward
 * in bf16 (eager attention); the softmax runs in fp32 over chunks of
 * positions whose partial results are merged at the end. */
int lrmoe_attn_decode(const uint16_t *hidden, int tokens, const uint16_t *q_proj, const uint16_t *k_proj,
                      const uint16_t *v_proj, const uint16_t *o_proj, const uint16_t *q_norm, const uint16_t *k_norm,
                      float eps, const uint16_t *cos, const uint16_t *sin, uint16_t *k_cache, uint16_t *v_cache,
                      int capacity, int length, uint16_t *out, void *workspace, size_t workspace_bytes,
                      void *stream);

/* lrmoe_attn_decode with the cached length read on the device from
 * *length (int32) when the launches run, so that one captured graph serves
 * a cache that grows between replays (a verify loop: the reference's
 * dflash_probe.py:111-148 advances the cache after every accepted block).
 * The positions are split into chunks sized for `capacity`; chunks past
 * *length + tokens do no work.  *length must lie in [0, capacity - tokens]:
 * a value outside it is clamped for every cache access and the call's out
 * rows are NaN.  Host-side argument checks as lrmoe_attn_decode's. */
int lrmoe_attn_decode_at(const uint16_t *hidden, int tokens, const uint16_t *q_proj, const uint16_t *k_proj,
                         const uint16_t *v_proj, const uint16_t *o_proj, const uint16_t *q_norm,
                         const uint16_t *k_norm, float eps, const uint16_t *cos, const uint16_t *sin,
                         uint16_t *k_cache, uint16_t *v_cache, int capacity, const int32_t *length, uint16_t *out,
                         void *workspace, size_t workspace_bytes, void *stream);

/* The full-attention half of a decoder layer in one call, as
 * lrmoe_delta_mixer_step for the mixer: `residual` is the layer's input,
 * normed inside the projection launch with input_norm / input_eps; out is
 * the attention output and sum_out bf16(residual + out); norm_out, when not
 * NULL, the normed rows.  The cache length is `length`, or *length_dev read
 * on the device when length_dev is not NULL (lrmoe_attn_decode_at).  No
 * reference counterpart as one call.  Other arguments and workspace as
 * lrmoe_attn_decode's. */
int lrmoe_attn_decode_step(const uint16_t *residual, int tokens, const uint16_t *input_norm, float input_eps,
                           const uint16_t *q_proj, const uint16_t *k_proj, const uint16_t *v_proj,
                           const uint16_t *o_proj, const uint16_t *q_norm, const uint16_t *k_norm, float eps,
                           const uint16_t *cos, const uint16_t *sin, uint16_t *k_cache, uint16_t *v_cache,
                           int capacity, int length, const int32_t *length_dev, uint16_t *out, uint16_t *sum_out,
                           uint16_t *norm_out, void *workspace, size_t workspace_bytes, void *stream);

#ifdef __cplusplus
}
#endif

#endif /* LRMOE_H */
