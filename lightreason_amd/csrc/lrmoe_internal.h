// Host/device shared definitions for the lrmoe library: status codes, the
// workspace layout and the launch declarations each .hip file provides.
#pragma once

#include <hip/hip_ext.h>
#include <hip/hip_runtime.h>
#include <stddef.h>
#include <stdint.h>

#include "../../include/lrmoe.h"

namespace lrmoe {

// Bits of the device status word (workspace control block).
constexpr int32_t kStatusBadExpert = 1;     // expert id outside [0, 256)
constexpr int32_t kStatusRepeatedExpert = 2;  // a token routes to one expert twice
constexpr int32_t kStatusCodecRow = 4;      // gather met (and decoded) an escape-codec descriptor
constexpr int32_t kStatusTimeout = 8;       // a bounded cross-workgroup wait expired (results invalid)

// Decode layer (one persistent kernel) limits.
constexpr int kDecodeMaxTokens = 16;
constexpr int kDecodeSlots = 8 * kDecodeMaxTokens + 1;  // unique routed experts + the shared expert
constexpr int kSyncStride = 64;  // counters 256 bytes apart (separate memory channels)
constexpr int kPassTok = 128;    // prefill: tokens of one expert per work unit
constexpr int kCodecTile = 256;        // values per codec tile
constexpr int kCodecTileBytes = 384;   // packed bytes per tile (low bytes, then 4-bit codes)
constexpr int kCodecTableColumns = 10;  // int64 per expert in a decode codec table
constexpr int kCodecMisfit = 255;      // base of a tile whose exponent fields span more than 8 values

// Cross-workgroup counter of one decode call.
struct DecodeCounters {
    uint32_t claim;                              // work items handed out past the first two rounds
    uint32_t pad[kSyncStride - 1];
};

// Decode kernel synchronisation.  `finished` counts finished workgroups over
// all calls, so a call's number is finished / G (G = grid size, fixed per
// device) whenever one of its workgroups reads it: at most G - 1 of its own
// workgroups can have finished by then.  Call c uses set[c % 2] and zeroes
// set[(c + 1) % 2] for the next call, so nothing is reset at the end of a
// call and a zero-initialised workspace is valid.  The call number also tags
// the rows one workgroup writes for another (see kDecodeTagShift).
// A chain launch (several layers in one grid) numbers its layers c, c + 1,
// ... and adds its layer count per workgroup to `finished` at its end.
// `chain_arrive` counts workgroup arrivals at the grid barriers between a
// chain's layers and is never reset: a chain launch reads it at its start and
// rounds down to a multiple of G, since at most G - 1 of its own workgroups
// can have arrived at its first barrier by then.  The workgroup whose arrival
// completes a barrier stores the arrival count it completed in
// `chain_release`, which the others poll (a word that takes no atomics:
// polling the arrival counter itself slows the other workgroups' traffic).
struct DecodeSync {
    unsigned long long finished;
    uint32_t pad0[kSyncStride - 2];
    unsigned long long chain_arrive;
    uint32_t pad1[kSyncStride - 2];
    unsigned long long chain_release;
    uint32_t pad2[kSyncStride - 2];
    DecodeCounters set[2];
};

// Rows exchanged between decode workgroups are 8-byte words: two bf16 values
// in the low half and the writing call's tag (call number mod 2^32 - 1, plus
// 1, so never 0) in the high half.  A reader that sees its own call's tag in
// a word has that word's data; an 8-byte store is seen whole or not at all.
// (A tag repeats only after 2^32 - 1 decode calls on one workspace.)
constexpr int kDecodeTagShift = 32;
// The router's tagged logit rows are written in one copy per XCD (copy
// b % 8 read by workgroup b): every workgroup polls them, and 256 readers
// of one 1 KiB row crowd the few memory channels that hold it.
constexpr int kDecodeLogitCopies = 8;
constexpr int kDecodeLogitCopyWords = kDecodeMaxTokens * 128;  // 16 KiB apart

// Control block at the start of every workspace.  The route counter is reset
// to zero by the workgroup that consumes it, so a zero-initialised workspace
// stays valid across launches and graph replays.
struct Control {
    uint32_t route_counter;
    int32_t status;
    int32_t unique;
    int32_t n_units;    // prefill work units of the current plan
    uint32_t claim[8];  // prefill: items claimed from each of the 8 work lists (zeroed by pf_fill)
    uint32_t reserved[52];
};

// Route plan: unique experts ascending, per-expert (token, slot) pairs in
// ascending token order, and per token the pair index of each of its routes
// in ascending expert order.
struct Plan {
    int32_t* expert;      // [256]
    int32_t* offset;      // [257]
    int32_t* pair_token;  // [8T]
    int32_t* pair_slot;   // [8T]
    int32_t* route_pair;  // [T][8]
    int32_t* unique;      // [1] (in the control block)
    int32_t* status;      // [1] (in the control block)
};

// Carves one caller-provided device buffer into the per-call arrays.  The
// layout depends only on `tokens`, so any buffer of at least
// workspace_bytes(tokens) serves a call with that many tokens.
struct Workspace {
    Control* control;
    uint16_t* logits;     // [T][256]
    uint16_t* normed;     // [T][2048]
    int64_t* indices;     // [T][8]
    uint16_t* weights;    // [T][8]
    uint16_t* sg;         // [T]
    Plan plan;
    uint16_t* act;        // [8T + T + 16][512]: routed pairs, shared rows, padding
    uint16_t* y;          // [8T + T][2048]: routed pairs, then shared rows
    uint64_t* dact;       // decode: act as tagged words, [9*16 + 16][256]
    uint64_t* dy;         // decode: y as tagged words, [9*16][1024]
    uint64_t* dlogits;    // decode: router logits as tagged words, [16][128]
    uint16_t* chain;      // decode chain: [2][T][2048] outputs of the inner layers
    uint32_t* counts;     // [256] prefill: pairs per expert
    DecodeSync* sync;     // decode kernel counters
    uint8_t* bmask;       // prefill: [256][nblk_pad] token masks per 8-token block
    uint32_t* blk_base;   // prefill: [256][nblk_pad] pairs of the expert before the block
    int32_t* bstatus;     // prefill: [nblk] route status per block
    int4* units;          // prefill: work units (expert + 1 or 0 = shared, first pair, pairs, 0)
    uint32_t* unit_done;  // prefill: gate/up items done per work unit (zeroed by pf_fill)
    int max_units;
    int nblk_pad;
    size_t bytes;
};

inline size_t align_up(size_t value, size_t alignment) { return (value + alignment - 1) / alignment * alignment; }

inline Workspace carve(void* base, int tokens) {
    Workspace ws{};
    const size_t T = static_cast<size_t>(tokens > 0 ? tokens : 1);
    const size_t P = 8 * T;
    size_t offset = 0;
    auto take = [&](size_t bytes) {
        const size_t at = offset;
        offset = align_up(offset + bytes, 256);
        return static_cast<char*>(base) + at;
    };
    ws.control = reinterpret_cast<Control*>(take(sizeof(Control)));
    // Counters that persist between calls sit at a fixed offset, whatever
    // the token count of the call.
    ws.sync = reinterpret_cast<DecodeSync*>(take(sizeof(DecodeSync)));
    // So are the decode kernel's tagged rows (sized for 16 tokens): only
    // decode calls ever write them, so a word carrying a call's tag was
    // written by that call.
    ws.dact = reinterpret_cast<uint64_t*>(take((9 * kDecodeMaxTokens + 16) * 256 * 8));
    ws.dy = reinterpret_cast<uint64_t*>(take(9 * kDecodeMaxTokens * 1024 * 8));
    ws.dlogits = reinterpret_cast<uint64_t*>(take(kDecodeLogitCopies * kDecodeLogitCopyWords * 8));
    ws.logits = reinterpret_cast<uint16_t*>(take(T * 256 * 2));
    ws.normed = reinterpret_cast<uint16_t*>(take(T * 2048 * 2));
    ws.indices = reinterpret_cast<int64_t*>(take(T * 8 * 8));
    ws.weights = reinterpret_cast<uint16_t*>(take(T * 8 * 2));
    ws.sg = reinterpret_cast<uint16_t*>(take(T * 2));
    ws.plan.expert = reinterpret_cast<int32_t*>(take(256 * 4));
    ws.plan.offset = reinterpret_cast<int32_t*>(take(257 * 4));
    ws.plan.pair_token = reinterpret_cast<int32_t*>(take(P * 4));
    ws.plan.pair_slot = reinterpret_cast<int32_t*>(take(P * 4));
    ws.plan.route_pair = reinterpret_cast<int32_t*>(take(P * 4));
    // 16 rows of padding: the decode kernel stages 16 act rows per slot.
    ws.act = reinterpret_cast<uint16_t*>(take((P + T + 16) * 512 * 2));
    ws.y = reinterpret_cast<uint16_t*>(take((P + T) * 2048 * 2));

    ws.chain = reinterpret_cast<uint16_t*>(take(2 * T * 2048 * 2));
    ws.counts = reinterpret_cast<uint32_t*>(take(256 * 4));
    const size_t nblk = (T + 7) / 8;
    const size_t nblk_pad = (nblk + 15) / 16 * 16;
    ws.nblk_pad = static_cast<int>(nblk_pad);
    ws.bmask = reinterpret_cast<uint8_t*>(take(256 * nblk_pad));
    ws.blk_base = reinterpret_cast<uint32_t*>(take(256 * nblk_pad * 4));
    ws.bstatus = reinterpret_cast<int32_t*>(take(nblk * 4));
    const size_t units = (T + kPassTok - 1) / kPassTok + 256 + (8 * T + kPassTok - 1) / kPassTok + 8;
    ws.units = reinterpret_cast<int4*>(take(units * sizeof(int4)));
    ws.unit_done = reinterpret_cast<uint32_t*>(take(units * sizeof(uint32_t)));
    ws.max_units = static_cast<int>(units);
    ws.plan.unique = &ws.control->unique;
    ws.plan.status = &ws.control->status;
    ws.bytes = offset;
    return ws;
}

inline size_t workspace_bytes(int tokens) { return carve(nullptr, tokens).bytes; }

// Arguments of the router stage (decode and prefill share them).
struct RouteArgs {
    const uint16_t* x;            // [T][2048] layer input
    const uint16_t* norm;         // [2048] RMSNorm weight, or null for no norm
    float eps;
    const uint16_t* router;       // [256][2048], or null when logits_in is given
    const uint16_t* logits_in;    // [T][256] caller logits for top-k, or null
    const uint16_t* shared_gate;  // [2048] shared_expert_gate weight, or null
    int tokens;
    uint16_t* normed;             // [T][2048] normalised input (when norm)
    uint16_t* logits;             // [T][256]
    int64_t* indices;             // [T][8]
    uint16_t* weights;            // [T][8]
    uint16_t* sg;                 // [T]
    const uint16_t* shared_down;  // shared expert present (prefill work units) when non-null
    Plan plan;
    Workspace ws;
};

// Expert stage arguments.  Experts are addressed through a per-layer table of
// 256 (gate_up, down) device addresses; the shared expert through its three
// projection pointers.
struct ExpertArgs {
    const uint16_t* x;            // [T][2048] expert input (normalised when the layer norms)
    const int64_t* expert_ptrs;   // [256][2] gate_up [1024,2048] and down [2048,512] addresses
    const uint16_t* shared_gate_proj;  // [512][2048] or null
    const uint16_t* shared_up_proj;    // [512][2048]
    const uint16_t* shared_down;       // [2048][512]
    const uint16_t* weights;      // [T][8] routing weights by slot
    const uint16_t* sg;           // [T] shared gate values
    const uint16_t* residual;     // [T][2048] or null
    uint16_t* out;                // [T][2048]
    int tokens;
    Plan plan;
    Workspace ws;
};

// Arguments of the decode layer kernel (T <= 16).  Exactly one route source:
// router (GEMV in the kernel), logits_in, or indices_in + weights_in.
struct DecodeArgs {
    const uint16_t* x;            // [T][2048] layer input
    const uint16_t* norm;         // [2048] RMSNorm weight or null
    float eps;
    const uint16_t* router;       // [256][2048] or null
    const uint16_t* logits_in;    // [T][256] or null
    const int64_t* indices_in;    // [T][8] or null
    const uint16_t* weights_in;   // [T][8] with indices_in
    const uint16_t* shared_expert_gate;  // [2048] or null
    const uint16_t* sh_gate;      // shared expert [512][2048], or null
    const uint16_t* sh_up;        // [512][2048]
    const uint16_t* sh_down;      // [2048][512]
    const int64_t* expert_ptrs;   // [256][2] (gate_up, down)
    const int64_t* codec;         // [257][10] per expert, row 256 the shared expert: tile-codec addresses
                                  // (packed gate_up, packed down, gate_up bases, down bases), then 48 bytes of
                                  // per-(item, wave) raw flags; a zero row reads raw; or null
    uint16_t* out;                // [T][2048]
    int64_t* indices_out;         // [T][8] or null
    uint16_t* weights_out;        // [T][8] or null
    uint64_t* logits;             // [16][128] tagged words (workspace): router output, logits 2k, 2k+1 in word k
    uint64_t* act;                // [9T + 16][256] tagged words (workspace)
    uint64_t* y;                  // [9T][1024] tagged words (workspace)
    DecodeSync* sync;             // workspace counters
    int32_t* status;              // workspace status word
    int tokens;
    int residual;                 // out = x + MoE(...) (decoder layer with norm)
};

// A chain of decode layers in one launch.  Layer l reads the previous
// layer's output (layer 0 the caller's rows) and, when it is not the last,
// writes the next one's input to a workspace buffer.  The per-layer weight
// addresses travel in the kernel arguments.
struct ChainLayer {
    const uint16_t* router;              // [256][2048]
    const int64_t* expert_ptrs;          // [256][2] (gate_up, down)
    const uint16_t* sh_gate;             // shared expert [512][2048], or null (no shared expert)
    const uint16_t* sh_up;               // [512][2048]
    const uint16_t* sh_down;             // [2048][512]
    const uint16_t* shared_expert_gate;  // [2048]
    const uint16_t* norm;                // [2048] RMSNorm weight, or null (no norm, no residual)
    const int64_t* codec;                // [257][10] tile-codec table (DecodeArgs::codec), or null
};
constexpr int kChainMaxLayers = 48;  // the arguments stay under 4 KiB
struct ChainArgs {
    DecodeArgs base;              // tokens, eps, workspace buffers, status; per-layer fields unset
    const uint16_t* hidden;       // [T][2048] input of layer 0
    uint16_t* out;                // [T][2048] output of the last layer
    uint16_t* inner;              // [2][T][2048] outputs of the inner layers (ping-pong)
    int layers;
    ChainLayer layer[kChainMaxLayers];
};
static_assert(sizeof(ChainArgs) <= 4096, "chain kernel arguments must stay under 4 KiB");

// Optional per-stage timing.  When a stage's bit is enabled, timing_events()
// hands out the next (start, stop) event pair of that stage; the stage's
// first kernel is launched with the start event and its last kernel with the
// stop event through hipExtLaunchKernelGGL, so the two timestamps are taken
// by the kernels' own dispatches (no separate marker packets).  Both events
// are null when the stage is not timed (or its event list is full), and the
// launch is then an ordinary one.
enum Stage : int {
    kStageRoute = 1,
    kStageGateUp = 2,
    kStageDown = 4,
    kStageCombine = 8,
    kStageGather = 16,
    kStageLayer = 32,
    kStageDeltaMixer = 64,  // Gated DeltaNet: the mixer step (dn_mixer)
    kStageDeltaRule = 128,  // Gated DeltaNet: the delta rule (dn_rule)
    kStageAttention = 256,  // full-attention decode step (first to last of its launches)
};
struct StageEvents {
    hipEvent_t start = nullptr;
    hipEvent_t stop = nullptr;
};
StageEvents timing_events(int stage);

// Launch with optional start/stop timing events (see timing_events).
#define LRMOE_LAUNCH(kernel, grid, block, lds, stream, start_event, stop_event, ...)                            \
    do {                                                                                                      \
        const hipEvent_t lrmoe_start_ = (start_event);                                                        \
        const hipEvent_t lrmoe_stop_ = (stop_event);                                                          \
        if (lrmoe_start_ != nullptr || lrmoe_stop_ != nullptr) {                                              \
            hipExtLaunchKernelGGL(kernel, grid, block, lds, stream, lrmoe_start_, lrmoe_stop_, 0, __VA_ARGS__); \
        } else {                                                                                              \
            hipLaunchKernelGGL(kernel, grid, block, lds, stream, __VA_ARGS__);                                \
        }                                                                                                     \
    } while (0)

hipError_t launch_gather_tiles(const int64_t* descriptors, const int64_t* destinations, const int64_t* sizes,
                               const int32_t* src_ids, const int32_t* dst_ids, const int64_t* count, int experts,
                               int banks, int max_copies, int stripes, int threads, int compact, hipStream_t stream);
hipError_t launch_route(const RouteArgs& args, hipStream_t stream);
hipError_t launch_bucket(const int64_t* indices, int tokens, const Workspace& ws, const Plan& plan, hipStream_t stream);
hipError_t launch_gather(const int64_t* descriptors, const int64_t* destinations, const int64_t* sizes,
                         const int32_t* src_ids, const int32_t* dst_ids, const int64_t* count, int experts, int banks,
                         int max_copies, int stripes, int threads, int keep_in_l2, int32_t* status,
                         hipStream_t stream);
hipError_t launch_matvec(const int64_t* table, const uint16_t* x, uint16_t* result, int K, int N, int column,
                         int shared_x, int stride, int experts, hipStream_t stream);
hipError_t launch_ordered_sum(const int64_t* table, const uint16_t* hot, const uint16_t* cold, const uint16_t* router,
                              uint16_t* out, int stride, hipStream_t stream);
hipError_t launch_gate_silu(const int64_t* table, const uint16_t* hidden, uint16_t* active, int stride, int experts,
                            hipStream_t stream);
hipError_t launch_project(const int64_t* pointers, const int32_t* routes, const uint16_t* X, uint16_t* Y, int in,
                          int out, int down, int experts, hipStream_t stream);
hipError_t launch_swiglu_rows(const uint16_t* gates, uint16_t* active, int rows, hipStream_t stream);
hipError_t launch_add_rmsnorm(const uint16_t* x, const uint16_t* add, int tokens, const uint16_t* norm, float eps,
                              uint16_t* sum_out, uint16_t* norm_out, hipStream_t stream);
hipError_t launch_block_combine(const int32_t* inverse, const uint16_t* X, const uint16_t* cold, const uint16_t* router,
                                uint16_t* out, int tokens, int hybrid, hipStream_t stream);
hipError_t launch_experts(const ExpertArgs& args, hipStream_t stream);
hipError_t launch_moe_decode(const DecodeArgs& args, hipStream_t stream);
hipError_t launch_moe_chain(const ChainArgs& args, hipStream_t stream);
// Prefill plan (T > 16): top-8 from `logits` (or the validated caller indices)
// and the bucketing plan with its work units.
hipError_t launch_prefill_plan(const uint16_t* logits, const int64_t* indices_in, const uint16_t* weights_in,
                               int64_t* indices, uint16_t* weights, int tokens, int shared_present,
                               const Workspace& ws, const Plan& plan, hipStream_t stream);
hipError_t launch_prefill_experts(const ExpertArgs& args, hipStream_t stream);
size_t decode_lds_bytes(int tokens, bool codec);
hipError_t launch_codec_pack(const uint16_t* w, int64_t rows, int cols, uint8_t* packed, uint8_t* bases,
                             unsigned long long* misfit, hipStream_t stream);
hipError_t launch_codec_unpack(const uint8_t* packed, const uint8_t* bases, int64_t rows, int cols, uint16_t* w,
                               hipStream_t stream);
hipError_t launch_fill_normal(uint16_t* out, int64_t count, uint64_t seed, uint64_t stream_id, double sigma,
                              int64_t first, hipStream_t stream);

// ---- Gated DeltaNet decode (delta.hip) ----

// Weights, states and rows of one mixer step.
struct DnProjectArgs {
    const uint16_t* x;        // hidden [T][2048]
    const uint16_t* w_qkv;    // in_proj_qkv [8192][2048]
    const uint16_t* w_z;      // in_proj_z [4096][2048]
    const uint16_t* w_b;      // in_proj_b [32][2048]
    const uint16_t* w_a;      // in_proj_a [32][2048]
    const uint16_t* conv_w;   // conv1d weight [8192][4]
    const uint16_t* A_log;    // [32]
    const uint16_t* dt_bias;  // [32]
    const uint16_t* norm_w;   // gated RMSNorm weight [128]
    const uint16_t* w_out;    // out_proj [2048][4096]
    float eps;
    uint16_t* conv_state;     // [8192][4], updated in place
    uint16_t* conv_record;    // [T][8192][4] per-token conv states, or null
    uint16_t* act;            // [T][8192] conv + SiLU outputs (q | k | v)
    uint16_t* z;              // [T][4096]
    uint16_t* beta;           // [T][32]
    float* G;                 // [T][32] exp(g)
    uint16_t* out;            // [T][2048]
    int tokens;
    // The decoder layer's glue, fused (all null for a plain mixer call):
    const uint16_t* in_norm;  // input RMSNorm weight [2048]: x is then the raw residual stream, normed here
    float in_eps;
    uint16_t* norm_out;       // [T][2048] the normed rows (written by workgroup 0), or null
    uint16_t* sum_out;        // [T][2048] bf16(x + out), the residual add, or null
};

// The delta rule over `tokens` tokens for `heads` value heads of state
// width `width` (E); q/k head of value head h is h >> kv_shift.
struct DnRuleArgs {
    const uint16_t* q;
    const uint16_t* k;
    const uint16_t* v;
    int64_t qk_stride;  // elements between consecutive tokens of q and k
    int64_t v_stride;   // elements between consecutive tokens of v
    int kv_shift;
    const float* G;         // [T][H]
    const uint16_t* beta;   // [T][H]
    const void* initial;    // [H][D][E]
    void* final_state;      // [H][D][E] or null (may equal initial)
    void* record;           // [T][H][D][E] or null
    uint16_t* out;          // [T][H][E]
    int tokens;
    int heads;
    int width;
    int normalize;
};

struct DeltaWorkspace {
    int32_t* status;               // LRMOE_STATUS_TIMEOUT when a wait expired
    unsigned long long* heads;     // [32] rule workgroups done per head (8 per call, never reset)
    unsigned long long* normed;    // [32] per head: number of the last call whose normed rows are stored
    unsigned long long* staged;    // [256] per workgroup: number of the last call whose q, k, v rows are stored
    uint16_t* act;
    uint16_t* z;
    uint16_t* beta;
    float* G;
    uint16_t* o;
    uint16_t* core;
    size_t bytes;
};

// Offsets of the mixer workspace's control block: the status word, the 32
// per-head counters, the 32 per-head "normed rows stored" flags and the 256
// per-workgroup "q, k and v rows stored" flags, each counter or flag in its
// own 128-byte line.
constexpr size_t kDeltaWsStatus = 0;
constexpr size_t kDeltaWsHeads = 1024;
constexpr size_t kDeltaWsNormed = 5120;
constexpr size_t kDeltaWsStaged = 9216;
constexpr size_t kDeltaWsStride = 16;  // u64 words between counters or flags
constexpr size_t kDeltaWsControl = 41984;

struct DnMixerArgs {
    DnProjectArgs p;
    void* state;
    void* state_record;
    uint16_t* o;
    uint16_t* core;
    int32_t* status;
    unsigned long long* heads;
    unsigned long long* normed;
    unsigned long long* staged;
};

constexpr int kDeltaMaxTokens = 16;

// ---- full-attention decode step (attention.hip) ----
constexpr int kAttnMaxTokens = 16;
constexpr int kAttnMaxChunks = 128;  // position chunks per key/value head (up to 8 tokens; 64 above)
struct AttnArgs {
    uint16_t* proj;         // [T][9216]: per token q/gate (8192), k (512), v (512) rows, bf16
    const uint16_t* q_norm; // [256]
    const uint16_t* k_norm; // [256]
    float eps;
    const uint16_t* cos;    // [T][64] bf16
    const uint16_t* sin;    // [T][64] bf16
    uint16_t* k_cache;      // [2][capacity][256] bf16 (normed, rotated keys)
    uint16_t* v_cache;      // [2][capacity][256] bf16
    int capacity;
    int length;             // cached positions before the call
    const int32_t* length_dev;  // or, when set, read on the device (a graph replayed as the cache grows)
    int tokens;
    int sub_blocks;         // 32-position sub-blocks the chunks cover (ceil(span / 32))
    int per;                // sub-blocks per chunk: chunk c covers sub-blocks c per .. (c + 1) per - 1,
    int chunks;             // the last one the rest; chunks per key/value head (<= kAttnMaxChunks)
    int halves;             // 1, or 2: a chunk's query rows in two workgroups, tokens split at t_half
    int t_half;
    uint16_t* part_o;       // [2][chunks][8 T][256] unnormalised rows, bf16
    float* part_ml;         // [2][chunks][8 T][2] running max and sum
    uint16_t* att;          // [T][4096] gated attention rows, bf16
};
struct AttnWorkspace {
    uint16_t* proj;
    uint16_t* att;
    uint16_t* part_o;
    float* part_ml;
    size_t bytes;
};
AttnWorkspace carve_attn(void* base, int tokens);
size_t attn_workspace_bytes(int tokens);
// The chunking of `span` positions for `tokens` tokens: sets sub_blocks,
// chunks, halves and t_half of a.
void attn_geometry(AttnArgs& a, int tokens, int span);
// The decoder layer's glue fused into an attention step (all null for a
// plain call): x is then the raw residual stream, normed in the projection
// launch with in_norm / in_eps (the normed rows also to norm_out when not
// null), and sum_out receives bf16(x + out).
struct AttnGlue {
    const uint16_t* in_norm;
    float in_eps;
    uint16_t* norm_out;
    uint16_t* sum_out;
};
hipError_t launch_attn_decode(AttnArgs a, const uint16_t* x, const uint16_t* w_q, const uint16_t* w_k,
                              const uint16_t* w_v, const uint16_t* w_o, uint16_t* out, const AttnGlue& fused,
                              hipStream_t stream);
DeltaWorkspace carve_delta(void* base, int tokens);
size_t delta_workspace_bytes(int tokens);
hipError_t launch_delta_rule(const DnRuleArgs& a, int key_width, bool state_bf16, hipStream_t stream);
hipError_t launch_delta_mixer(DnProjectArgs p, void* state, bool state_bf16, void* state_record,
                              const DeltaWorkspace& w, hipStream_t stream);

}  // namespace lrmoe
