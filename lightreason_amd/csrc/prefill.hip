// Prefill (T > 16 tokens): routing plan and grouped expert GEMMs on MFMA.
//
// Plan (same layout as the decode/bucketing plan, experts ascending, tokens
// ascending within an expert: edge35b/pipeline.py:59-76 _routes,
// block_experts.py:102-121):
//   pf_topk   top-8 per token (or the caller's indices, validated); per block
//             of 8 tokens an 8-bit token mask per expert, built in LDS
//             (no global atomics);
//   pf_scan   one workgroup per expert: prefix of its mask popcounts over the
//             blocks, and its pair count;
//   pf_fill   expert offsets and ranks, every route placed, and the list of
//             work units (slot, first pair) of at most kPassTok tokens.
//
// Experts (cpu_experts.c:54-69 rounding points; the shared expert is slot 0),
// one persistent launch (pf_experts) whose workgroups take, from 8 work
// lists, gate/up items and then down items:
//   gate/up   one item per (unit, 128-row tile): 128 gate + 128 up rows
//             of one expert against up to 128 tokens.  Each of the 8 waves
//             streams its 32 weight rows (16 gate, 16 up) from HBM straight
//             into MFMA A operands, two K-chunks ahead; the same waves stage
//             the unit's token rows in LDS chunk by chunk (three chunks ahead
//             in registers), shared by all 8 waves, so a weight byte is read
//             once per 128 tokens and feeds up to 8 16x16x32 MFMAs.  SwiGLU
//             in the epilogue, act rows out.
//   down      one item per (unit, 512 output rows): the unit's act rows are
//             staged in LDS once, then 4 tiles of 128 down rows over k = 512
//             pass through registers, each wave loading the next tile's rows
//             while it multiplies the current one; y rows out (bf16).
//   The ordered combine is experts.hip's combine_kernel.
//
// A list is a contiguous eighth of the units, served by the workgroups b
// with b % 8 = the list (on XCD b % 8): a unit's token and act rows are
// fetched into one XCD's L2, and an expert's units (consecutive in the
// plan) run together on one XCD, its weight tiles shared through that L2.
// Act rows go out and come back with agent-scope stores and loads, so
// results do not depend on that placement.
#include "lrmoe_device.h"
#include "lrmoe_internal.h"

namespace lrmoe {
namespace {

constexpr int kBlkTok = 8;                 // tokens per routing block
constexpr int kGuRows = 128;                // intermediate rows (gate and up) per gate/up workgroup
constexpr int kGuTiles = kInner / kGuRows;  // 4 gate/up tiles per expert
constexpr int kGuChunk = 128;              // k per LDS chunk
constexpr int kGuChunks = kHidden / kGuChunk;
constexpr int kGuSteps = kGuChunk / 32;    // MFMA k-steps (and A loads per lane) per chunk
constexpr int kXsStride = kGuChunk + 8;    // LDS token row stride (bf16)
constexpr int kDnThreads = 512;            // down workgroup: 8 waves of 16 output rows
constexpr int kDnRows = kDnThreads / kWave * 16;  // 128 output rows per down workgroup
constexpr int kDnTiles = kHidden / kDnRows;       // 16 down tiles per expert
constexpr int kDnItemTiles = 4;                   // tiles per down item
constexpr int kDnItems = kDnTiles / kDnItemTiles; // 4 down items per unit
constexpr int kDnPieces = kPassTok * (kInner / 8) / kDnThreads;  // 16-byte act pieces per thread: a whole unit
constexpr int kActStride = kInner + 8;     // LDS act row stride (bf16)
constexpr uint64_t kPfSpinTicks = 5000000; // 50 ms of the 100 MHz wall clock
constexpr int32_t kStatusTimeoutPf = LRMOE_STATUS_TIMEOUT;

// ---- plan ----------------------------------------------------------------------

__global__ __launch_bounds__(256) void pf_topk(const uint16_t* logits, const int64_t* indices_in,
                                               const uint16_t* weights_in, int64_t* indices, uint16_t* weights,
                                               int tokens, Workspace ws) {
    __shared__ uint32_t mask[kExperts];
    __shared__ int32_t bad;
    const int blk = blockIdx.x;
    const int wave = threadIdx.x >> 6;
    const int lane = threadIdx.x & 63;
    mask[threadIdx.x] = 0u;
    if (threadIdx.x == 0) bad = 0;
    __syncthreads();
#pragma unroll
    for (int j = 0; j < 2; ++j) {
        const int i = 2 * wave + j;
        const int t = blk * kBlkTok + i;
        if (t >= tokens) continue;
        int e = 0;
        bool ok = true;
        if (indices_in == nullptr) {
            const uint64_t packed = *reinterpret_cast<const uint64_t*>(logits + static_cast<size_t>(t) * kExperts + 4 * lane);
            uint32_t w = 0;
            topk8_wave(packed, e, w, static_cast<int>(threadIdx.x & 63));
            if (lane < kTopK) {
                indices[t * kTopK + lane] = e;
                weights[t * kTopK + lane] = static_cast<uint16_t>(w);
            }
        } else if (lane < kTopK) {
            const int64_t v = indices_in[t * kTopK + lane];
            int32_t flags = (v < 0 || v >= kExperts) ? kStatusBadExpert : 0;
            for (int q = 0; q < lane; ++q) flags |= indices_in[t * kTopK + q] == v ? kStatusRepeatedExpert : 0;
            if (flags) atomicOr(&bad, flags);
            ok = flags == 0;
            e = ok ? static_cast<int>(v) : 0;
        }
        if (lane < kTopK && ok) atomicOr(&mask[e], 1u << i);
    }
    __syncthreads();
    ws.bmask[static_cast<size_t>(threadIdx.x) * ws.nblk_pad + blk] = static_cast<uint8_t>(mask[threadIdx.x]);
    if (threadIdx.x == 0) ws.bstatus[blk] = bad;
}

__global__ __launch_bounds__(256) void pf_scan(int nblk, Workspace ws, Plan plan) {
    __shared__ uint32_t scratch[4];
    const int e = blockIdx.x;
    const int per = (nblk + 255) / 256;
    const int b0 = threadIdx.x * per;
    const int b1 = min(b0 + per, nblk);
    const uint8_t* row = ws.bmask + static_cast<size_t>(e) * ws.nblk_pad;
    uint32_t local = 0;
    for (int b = b0; b < b1; ++b) local += __popc(row[b]);
    uint32_t total = 0;
    uint32_t running = block_scan256(local, scratch, &total, static_cast<int>(threadIdx.x));
    for (int b = b0; b < b1; ++b) {
        ws.blk_base[static_cast<size_t>(e) * ws.nblk_pad + b] = running;
        running += __popc(row[b]);
    }
    if (threadIdx.x == 0) ws.counts[e] = total;
    if (e == 0) {
        int32_t flags = 0;
        for (int b = threadIdx.x; b < nblk; b += 256) flags |= ws.bstatus[b];
        __shared__ int32_t all;
        if (threadIdx.x == 0) all = 0;
        __syncthreads();
        if (flags) atomicOr(&all, flags);
        __syncthreads();
        if (threadIdx.x == 0) *plan.status = all;
    }
}

__global__ __launch_bounds__(256) void pf_fill(const int64_t* indices, int tokens, int shared_present, Workspace ws,
                                               Plan plan) {
    __shared__ uint32_t scratch[4];
    __shared__ uint32_t off[kExperts];
    const int blk = blockIdx.x;
    const int e = threadIdx.x;
    const int32_t status = *plan.status;
    if (status != 0) {
        for (int i = threadIdx.x; i < kBlkTok * kTopK; i += 256) {
            const int t = blk * kBlkTok + i / kTopK;
            if (t < tokens) plan.route_pair[t * kTopK + i % kTopK] = -1;
        }
        if (blk == 0 && threadIdx.x == 0) {
            *plan.unique = 0;
            plan.offset[0] = 0;
            ws.control->n_units = 0;
        }
        if (blk == 0 && threadIdx.x < 8) ws.control->claim[threadIdx.x] = 0u;
        return;
    }
    if (blk == 0) {
        // pf_experts' claim counters and per-unit gate/up counts, for this call
        for (int i = threadIdx.x; i < ws.max_units; i += 256) ws.unit_done[i] = 0u;
        if (threadIdx.x < 8) ws.control->claim[threadIdx.x] = 0u;
    }
    const uint32_t count = ws.counts[e];
    uint32_t pairs = 0, unique = 0;
    const uint32_t pair0 = block_scan256(count, scratch, &pairs, static_cast<int>(threadIdx.x));
    const uint32_t rank = block_scan256(count ? 1u : 0u, scratch, &unique, static_cast<int>(threadIdx.x));
    off[e] = pair0;
    if (blk == 0) {
        if (count) {
            plan.expert[rank] = e;
            plan.offset[rank] = static_cast<int32_t>(pair0);
        }
        // Work units: the shared expert's passes, then each routed expert's.
        const uint32_t passes = (count + kPassTok - 1) / kPassTok;
        uint32_t unit_total = 0;
        const uint32_t shared_units = shared_present ? (tokens + kPassTok - 1) / kPassTok : 0u;
        const uint32_t first_unit = shared_units + block_scan256(passes, scratch, &unit_total, static_cast<int>(threadIdx.x));
        // A unit names its expert and pair range directly, so an expert
        // workgroup reaches its weight addresses in two dependent loads.
        for (uint32_t j = threadIdx.x; j < shared_units; j += 256) {
            const int first = static_cast<int>(j) * kPassTok;
            ws.units[j] = make_int4(0, kTopK * tokens + first, min(kPassTok, tokens - first), 0);
        }
        for (uint32_t j = 0; j < passes; ++j) {
            const int first = static_cast<int>(j) * kPassTok;
            ws.units[first_unit + j] = make_int4(1 + e, static_cast<int>(pair0) + first,
                                                 min(kPassTok, static_cast<int>(count) - first), 0);
        }
        if (threadIdx.x == 0) {
            plan.offset[unique] = static_cast<int32_t>(pairs);
            *plan.unique = static_cast<int32_t>(unique);
            ws.control->n_units = static_cast<int32_t>(shared_units + unit_total);
        }
    }
    __syncthreads();
    if (threadIdx.x < kBlkTok * kTopK) {
        const int i = threadIdx.x / kTopK;
        const int k = threadIdx.x % kTopK;
        const int t = blk * kBlkTok + i;
        if (t < tokens) {
            const int ex = static_cast<int>(indices[t * kTopK + k]);
            const size_t at = static_cast<size_t>(ex) * ws.nblk_pad + blk;
            const int p = static_cast<int>(off[ex] + ws.blk_base[at] + __popc(ws.bmask[at] & ((1u << i) - 1u)));
            plan.pair_token[p] = t;
            plan.pair_slot[p] = k;
            int order = 0;
#pragma unroll
            for (int q = 0; q < kTopK; ++q) order += indices[t * kTopK + q] < ex ? 1 : 0;
            plan.route_pair[t * kTopK + order] = p;
        }
    }
}

// ---- experts -------------------------------------------------------------------

struct Unit {
    const uint16_t* gate;
    const uint16_t* up;
    const uint16_t* down;
    const int32_t* tokens;  // token of each pair of the unit, or null for pair index = token (shared)
    int pair0;              // first act/y row of the unit
    int count;              // pairs in the unit, 1..kPassTok
};

// The unit table, the unit count and the expert table are written before
// the expert launch and only read during it: they are read through the
// constant address space, so a wave-uniform lookup is a scalar load, counted
// apart from the vector loads that stream weights and rows.
template <typename T>
__device__ __forceinline__ T ld_const(const T* p) {
    return *reinterpret_cast<const __attribute__((address_space(4))) T*>(reinterpret_cast<uintptr_t>(p));
}

__device__ __forceinline__ bool load_unit(const ExpertArgs& a, int u, Unit& w) {
    if (u >= ld_const(&a.ws.control->n_units)) return false;
    const int* rec = reinterpret_cast<const int*>(a.ws.units + u);
    const int4 unit = make_int4(ld_const(rec), ld_const(rec + 1), ld_const(rec + 2), ld_const(rec + 3));
    w.pair0 = unit.y;
    w.count = unit.z;
    if (unit.x == 0) {
        w.gate = a.shared_gate_proj;
        w.up = a.shared_up_proj;
        w.down = a.shared_down;
        w.tokens = nullptr;
        return true;
    }
    const int e = unit.x - 1;
    const uint16_t* gate_up = reinterpret_cast<const uint16_t*>(ld_const(a.expert_ptrs + 2 * e));
    w.gate = gate_up;
    w.up = gate_up + static_cast<size_t>(kInner) * kHidden;
    w.down = reinterpret_cast<const uint16_t*>(ld_const(a.expert_ptrs + 2 * e + 1));
    w.tokens = a.plan.pair_token + unit.y;
    return true;
}

// gate/up workgroup (128 intermediate rows of one work unit): 8 waves, each
// owning two 16-row MFMA tiles (tile r = 8 gate rows and the 8 up rows with
// the same indices).  The waves also move the unit's token rows into LDS,
// one 128-column chunk at a time.  A wave issues, per chunk, its token pieces
// three chunks ahead and its weights two chunks ahead, in that order; every
// wait is then for exactly the data used next (the memory counter retires in
// order), and two chunks of weights (16 KiB per wave) stay in flight.  With
// 8 waves per CU each wave has 256 VGPRs for the 3 weight buffers, the 3
// token-piece buffers and the accumulators.  A B operand read from LDS feeds
// both row tiles, and the 4 workgroups of a unit each read its token rows
// once.
constexpr int kGuWaves = kGuRows / 16;
constexpr int kGuThreads = kGuWaves * kWave;
constexpr int kGuPieces = kPassTok * kGuChunk / 8 / kGuThreads;  // 16-byte token pieces per thread per chunk
constexpr int kGuWAhead = 2;  // weight chunks in flight ahead of the MFMAs
constexpr int kGuTAhead = 3;  // token chunks in flight ahead of the MFMAs

// The K loop for NB 16-token column blocks (blocks past the unit's tokens
// read rows whose results are dropped), then SwiGLU.  xrow[j] is this
// thread's token piece j (row xrow_row[j] of the unit, 16 bytes at column
// 8 * piece of each chunk).
template <int NB>
__device__ __forceinline__ void gateup_mfma(const uint16_t* arow0, const uint16_t* arow1, const uint16_t* const* xrow,
                                            const int* xrow_row, int piece, uint16_t* xs, uint16_t* act0,
                                            uint16_t* act1, int count) {
    const int lane = threadIdx.x & 63;
    const int m = lane & 15;
    const int g = lane >> 4;
    f32x4 acc[2][NB];
#pragma unroll
    for (int b = 0; b < NB; ++b) acc[0][b] = acc[1][b] = f32x4{0.0f, 0.0f, 0.0f, 0.0f};
    // Weights of a chunk: kGuSteps k-steps of both tiles, 256 contiguous
    // bytes per row, so each DRAM row is read in one burst.
    uint4 wb[kGuWAhead + 1][kGuSteps][2];
    uint4 xr[kGuTAhead][kGuPieces];
    auto load_w = [&](int c, uint4 (*dst)[2]) {
#pragma unroll
        for (int j = 0; j < kGuSteps; ++j) {
            dst[j][0] = ldg16(arow0 + 32 * (kGuSteps * c + j));
            dst[j][1] = ldg16(arow1 + 32 * (kGuSteps * c + j));
        }
    };
    auto load_t = [&](int c, uint4* dst) {
#pragma unroll
        for (int j = 0; j < kGuPieces; ++j) dst[j] = ldg16(xrow[j] + c * kGuChunk);
    };
    auto store_t = [&](int c, const uint4* src) {
#pragma unroll
        for (int j = 0; j < kGuPieces; ++j)
            *reinterpret_cast<uint4*>(xs + ((c & 1) * kPassTok + xrow_row[j]) * kXsStride + 8 * piece) = src[j];
    };
#pragma unroll
    for (int c = 0; c < kGuTAhead; ++c) load_t(c, xr[c]);
#pragma unroll
    for (int c = 0; c < kGuWAhead; ++c) load_w(c, wb[c]);
    store_t(0, xr[0]);
    const uint16_t* xb = xs + m * kXsStride + 8 * g;
#pragma unroll
    for (int c = 0; c < kGuChunks; ++c) {
        // Chunk c is in LDS buffer c & 1; chunk c-1's buffer and registers
        // are free.
        __syncthreads();
        if (c + 1 < kGuChunks) store_t(c + 1, xr[(c + 1) % kGuTAhead]);
        if (c + kGuTAhead < kGuChunks) load_t(c + kGuTAhead, xr[(c + kGuTAhead) % kGuTAhead]);
        if (c + kGuWAhead < kGuChunks) load_w(c + kGuWAhead, wb[(c + kGuWAhead) % (kGuWAhead + 1)]);
        const uint16_t* xcb = xb + (c & 1) * kPassTok * kXsStride;
#pragma unroll
        for (int j = 0; j < kGuSteps; ++j) {
            const uint4* ab = wb[c % (kGuWAhead + 1)][j];
#pragma unroll
            for (int b = 0; b < NB; ++b) {
                const uint4 bv = *reinterpret_cast<const uint4*>(xcb + 16 * b * kXsStride + 32 * j);
                acc[0][b] = mfma16x16x32(ab[0], bv, acc[0][b]);
                acc[1][b] = mfma16x16x32(ab[1], bv, acc[1][b]);
            }
        }
    }
    // SwiGLU: lanes g < 2 hold gate rows 4g..4g+3 of a tile's 8, lane + 32 the
    // up rows with the same index.  act0/act1 point at this lane's first act
    // element of column 0 for tile 0 and 1 (4 consecutive intermediate rows).
#pragma unroll
    for (int r = 0; r < 2; ++r) {
#pragma unroll
        for (int b = 0; b < NB; ++b) {
            f32x4 up;
#pragma unroll
            for (int i = 0; i < 4; ++i) up[i] = __shfl_xor(acc[r][b][i], 32, kWave);
            const int col = 16 * b + m;
            if (g < 2 && col < count) {
                uint32_t v[4];
#pragma unroll
                for (int i = 0; i < 4; ++i) v[i] = swiglu_bf16(rbf(acc[r][b][i]), rbf(up[i]));
                st_agent64((r ? act1 : act0) + static_cast<size_t>(16 * b) * kInner,
                           static_cast<uint64_t>(v[0] | (v[1] << 16)) | (static_cast<uint64_t>(v[2] | (v[3] << 16)) << 32));
            }
        }
    }
}

// The expert stage of a prefill layer in one persistent launch: one
// workgroup per CU.  Workgroup b serves list b % 8 (a contiguous eighth of
// the units, so a unit's items and an expert's units share an XCD's L2
// when workgroup b runs on XCD b % 8): first the 4 gate/up items of each of
// its units, then
// the 4 down items of each, claimed from the list's counter one item ahead
// (a gate/up item claims its successor when it starts, a down item during
// its third tile).  A down item first waits (bounded) until its unit's 4
// gate/up items have counted themselves in.  Every gate/up item is claimed
// before any down item of its list and a claimed gate/up item never waits,
// so the waits end whether or not all workgroups are resident.  The claim
// counters and per-unit counts are zeroed by pf_fill.
__global__ __launch_bounds__(kDnThreads, 1) void pf_experts(ExpertArgs a) {
    extern __shared__ __attribute__((aligned(16))) uint16_t lds[];
    __shared__ int claimed_s;
    __shared__ int timeout_s;
    const int tid = threadIdx.x;
    const int list = blockIdx.x % 8;
    const int n_units = ld_const(&a.ws.control->n_units);
    const int first = n_units * list / 8;  // the list's units: [first, first + units)
    const int units = n_units * (list + 1) / 8 - first;
    const int n_gu = kGuTiles * units;
    const int n_items = n_gu + kDnItems * units;
    uint32_t* claim = &a.ws.control->claim[list];
    auto take = [&]() -> uint32_t { return __builtin_amdgcn_atomic_inc32(claim, 0xffffffffu, __ATOMIC_RELAXED, "agent"); };
    // The claimed item, broadcast to the workgroup (item indices are
    // wave-uniform, so the unit lookups are scalar loads).
    auto publish = [&](uint32_t claimed) -> int {
        if (tid == 0) claimed_s = static_cast<int>(claimed);
        __syncthreads();
        const int item = __builtin_amdgcn_readfirstlane(claimed_s);
        __syncthreads();  // every thread has read claimed_s before it is written again
        return item;
    };
    if (tid == 0) timeout_s = 0;
    int cur = publish(tid == 0 ? take() : 0u);

    // ---- gate/up items (every one claimed before any down item) ----
    while (cur < n_gu) {
        uint32_t claimed = 0u;
        if (tid == 0) claimed = take();
        const int u = first + cur / kGuTiles;
        const int tile = cur % kGuTiles;
        // The item's code is written out here rather than called as an
        // inlined function: that form spills registers.
        Unit w;
        if (load_unit(a, u, w)) {
            const int wave = tid >> 6;
            const int lane = tid & 63;
            // Token pieces of this thread: piece tid % 16 of unit rows tid / 16 + 32 j
            // (rows past the unit's count repeat its first token).
            const int piece = tid & 15;
            const uint16_t* xrow[kGuPieces];
            int xrow_row[kGuPieces];
#pragma unroll
            for (int j = 0; j < kGuPieces; ++j) {
                const int c = tid / 16 + (kGuThreads / 16) * j;  // token row of the unit, 0..127
                const int cc = c < w.count ? c : 0;
                const int t = w.tokens ? w.tokens[cc] : w.pair0 - kTopK * a.tokens + cc;
                xrow[j] = a.x + static_cast<size_t>(t) * kHidden + 8 * piece;
                xrow_row[j] = c;
            }
            const int m = lane & 15;
            const int g = lane >> 4;
            const int nblk = (w.count + 15) / 16;
            // MFMA row m < 8 of tile r is gate row 128*tile + 16*wave + 8r + m, m >= 8
            // the up row with the same index.
            const uint16_t* rows = m < 8 ? w.gate : w.up;
            const int row0 = kGuRows * tile + 16 * wave + (m & 7);
            const uint16_t* arow0 = rows + static_cast<size_t>(row0) * kHidden + 8 * g;
            const uint16_t* arow1 = rows + static_cast<size_t>(row0 + 8) * kHidden + 8 * g;
            uint16_t* act0 = a.ws.act + static_cast<size_t>(w.pair0 + m) * kInner + kGuRows * tile + 16 * wave + 4 * g;
            uint16_t* act1 = act0 + 8;
            if (nblk <= 2) {
                gateup_mfma<2>(arow0, arow1, xrow, xrow_row, piece, lds, act0, act1, w.count);
            } else if (nblk <= 4) {
                gateup_mfma<4>(arow0, arow1, xrow, xrow_row, piece, lds, act0, act1, w.count);
            } else {
                gateup_mfma<8>(arow0, arow1, xrow, xrow_row, piece, lds, act0, act1, w.count);
            }
        }
        __builtin_amdgcn_s_waitcnt(0);  // this wave's act rows are written
        __syncthreads();
        if (tid == 0) __hip_atomic_fetch_add(a.ws.unit_done + u, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        cur = publish(claimed);
    }

    // ---- down items, one per (unit, quarter of the output rows) ----
    // The unit's act rows are staged in LDS once, then the item's 4 tiles of
    // 128 rows run in turn.  Each wave holds its 16 rows of a tile over
    // k = 512 (16 MFMA A operands per lane) in one of two register sets, and
    // issues the following tile's rows -- after the third tile, the next
    // item's first -- once the current tile's have arrived, so a wave
    // always has one tile's rows in flight while it multiplies.  (The
    // explicit waits keep the memory counter exact around the stores and
    // branches: it retires in order.)
    const int wave = tid >> 6;
    const int lane = tid & 63;
    const int m = lane & 15;
    const int g = lane >> 4;
    struct DnItem {
        const uint16_t* arow;  // this lane's first weight element of the item's first tile
        int u, h0, pair0, count;
    };
    auto dn_info = [&](int item, DnItem& d) {
        const int j = item - n_gu;
        Unit w;
        d.u = first + j / kDnItems;
        load_unit(a, d.u, w);
        d.h0 = kDnRows * kDnItemTiles * (j % kDnItems) + 16 * wave;
        d.arow = w.down + static_cast<size_t>(d.h0 + m) * kInner + 8 * g;
        d.pair0 = w.pair0;
        d.count = w.count;
    };
    auto tile_rows = [&](const uint16_t* arow, uint4* wt) {
#pragma unroll
        for (int s = 0; s < kInner / 32; ++s) wt[s] = ldg16(arow + 32 * s);
    };
    auto tile_mfma = [&](const DnItem& d, int t, const uint4* wt) {
        const int nb = (d.count + 15) / 16;
        for (int b = 0; b < nb; ++b) {
            const uint16_t* bp = lds + (16 * b + m) * kActStride + 8 * g;
            f32x4 acc0 = {0.0f, 0.0f, 0.0f, 0.0f}, acc1 = {0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
            for (int s = 0; s < kInner / 32; s += 2) {
                acc0 = mfma16x16x32(wt[s], *reinterpret_cast<const uint4*>(bp + 32 * s), acc0);
                acc1 = mfma16x16x32(wt[s + 1], *reinterpret_cast<const uint4*>(bp + 32 * (s + 1)), acc1);
            }
            const f32x4 y = acc0 + acc1;
            const int col = 16 * b + m;
            if (col < d.count) {
                uint16_t* dst = a.ws.y + static_cast<size_t>(d.pair0 + col) * kHidden + d.h0 + kDnRows * t + 4 * g;
                *reinterpret_cast<uint2*>(dst) = make_uint2(pack_bf2(y[0], y[1]), pack_bf2(y[2], y[3]));
            }
        }
    };
    constexpr size_t kTileStride = static_cast<size_t>(kDnRows) * kInner;
    uint4 wa[kInner / 32], wb[kInner / 32];
    DnItem d;
    if (cur < n_items) {
        dn_info(cur, d);
        tile_rows(d.arow, wa);
    }
    while (cur < n_items) {
        // The unit's 4 gate/up items have counted themselves in (bounded wait).
        if (tid == 0 && ld_agent32(a.ws.unit_done + d.u) < static_cast<uint32_t>(kGuTiles)) {
            const uint64_t start = wall_clock64();
            while (ld_agent32(a.ws.unit_done + d.u) < static_cast<uint32_t>(kGuTiles)) {
                if (wall_clock64() - start > kPfSpinTicks) {
                    timeout_s = 1;
                    break;
                }
                __builtin_amdgcn_s_sleep(2);
            }
        }
        __syncthreads();
        // The unit's act rows (1 KiB each, written by other workgroups of
        // this launch: agent-scope loads; rows past the unit's count read as
        // zeros).
        const uint16_t* act = a.ws.act + static_cast<size_t>(d.pair0) * kInner;
        const uint32_t act_bytes = static_cast<uint32_t>(d.count) * kInner * 2;
        uint4 st[kDnPieces];
#pragma unroll
        for (int q = 0; q < kDnPieces; ++q) st[q] = ld_agent16(act, static_cast<uint32_t>((tid + kDnThreads * q) * 16), act_bytes);
#pragma unroll
        for (int q = 0; q < kDnPieces; ++q) {
            const int idx = tid + kDnThreads * q;
            *reinterpret_cast<uint4*>(lds + (idx / 64) * kActStride + 8 * (idx % 64)) = st[q];
        }
        __syncthreads();
        __builtin_amdgcn_s_waitcnt(0);
        tile_rows(d.arow + kTileStride, wb);
        tile_mfma(d, 0, wa);
        __builtin_amdgcn_s_waitcnt(0);
        uint32_t claimed = 0u;
        if (tid == 0) claimed = take();
        tile_rows(d.arow + 2 * kTileStride, wa);
        tile_mfma(d, 1, wb);
        __builtin_amdgcn_s_waitcnt(0);
        tile_rows(d.arow + 3 * kTileStride, wb);
        tile_mfma(d, 2, wa);
        const int next = publish(claimed);
        DnItem dn = d;  // past the list's end: a harmless reload of this item's first tile
        if (next < n_items) dn_info(next, dn);
        __builtin_amdgcn_s_waitcnt(0);
        tile_rows(dn.arow, wa);
        tile_mfma(d, 3, wb);
        __syncthreads();  // every wave is done with the act rows in LDS
        cur = next;
        d = dn;
    }
    __builtin_amdgcn_s_waitcnt(0);  // the last reload is dropped
    if (tid == 0 && timeout_s) atomicOr(&a.ws.control->status, kStatusTimeoutPf);
}

int max_units(int tokens) {
    return (tokens + kPassTok - 1) / kPassTok + kExperts + (kTopK * tokens + kPassTok - 1) / kPassTok;
}

}  // namespace

size_t prefill_experts_lds() {
    const size_t gateup = static_cast<size_t>(2) * kPassTok * kXsStride * sizeof(uint16_t);
    const size_t down = static_cast<size_t>(kPassTok) * kActStride * sizeof(uint16_t);
    return gateup > down ? gateup : down;
}

hipError_t launch_prefill_plan(const uint16_t* logits, const int64_t* indices_in, const uint16_t* weights_in,
                               int64_t* indices, uint16_t* weights, int tokens, int shared_present,
                               const Workspace& ws, const Plan& plan, hipStream_t stream) {
    if (tokens <= 0) return hipSuccess;
    const int nblk = (tokens + kBlkTok - 1) / kBlkTok;
    hipLaunchKernelGGL(pf_topk, dim3(nblk), dim3(256), 0, stream, logits, indices_in, weights_in, indices, weights,
                       tokens, ws);
    hipLaunchKernelGGL(pf_scan, dim3(kExperts), dim3(256), 0, stream, nblk, ws, plan);
    hipLaunchKernelGGL(pf_fill, dim3(nblk), dim3(256), 0, stream, indices_in ? indices_in : indices, tokens,
                       shared_present, ws, plan);
    return hipGetLastError();
}

hipError_t launch_prefill_experts(const ExpertArgs& a, hipStream_t stream) {
    int device = 0;
    hipError_t err = hipGetDevice(&device);
    if (err != hipSuccess) return err;
    if (device < 0 || device >= 64) return hipErrorInvalidDevice;
    static int cus[64] = {0};  // per device: CU count, 0 until the LDS limit is raised
    if (cus[device] == 0) {
        err = hipFuncSetAttribute(reinterpret_cast<const void*>(pf_experts), hipFuncAttributeMaxDynamicSharedMemorySize,
                                  static_cast<int>(prefill_experts_lds()));
        if (err != hipSuccess) return err;
        int n = 0;
        err = hipDeviceGetAttribute(&n, hipDeviceAttributeMultiprocessorCount, device);
        if (err != hipSuccess) return err;
        cus[device] = n;
    }
    // one workgroup per CU (all resident: the down items wait for gate/up
    // items), a multiple of the 8 lists
    const int grid = cus[device] / 8 * 8;
    if (grid < 8) return hipErrorNotSupported;
    const StageEvents ev = timing_events(kStageGateUp);
    LRMOE_LAUNCH(pf_experts, dim3(grid), dim3(kDnThreads), prefill_experts_lds(), stream, ev.start, ev.stop, a);
    return hipGetLastError();
}

}  // namespace lrmoe
