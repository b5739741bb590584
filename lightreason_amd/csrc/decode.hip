// Decode / verify MoE layer (T <= 16 tokens) as one persistent kernel.
//
// One 512-thread workgroup per CU.  Every workgroup
//   1. stages the layer input rows in LDS (RMSNorm (x*r)*(1+w) applied when
//      the layer norms, Qwen3_5MoeRMSNorm.forward) and computes the
//      shared-expert gate bf16(sigmoid(bf16(x.w))) of every token;
//   2. workgroups 0..31 compute 8 router rows each (fixed fp32 order, see
//      route.hip) and publish them;
//   3. builds the route plan itself from the logits (top-8 by eight wave-max
//      extractions, renormalised weights, the unique experts as slots in
//      discovery order -- token 0's routes first -- with their token lists,
//      per token its routes in ascending expert order: fused_experts.py:47-54,
//      block_experts.py:102-121), so no other kernel or host step is needed;
//      the first item's weights are already streaming by then;
//   4. walks its share of one list of 128 KiB work items, each item's
//      weights prefetched one item ahead (the first two items of a workgroup
//      are fixed by its index, later ones are claimed from a counter two
//      items ahead -- three with codec experts, the first three fixed -- so
//      faster workgroups take more of them):
//        A (slot, 16-row tile): gate and up rows 16i..16i+15 of an expert over
//          k = 2048 -> SwiGLU with the cpu_experts.c:59-62 rounding points ->
//          act rows;
//        B (slot, 128-row tile): down rows over k = 512 for the slot's tokens
//          -> y rows (bf16, cpu_experts.c:64-69);
//      slot 0 is the shared expert, slot s >= 1 the (s-1)-th unique routed
//      expert in discovery order; every token routed to an expert is an MFMA
//      column (tokens ascending), so each
//      weight byte is read from HBM once per call;
//        C (128-row tile), the last 16 items: once every slot's B item of the
//          tile is done, the ordered combine of that tile (fused_experts.py:
//          27-37: ascending expert, acc = bf16(acc + bf16(y * w)) from 0),
//          the shared-expert add bf16(sg * y_shared) and the residual add.
//
// Cross-workgroup data is written with agent-scope stores and read with
// agent-scope loads (coherent across the XCDs' L2s).  The router logits and
// the act and y rows are 8-byte words that carry the call's tag beside two
// bf16 values, so the plan knows its logits are complete, a B item its
// slot's act rows and a C item its tile's y rows, by checking the tags of
// what it loaded: no producer waits for its own stores or signals anything.  A B
// item needs its slot's A items and a C item its tile's B items, all earlier
// in the list; every workgroup takes its items in increasing list order and
// all workgroups are co-resident, so the earliest waiting item always has
// its inputs written or in progress and the waits end.  Every wait is
// bounded: on timeout the status word gets kStatusTimeout and the kernel
// still exits.  Each call uses one of two counter sets (by call parity) and
// zeroes the other for the next call.
#include "lrmoe_device.h"
#include "lrmoe_internal.h"

// Timeline build (compiled with -DLRMOE_TIMELINE into liblrmoe_timeline.so
// by `python -m lightreason_amd.build --timeline`; the product library has
// none of it): thread 0 of every workgroup stamps the 100 MHz wall clock at
// the phases of a single decode layer into LDS and, at the end, copies the
// stamps to the buffer given by lrmoe_timeline_set (kTimelineWords per
// workgroup).  Word 0 launch entry, 1 top-8 in the plan, 2 first item's
// loads issued (wave 0), 3 plan done, 4 items done, 5 first item's loads
// issued (wave 7), 6 token rows staged, 7 call counters read; 8 + 5n the
// n-th item step (n < 22): start, its weights in, its inputs in, end, and
// item code (kind + 1) * 1e6 + slot * 1e3 + tile; 118 wave 0's top-8
// extracted, 119 expert masks built, 120 slots numbered, 121 token rows
// staged (wave 7), 122 token rows staged before the router, 123 router
// logits published (router workgroups), 124 every logit's tag seen, 125 the
// first half of the first item's loads issued (wave 0).
#ifdef LRMOE_TIMELINE
__device__ unsigned long long* g_timeline;
extern "C" int lrmoe_timeline_set(void* p) {
    return static_cast<int>(hipMemcpyToSymbol(HIP_SYMBOL(g_timeline), &p, sizeof(p)));
}
#define TL_DECLARE __shared__ unsigned long long tl_stamps[lrmoe::kTimelineWords]
#define TL(k, thread)                                                                                  \
    do {                                                                                               \
        if (threadIdx.x == (thread) && (k) < lrmoe::kTimelineWords) tl_stamps[(k)] = wall_clock64();   \
    } while (0)
#define TL_WORD(k, v)                                                                \
    do {                                                                             \
        if (threadIdx.x == 0 && (k) < lrmoe::kTimelineWords) tl_stamps[(k)] = (v);   \
    } while (0)
#define TL_CLEAR                                                                     \
    do {                                                                             \
        if (threadIdx.x < lrmoe::kTimelineWords) tl_stamps[threadIdx.x] = 0ull;      \
    } while (0)
#define TL_FLUSH(layer)                                                                                    \
    do {                                                                                                   \
        if ((layer) == 0 && g_timeline != nullptr && threadIdx.x < lrmoe::kTimelineWords)                  \
            g_timeline[blockIdx.x * lrmoe::kTimelineWords + threadIdx.x] = tl_stamps[threadIdx.x];         \
    } while (0)
#else
#define TL_DECLARE
#define TL(k, thread)
#define TL_WORD(k, v)
#define TL_CLEAR
#define TL_FLUSH(layer)
#endif

namespace lrmoe {
namespace {

[[maybe_unused]] constexpr int kTimelineWords = 128;  // timeline build: stamps per workgroup
constexpr int kWaves = 8;
constexpr int kThreads = kWaves * kWave;
constexpr int kMaxT = kDecodeMaxTokens;
constexpr int kATiles = kInner / 16;          // 32 A items per slot
constexpr int kBRows = 128;                   // output rows per B item
constexpr int kBTiles = kHidden / kBRows;     // 16 B items per slot
constexpr int kRouterWgs = kExperts / kWaves; // 32 workgroups x 8 router rows
constexpr int kXStride = kHidden + 8;         // LDS token row stride (bf16)
constexpr int kActStride = kInner + 8;        // LDS act row stride (bf16)
constexpr int kLoads = 16;                    // 16-byte weight loads per lane per item
// Raw items load their weights as 4 rows x 256 B per instruction (16-byte
// non-temporal loads; load i: MFMA row 4 (i % 4) + lane / 16 of the wave's
// 16, bytes 256 (i / 4) + 16 (lane % 16) of the row's slice) and pass them
// through a per-wave LDS stage of 16 rows x 256 B (+16 B pad: conflict-free
// in both directions) into the MFMA layout (lane (m, g) of step q: row m,
// elements 32 q + 8 g ..).  An instruction then covers four rows' whole
// 128-byte lines instead of sixteen rows' half lines: the HBM stream of a
// C2 layer runs about 7% faster.  Every MFMA sees the operands, in the
// order, of loads made directly in the MFMA layout.
constexpr int kStageRow = 256 + 16;           // bytes per staged row
constexpr int kStageBytes = 16 * kStageRow;   // per wave
constexpr int kCombineItems = kBTiles;        // C items, one per 128-row output tile
constexpr uint64_t kSpinTicks = 5000000;      // 50 ms of the 100 MHz wall clock
// gfx9 s_waitcnt immediate: vmcnt[3:0] | expcnt << 4 | lgkmcnt << 8 | vmcnt[5:4] << 14.
constexpr int kWaitVm16 = (16 & 15) | (7 << 4) | (15 << 8) | ((16 >> 4) << 14);

// ---- agent-scope memory operations (coherent across XCDs): lrmoe_device.h ----

// Four agent-scope (sc1) 8-byte loads at a uniform base plus a per-lane byte
// offset.  Written as assembly so that the compiler's wait insertion does not
// tie the next prefetch to them; the caller's "s_waitcnt vmcnt(16)" after
// that prefetch is what makes the results valid.
__device__ __forceinline__ void ld_agent64x4_async(uint64_t* out, const void* base, uint32_t byte_offset) {
    asm volatile(
        "global_load_dwordx2 %0, %4, %5 sc1\n\t"
        "global_load_dwordx2 %1, %4, %5 offset:8 sc1\n\t"
        "global_load_dwordx2 %2, %4, %5 offset:16 sc1\n\t"
        "global_load_dwordx2 %3, %4, %5 offset:24 sc1"
        : "=&v"(out[0]), "=&v"(out[1]), "=&v"(out[2]), "=&v"(out[3])
        : "v"(byte_offset), "s"(base)
        : "memory");
}

// Claims a work item: one agent-scope fetch-add by the lanes in `lanes`
// (wave-uniform: 1 = lane 0 in the claiming wave, 0 in the others), written
// as assembly so that no wait is tied to it.  The result is
// valid in lane 0 once the caller's "s_waitcnt vmcnt(16)" after the next
// prefetch has passed (returning atomics count in vmcnt, in order).
__device__ __forceinline__ uint32_t claim_async(uint32_t* counter, uint32_t lanes) {
    // The address operand must be scalar: pass it through readfirstlane (a
    // uniform value computed in vector registers is not moved by itself).
    counter = reinterpret_cast<uint32_t*>(uniform64(reinterpret_cast<uint64_t>(counter)));
    uint32_t old;
    uint64_t saved_exec;
    uint32_t mask;
    asm volatile(
        "v_readfirstlane_b32 %2, %6\n\t"
        "s_nop 4\n\t"
        "s_mov_b64 %1, exec\n\t"
        "s_mov_b32 exec_lo, %2\n\t"
        "s_mov_b32 exec_hi, 0\n\t"
        "global_atomic_add %0, %3, %4, %5 sc0\n\t"
        "s_mov_b64 exec, %1"
        : "=&v"(old), "=&s"(saved_exec), "=&s"(mask)
        : "v"(0u), "v"(1u), "s"(counter), "v"(lanes)
        : "memory");
    return old;
}

__device__ __forceinline__ uint64_t now_ticks() { return wall_clock64(); }


// 16 bytes of token rows at base + byte_offset (base wave-uniform).  In a
// chain, the rows were written by other workgroups of the same launch
// (possibly through another XCD's L2), so they are read with agent-scope
// (sc1) buffer loads.
template <bool kChained>
__device__ __forceinline__ uint4 ld_row16(const uint16_t* base, uint32_t byte_offset) {
    if constexpr (kChained) {
        return ld_agent16(base, byte_offset);
    } else {
        return ldg16(reinterpret_cast<const uint8_t*>(base) + byte_offset);
    }
}
template <bool kChained>
__device__ __forceinline__ uint64_t ld_row8(const uint16_t* p) {
    if constexpr (kChained) {
        return ld_agent64(p);
    } else {
        return *reinterpret_cast<const uint64_t*>(p);
    }
}
template <bool kChained>
__device__ __forceinline__ void st_row8(uint16_t* p, uint64_t v) {
    if constexpr (kChained) {
        st_agent64(p, v);
    } else {
        *reinterpret_cast<uint64_t*>(p) = v;
    }
}

// The call tag of a tagged 8-byte word.
__device__ __forceinline__ uint32_t tag_of(uint64_t word) { return static_cast<uint32_t>(word >> kDecodeTagShift); }

__device__ __forceinline__ uint64_t pack4(const uint32_t* v) {
    return static_cast<uint64_t>(v[0] | (v[1] << 16)) | (static_cast<uint64_t>(v[2] | (v[3] << 16)) << 32);
}

// ---- per-workgroup plan (LDS) -------------------------------------------------

struct SlotInfo {
    const uint16_t* gate;  // gate rows [512][2048]
    const uint16_t* up;    // up rows [512][2048]
    const uint16_t* down;  // [2048][512]
    uint32_t tok[4];       // token of column n in byte n
    int32_t count;         // tokens (columns), <= 16
    int32_t pair0;         // first act/y row
    int32_t pad[2];
};

// The tile-codec rows of a slot's expert (codec calls only).
struct SlotCodec {
    const uint8_t* pk_gu;  // tile-codec gate_up [1024 rows][8 tiles][384 B], or null (raw expert)
    const uint8_t* pk_dn;  // tile-codec down [2048][2][384]
    const uint8_t* b_gu;   // tile bases of gate_up [1024][8]
    const uint8_t* b_dn;   // tile bases of down [2048][2]
    int32_t crow;          // row of Plan::ecodec holding the expert's raw flags
    int32_t pad;
};

// kCodec: the codec kernel's plan (the other one carries no codec tables).
template <bool kCodec>
struct Plan {
    SlotInfo slot[kDecodeSlots];
    SlotCodec scodec[kCodec ? kDecodeSlots : 1];   // codec calls
    int16_t comb_pair[kMaxT][kTopK];  // per token: pair of the k-th smallest expert
    float comb_w[kMaxT][kTopK];       // its routing weight
    float sg[kMaxT];                  // shared-expert gate per token
    int32_t ids[kMaxT][kTopK];        // routed experts, rank order
    uint16_t wts[kMaxT][kTopK];       // routing weights (bf16), rank order
    uint4 eptr[kExperts];             // (gate_up, down) address of every expert
    uint4 ecodec[kCodec ? kExperts + 1 : 1][5];  // codec table rows of every expert and the shared one (codec calls):
                                      // 4 addresses, then 48 bytes of per-(item, wave) raw flags
    uint32_t tokmask[kExperts];
    uint32_t poff[kExperts];
    uint32_t scan[4];
    uint16_t lg[kMaxT][kWaves];       // router prologue: this workgroup's 8 logits per token
    int32_t n_slots;                  // active slots (shared + unique routed)
    int32_t first_slot;               // 0 with a shared expert, else 1
    int32_t status;
    int32_t claim[2];                 // claimed item index, by step parity
    uint32_t vote[2][kWaves];         // block_or: per-wave votes, two alternating rows
};

// Block-wide OR of a predicate.  Every thread of the workgroup calls it, in
// the same order, with the same `row` (flipped by each call).  A wave ballot
// and one LDS word per wave, then one barrier: a row is written again only
// two votes later, after a barrier that every thread reaches once it has read
// the row.  (__syncthreads_or reads the workgroup size from the dispatch
// packet with vector loads; the wait for those also waits for every older
// load in flight, such as the next item's prefetch.)
template <typename PlanT>
__device__ __forceinline__ bool block_or(bool pred, PlanT& P, int& row, int wave, int lane) {
    const uint64_t ballot = __ballot(pred);
    if (lane == 0) P.vote[row][wave] = ballot != 0ull ? 1u : 0u;
    __syncthreads();
    uint32_t any = 0u;
#pragma unroll
    for (int w = 0; w < kWaves; ++w) any |= P.vote[row][w];
    row ^= 1;
    return any != 0u;
}

// Dot of a lane's 32 contiguous elements (4 x 16 bytes) with the same
// elements of an LDS row, as an in-order fmaf chain from +0.
__device__ __forceinline__ float lane_dot32(const uint4* w, const uint16_t* row, int lane) {
    const uint4* x = reinterpret_cast<const uint4*>(row + 32 * lane);
    float acc = 0.0f;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        float wf[8], xf[8];
        unpack8(w[i], wf);
        unpack8(x[i], xf);
#pragma unroll
        for (int j = 0; j < 8; ++j) acc = __builtin_fmaf(wf[j], xf[j], acc);
    }
    return acc;
}

// Weight addresses of a slot: the raw rows, and (sc not null) the tile-codec
// rows when the expert has them (codec = {packed gate_up, packed down,
// gate_up bases, down bases} as two uint4, or null; crow = its row of
// Plan::ecodec).
__device__ __forceinline__ void set_slot_weights(SlotInfo& s, SlotCodec* sc, const uint16_t* gate,
                                                 const uint16_t* up, const uint16_t* down, const uint4* codec,
                                                 int crow) {
    auto ptr = [](uint32_t lo, uint32_t hi) {
        return reinterpret_cast<const uint8_t*>(static_cast<uintptr_t>(lo) | (static_cast<uintptr_t>(hi) << 32));
    };
    s.gate = gate;
    s.up = up;
    s.down = down;
    if (sc == nullptr) return;
    sc->pk_gu = codec != nullptr ? ptr(codec[0].x, codec[0].y) : nullptr;
    sc->pk_dn = codec != nullptr ? ptr(codec[0].z, codec[0].w) : nullptr;
    sc->b_gu = codec != nullptr ? ptr(codec[1].x, codec[1].y) : nullptr;
    sc->b_dn = codec != nullptr ? ptr(codec[1].z, codec[1].w) : nullptr;
    sc->crow = crow;
}

// ---- item geometry ------------------------------------------------------------

struct Item {
    int kind;   // 0 = A (gate/up), 1 = B (down), 2 = C (combine), -1 = none
    int slot;
    int tile;
};

__device__ __forceinline__ Item item_at(int k, int total, int n_slots, int first_slot) {
    Item it;
    const int n_a = kATiles * n_slots;
    if (k >= total + kCombineItems || n_slots == 0) {
        it.kind = -1;
        it.slot = first_slot;
        it.tile = 0;
    } else if (k >= total) {
        it.kind = 2;
        it.slot = first_slot;
        it.tile = k - total;
    } else if (k < n_a) {
        it.kind = 0;
        it.slot = first_slot + k / kATiles;
        it.tile = k % kATiles;
    } else {
        const int b = k - n_a;
        it.kind = 1;
        it.slot = first_slot + b / kBTiles;
        it.tile = b % kBTiles;
    }
    return it;
}

// Address of this lane's first 16-byte weight load of an item; the item's 16
// loads are at +32 elements each.  A: MFMA row m < 8 is gate row
// 16*tile + 8*(wave/4) + m, m >= 8 the up row with the same index; k starts at
// 512*(wave%4).  B: output row 128*tile + 16*wave + m over k = 512.
__device__ __forceinline__ const uint16_t* item_base(const SlotInfo& s, const Item& it, int wave, int lane) {
    const int m = lane & 15;
    const int g = lane >> 4;
    if (it.kind == 1) {
        return s.down + static_cast<size_t>(kBRows * it.tile + 16 * wave + m) * kInner + 8 * g;
    }
    const uint16_t* rows = m < 8 ? s.gate : s.up;
    const int row = 16 * it.tile + 8 * (wave >> 2) + (m & 7);
    return rows + static_cast<size_t>(row) * kHidden + kInner * (wave & 3) + 8 * g;
}

// The four row pointers of a lane's staged loads of an item (row
// 4 a + lane / 16 of the wave's 16 MFMA rows, at element 8 (lane % 16) of
// the wave's k slice); load 4 j + a reads 16 bytes at rows[a] + 128 j.
__device__ __forceinline__ void item_rows(const SlotInfo& s, const Item& it, int wave, int lane,
                                          const uint16_t* (&rows)[4]) {
    const int r = lane >> 4;
    const int e = 8 * (lane & 15);
#pragma unroll
    for (int a = 0; a < 4; ++a) {
        if (it.kind == 1) {
            rows[a] = s.down + static_cast<size_t>(kBRows * it.tile + 16 * wave + 4 * a + r) * kInner + e;
        } else {
            // MFMA rows 0..7 are gate rows, 8..15 up rows
            const int row = 16 * it.tile + 8 * (wave >> 2) + 4 * (a & 1) + r;
            rows[a] = (a < 2 ? s.gate : s.up) + static_cast<size_t>(row) * kHidden + kInner * (wave & 3) + e;
        }
    }
}

__device__ __forceinline__ void issue_rows(const uint16_t* const (&rows)[4], uint4* buf) {
#pragma unroll
    for (int i = 0; i < kLoads; ++i) buf[i] = ldg16_nt(rows[i & 3] + 128 * (i >> 2));
}

// The MFMAs of a raw item whose staged loads are in buf, B operand rows at
// bp (32 elements per step): per 128-element span j, the wave's four loads
// 4 j .. 4 j + 3 into its LDS stage, then steps 4 j .. 4 j + 3 read back in
// the MFMA layout (even steps into acc0, odd ones into acc1, in order).
__device__ __forceinline__ void staged_mfmas(const uint4* buf, uint8_t* stage, const uint16_t* bp, int lane,
                                             f32x4& acc0, f32x4& acc1) {
    const int m = lane & 15;
    const int g = lane >> 4;
#pragma unroll
    for (int j = 0; j < kLoads / 4; ++j) {
#pragma unroll
        for (int a = 0; a < 4; ++a)
            *reinterpret_cast<uint4*>(stage + (4 * a + (lane >> 4)) * kStageRow + 16 * (lane & 15)) = buf[4 * j + a];
        // (the stage is the wave's own: in-order LDS access within the wave,
        // and no reordering by the compiler across these fences)
        __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
        __builtin_amdgcn_wave_barrier();
        __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
        uint4 op[4];
#pragma unroll
        for (int q = 0; q < 4; ++q) op[q] = *reinterpret_cast<const uint4*>(stage + m * kStageRow + 16 * (4 * q + g));
        __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
        __builtin_amdgcn_wave_barrier();
        __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
#pragma unroll
        for (int q = 0; q < 4; q += 2) {
            acc0 = mfma16x16x32(op[q], *reinterpret_cast<const uint4*>(bp + 32 * (4 * j + q)), acc0);
            acc1 = mfma16x16x32(op[q + 1], *reinterpret_cast<const uint4*>(bp + 32 * (4 * j + q + 1)), acc1);
        }
    }
}

// Tile-codec rows of a lane in an item of a codec slot (format in
// codec.hip): the lane's MFMA row has two tiles in the item's k range (A:
// tiles 2q, 2q+1 of the gate/up row, q = wave % 4; B: tiles 0, 1 of the down
// row), with their bases side by side (an even byte).  Per tile the lane
// issues 8 loads, like the 8 of a raw row's tile: when the tile fits the
// codec, its six 16-byte blocks at tile + 16g + 64u (u = 0..5, the offsets of
// the raw loads) and the 16-byte aligned block holding both bases, twice.
struct PackedLane {
    const uint8_t* tile0;    // first of the lane's two tiles
    const uint8_t* bases16;  // 16-byte block holding its two tile bases
    const uint8_t* bases2;   // the two bases
    int base_byte;           // byte of the first base in that block
};

__device__ __forceinline__ PackedLane packed_lane(const SlotCodec& s, const Item& it, int wave, int lane) {
    const int m = lane & 15;
    PackedLane p;
    uintptr_t b;
    if (it.kind == 1) {
        const int row = kBRows * it.tile + 16 * wave + m;
        p.tile0 = s.pk_dn + static_cast<size_t>(row) * 2 * kCodecTileBytes;
        b = reinterpret_cast<uintptr_t>(s.b_dn) + static_cast<uintptr_t>(row) * 2;
    } else {
        // Gate row (m < 8) or up row (m >= 8) 16*tile + 8*(wave/4) + m%8 of the packed gate_up.
        const int row = (m < 8 ? 0 : kInner) + 16 * it.tile + 8 * (wave >> 2) + (m & 7);
        const int q = wave & 3;
        p.tile0 = s.pk_gu + (static_cast<size_t>(row) * 8 + 2 * q) * kCodecTileBytes;
        b = reinterpret_cast<uintptr_t>(s.b_gu) + static_cast<uintptr_t>(row) * 8 + 2 * q;
    }
    p.bases2 = reinterpret_cast<const uint8_t*>(b);
    p.bases16 = reinterpret_cast<const uint8_t*>(b & ~static_cast<uintptr_t>(15));
    p.base_byte = static_cast<int>(b & 15);
    return p;
}

// Byte i (0..15) of a 16-byte block, by shifts (an indexed pick of a
// component would put the whole register array in scratch memory).
__device__ __forceinline__ uint32_t byte_of(const uint4& v, int i) {
    const uint64_t lo = static_cast<uint64_t>(v.x) | (static_cast<uint64_t>(v.y) << 32);
    const uint64_t hi = static_cast<uint64_t>(v.z) | (static_cast<uint64_t>(v.w) << 32);
    return static_cast<uint32_t>(((i < 8 ? lo : hi) >> (8 * (i & 7))) & 0xffu);
}

// Register order of a raw tile's 8 loads (every item, so that one load
// sequence serves all): register 8t + j holds k-step 8t + kRawStep[j].  Packed, register j
// holds block j, whose last reader is k-step 1, 3, 5, 7, 3, 7 for j = 0..5
// (registers 6, 7: the bases, read first); this order ends each register's
// raw use near its packed one, which keeps the registers of a wave that
// mixes packed and raw lanes free as early as those of a packed one.
__device__ constexpr int kRawStep[8] = {2, 3, 5, 6, 4, 7, 0, 1};
__device__ constexpr int raw_reg(int s) {
    const int u = s & 7;
    int j = 0;
    for (int i = 0; i < 8; ++i) j = kRawStep[i] == u ? i : j;
    return (s & 8) + j;
}

// a where mask is all ones, b where it is zero: v_bfi_b32 per word (a
// conditional would let the compiler branch around the computation of a;
// the same bit operations in C become two instructions).
__device__ __forceinline__ uint32_t bfi(uint32_t mask, uint32_t a, uint32_t b) {
    uint32_t r;
    asm("v_bfi_b32 %0, %1, %2, %3" : "=v"(r) : "v"(mask), "v"(a), "v"(b));
    return r;
}
__device__ __forceinline__ uint4 pick(uint32_t mask, const uint4& a, const uint4& b) {
    return make_uint4(bfi(mask, a.x, b.x), bfi(mask, a.y, b.y), bfi(mask, a.z, b.z), bfi(mask, a.w, b.w));
}

// A bases pair of two tiles that do not fit the codec: the dummy source of
// items without codec rows.
__device__ const uint16_t kBothMisfit = 0xffffu;

// The MFMA A operand of k-step s (0..15) of a lane's packed tile s / 8: the
// 8 bf16 values a raw item's load s holds (k = 8g + 32s .. +7 of the lane's
// row); base4 = the tile's base * 0x01010101.
__device__ __forceinline__ uint4 packed_operand(const uint4* buf, int s, uint32_t base4) {
    const int t = s >> 3;
    const int u = s & 7;
    const uint4 l = buf[8 * t + (u >> 1)];
    const uint32_t lo = (u & 1) ? l.z : l.x;
    const uint32_t hi = (u & 1) ? l.w : l.y;
    const uint4 cq = buf[8 * t + 4 + (u >> 2)];
    const uint32_t c = (u & 3) == 0 ? cq.x : (u & 3) == 1 ? cq.y : (u & 3) == 2 ? cq.z : cq.w;
    return codec_decode8(lo, hi, c, base4);
}

__device__ __forceinline__ int column_token(const SlotInfo& s, int n) {
    return static_cast<int>((s.tok[n >> 2] >> (8 * (n & 3))) & 0xffu);
}

// Ordered combine of output rows [128*tile, +128) of every token (512
// threads: token tid/32, rows 4*(tid%32)..+3), then the shared-expert and
// residual adds.  The tile's y words are reloaded (bounded) until each
// carries this call's tag.
template <bool kChained, typename PlanT>
__device__ __forceinline__ void combine_tile(const DecodeArgs& a, PlanT& P, int tid, int tile, int T, bool shared,
                                             uint32_t tag, int& vote_row) {
    const int wave = tid >> 6;
    const int lane = tid & 63;
    const int t = tid >> 5;
    const bool active = t < T;
    const int h = kBRows * tile + (tid & 31) * 4;
    // One pass over the pairs in combine order; it reports whether any word
    // was stale (the sums of such a pass are discarded and the pass re-run).
    // The pass's loads are all issued before any is used, so that their
    // latencies overlap.
    float acc[4];
    auto pass = [&]() {
        bool stale = false;
#pragma unroll
        for (int i = 0; i < 4; ++i) acc[i] = 0.0f;
        if (!active) return false;
        uint64_t words[kTopK + 1][2];
#pragma unroll
        for (int q = 0; q <= kTopK; ++q) {
            const int pair = q < kTopK ? P.comb_pair[t][q] : kTopK * T + t;
            const uint64_t* row = a.y + static_cast<size_t>(pair) * (kHidden / 2) + h / 2;
            if (q < kTopK || shared) {
                words[q][0] = ld_agent64(row);
                words[q][1] = ld_agent64(row + 1);
            }
        }
#pragma unroll
        for (int q = 0; q <= kTopK; ++q) {
            if (q == kTopK && !shared) break;
            const uint64_t w0 = words[q][0];
            const uint64_t w1 = words[q][1];
            stale |= static_cast<uint32_t>(w0 >> kDecodeTagShift) != tag ||
                     static_cast<uint32_t>(w1 >> kDecodeTagShift) != tag;
            const uint32_t bits[4] = {static_cast<uint32_t>(w0) & 0xffffu, static_cast<uint32_t>(w0 >> 16) & 0xffffu,
                                      static_cast<uint32_t>(w1) & 0xffffu, static_cast<uint32_t>(w1 >> 16) & 0xffffu};
            const float w = q < kTopK ? P.comb_w[t][q] : P.sg[t];
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                // acc + bf16(y * w) for a routed pair, acc + bf16(gate * y) for the shared row.
                const float prod = q < kTopK ? bf2f(bits[i]) * w : w * bf2f(bits[i]);
                acc[i] = rbf(acc[i] + rbf(prod));
            }
        }
        return stale;
    };
    if (block_or(pass(), P, vote_row, wave, lane)) {
        const uint64_t start = now_ticks();
        while (true) {
            if (block_or(now_ticks() - start > kSpinTicks, P, vote_row, wave, lane)) {
                if (tid == 0) P.status |= kStatusTimeout;
                break;
            }
            __builtin_amdgcn_s_sleep(2);
            if (!block_or(pass(), P, vote_row, wave, lane)) break;
        }
    }
    if (active) {
        if (a.residual) {
            const uint64_t x = ld_row8<kChained>(a.x + static_cast<size_t>(t) * kHidden + h);
#pragma unroll
            for (int i = 0; i < 4; ++i) acc[i] = rbf(bf2f(static_cast<uint32_t>(x >> (16 * i)) & 0xffffu) + acc[i]);
        }
        uint32_t o[4];
#pragma unroll
        for (int i = 0; i < 4; ++i) o[i] = f2bf(acc[i]);
        st_row8<kChained>(a.out + static_cast<size_t>(t) * kHidden + h, pack4(o));
    }
}

// One decode layer, run by every workgroup of the grid.  `finished` is the
// value of DecodeSync::finished read at the start of the launch, `layer` the
// index of this layer in the launch (0 for a single layer).  wait_input() is
// called by every thread once the loads that do not depend on the layer
// input are issued; it returns when the input rows are complete.  Ends with
// all of the workgroup's memory operations complete; returns kStatusTimeout
// when one of its bounded waits expired.
template <bool kChained, bool kCodec, typename WaitInput>
__device__ __forceinline__ int32_t decode_layer(const DecodeArgs& a, Plan<kCodec>& P, uint8_t* dyn,
                                                unsigned long long finished, int layer, WaitInput wait_input) {
    const int T = a.tokens;
    // Thread and workgroup indices as opaque values: what is derived from
    // them is computed again for each layer of a chain rather than held in
    // registers across layers.
    int lane = static_cast<int>(threadIdx.x & 63);
    int wave = __builtin_amdgcn_readfirstlane(static_cast<int>(threadIdx.x >> 6));
    int block = static_cast<int>(blockIdx.x);
    asm volatile("" : "+v"(lane));
    asm volatile("" : "+s"(wave), "+s"(block));
    const int tid = wave * kWave + lane;
    const int G = gridDim.x;
    uint16_t* x_lds = reinterpret_cast<uint16_t*>(dyn);                       // [T][kXStride]
    uint16_t* act_lds = x_lds + T * kXStride;                                  // [16][kActStride]
    f32x4* part = reinterpret_cast<f32x4*>(act_lds + kMaxT * kActStride);      // [2][8][64]
    // the wave's weight stage (raw kernel only)
    uint8_t* const stage = reinterpret_cast<uint8_t*>(part + 2 * kWaves * kWave) + (kCodec ? 0 : wave * kStageBytes);
    DecodeSync* sync = a.sync;
    TL_DECLARE;
    TL_CLEAR;
    TL(0, 0);

    // ---- 1. every load that depends on nothing, issued first ----
    // In order of need: the caller's logits rows of this wave's tokens
    // (tokens wave and wave + 8), the 256-entry expert address table, the
    // token rows, the RMSNorm and shared-gate rows and a router workgroup's
    // router row.
    const int t_lo = wave;
    const int t_hi = wave + kWaves;
    const bool has_lo = t_lo < T;
    const bool has_hi = t_hi < T;
    const bool router_wg = a.router != nullptr && block < kRouterWgs;
    const bool logits_given = a.logits_in != nullptr;
    const uint16_t* lg_src = logits_given ? a.logits_in : a.x;
    uint64_t lg_lo = 0ull, lg_hi = 0ull;
    if (logits_given && has_lo) lg_lo = *reinterpret_cast<const uint64_t*>(lg_src + static_cast<size_t>(t_lo) * kExperts + 4 * lane);
    if (logits_given && has_hi) lg_hi = *reinterpret_cast<const uint64_t*>(lg_src + static_cast<size_t>(t_hi) * kExperts + 4 * lane);
    uint4 eptr = make_uint4(0u, 0u, 0u, 0u);
    if (tid < kExperts) eptr = ldg16(a.expert_ptrs + 2 * tid);
    // Codec table row of expert tid (tid 256: the shared expert).
    uint4 ec[5];
#pragma unroll
    for (int i = 0; i < 5; ++i) ec[i] = make_uint4(0u, 0u, 0u, 0u);
    if (kCodec && a.codec != nullptr && tid <= kExperts) {
#pragma unroll
        for (int i = 0; i < 5; ++i) ec[i] = ldg16(a.codec + kCodecTableColumns * tid + 2 * i);
    }
    // Rows are loaded only by the waves that use them (wave-uniform
    // branches): the norm and shared-gate rows by waves with a token, a
    // router row by the router workgroups.  Every load instruction costs
    // the CU's load path 1 KiB however few distinct bytes it reads, and the
    // prologue's loads are all issued before the first result is needed.
    const bool token_wave = has_lo || has_hi;
    const uint32_t xr_lo = static_cast<uint32_t>((t_lo * kHidden + 32 * lane) * 2);
    const uint32_t xr_hi = static_cast<uint32_t>((t_hi * kHidden + 32 * lane) * 2);
    uint4 x_lo[4], x_hi[4], w_norm[4], w_sg[4], w_router[4];
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        x_lo[i] = x_hi[i] = w_norm[i] = w_sg[i] = w_router[i] = make_uint4(0u, 0u, 0u, 0u);
    }
    if (token_wave && a.norm != nullptr) {
#pragma unroll
        for (int i = 0; i < 4; ++i) w_norm[i] = ldg16(a.norm + 32 * lane + 8 * i);
    }
    if (token_wave && a.shared_expert_gate != nullptr) {
#pragma unroll
        for (int i = 0; i < 4; ++i) w_sg[i] = ldg16(a.shared_expert_gate + 32 * lane + 8 * i);
    }
    if (router_wg) {
        const uint16_t* rr = a.router + static_cast<size_t>(kWaves * block + wave) * kHidden + 32 * lane;
#pragma unroll
        for (int i = 0; i < 4; ++i) w_router[i] = ldg16(rr + 8 * i);
    }
    if (tid < kExperts) P.tokmask[tid] = 0u;
    if (tid == 0) P.status = 0;
    // The layer input and the counters are touched only once the input is
    // complete (a chain waits for the previous layer here; the loads above
    // are already in flight).
    wait_input();
    if (has_lo) {
#pragma unroll
        for (int i = 0; i < 4; ++i) x_lo[i] = ld_row16<kChained>(a.x, xr_lo + 16 * i);
    }
    if (has_hi) {
#pragma unroll
        for (int i = 0; i < 4; ++i) x_hi[i] = ld_row16<kChained>(a.x, xr_hi + 16 * i);
    }
    // A workgroup's first item: item (block - 32) mod G with a router (the
    // router workgroups take items last), else item block.
    const int first_item = (block - (a.router != nullptr ? kRouterWgs : 0) + G) % G;
    // With a router and a shared expert (raw weights), the workgroups whose
    // first item is a shared-expert A tile (not named by routing) run it
    // while the router works, right after the token rows are staged; their
    // fixed items are then first_item + G and 2G + first_item, and claims
    // number items from 2G + kATiles on.  With every routed A item of a T=1
    // layer then in the first round, no down item waits for a second one.
    const bool early_path =  // launch-uniform; the early workgroups are not router workgroups
        !kCodec && a.router != nullptr && a.sh_down != nullptr && G >= kRouterWgs + kATiles;
    const bool early = early_path && first_item < kATiles;
    uint4 b0[kLoads], b1[kLoads];
    // Otherwise, a workgroup whose first item is a shared-expert A tile
    // brings that tile's 1,024 lines of 128 bytes into its L2 during
    // routing, one 4-byte load per line (two lines per lane), so that the
    // tile arrives from L2 when it is issued after top-8, ahead of the first
    // items of the other workgroups; the others load two words of the expert
    // table (read-only, cached).  Issued after the token rows, so that no
    // wait for those covers them, and after a chain's input wait, whose
    // poll would otherwise wait for them; consumed just before the first
    // item's loads.  (The warming loads are issued on every path, so that
    // the early tile's loads never reuse their registers: that reuse made
    // the compiler wait for every entry load before issuing the tile.)
    uint32_t warm0 = 0u, warm1 = 0u;
    {
        const bool warm = !early && a.sh_down != nullptr && first_item < kATiles;
        const int r = (2 * tid) / 32;     // row of the tile: 16 gate rows, then 16 up rows
        const int line = (2 * tid) % 32;  // first of the lane's two lines of that row
        const uint16_t* row = (r < 16 ? a.sh_gate + static_cast<size_t>(16 * first_item + r) * kHidden
                                      : a.sh_up + static_cast<size_t>(16 * first_item + r - 16) * kHidden);
        const uint16_t* table = reinterpret_cast<const uint16_t*>(a.expert_ptrs);
        const uint16_t* w0 = warm ? row + 64 * line : table;
        const uint16_t* w1 = warm ? row + 64 * (line + 1) : table + 2;
        warm0 = *reinterpret_cast<const __attribute__((address_space(1))) uint32_t*>(reinterpret_cast<uintptr_t>(w0));
        warm1 = *reinterpret_cast<const __attribute__((address_space(1))) uint32_t*>(reinterpret_cast<uintptr_t>(w1));
    }
    if (early) {
        SlotInfo sh;
        sh.gate = a.sh_gate;
        sh.up = a.sh_up;
        const uint16_t* rows[4];
        item_rows(sh, Item{0, 0, first_item}, wave, lane, rows);
        issue_rows(rows, b0);
    }
    // This call's number, tag and counter set, resolved where they are first
    // needed: before the router's logits are published, or (with caller
    // logits) once the first item's weights are issued.  A single layer's
    // count comes from an agent-scope load issued at launch, whose ~2 us
    // latency would otherwise hold up routing; it stays in VGPRs until then,
    // so that its wait is placed there (a chain's count comes from LDS).
    uint32_t fin_lo = static_cast<uint32_t>(finished), fin_hi = static_cast<uint32_t>(finished >> 32);
    int parity = 0;
    uint32_t tag = 0u;
    DecodeCounters* cnt = nullptr;
    uint64_t tag_bits = 0ull;
    auto resolve_call = [&]() __attribute__((always_inline)) {
        if constexpr (!kChained) asm volatile("" : "+v"(fin_lo), "+v"(fin_hi));
        const unsigned long long call = ((static_cast<unsigned long long>(fin_hi) << 32) | fin_lo) /
                                            static_cast<unsigned long long>(G) +
                                        static_cast<unsigned>(layer);
        parity = static_cast<int>(call & 1ull);
        tag = static_cast<uint32_t>(call % 0xffffffffull) + 1u;
        cnt = &sync->set[parity];
        tag_bits = static_cast<uint64_t>(tag) << kDecodeTagShift;
        if (block == 0 && tid == kThreads - 1) {
            // The next call's counter (this call never touches it).
            st_agent32(&sync->set[parity ^ 1].claim, 0u);
        }
    };
    int vote_row = 0;  // block_or row
    __syncthreads();
    TL(7, 0);

    // Token rows (normalised when the layer norms) into LDS, and the
    // shared-expert gate of each token.
    auto stage_row = [&](int t, uint4* v) {
        if (a.norm != nullptr) {
            float f[32];
#pragma unroll
            for (int i = 0; i < 4; ++i) unpack8(v[i], f + 8 * i);
            float acc = 0.0f;
#pragma unroll
            for (int j = 0; j < 32; ++j) acc = __builtin_fmaf(f[j], f[j], acc);
            const float mean = wave_butterfly_sum(acc) / static_cast<float>(kHidden);
            const float r = 1.0f / __builtin_sqrtf(mean + a.eps);
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                float wf[8];
                unpack8(w_norm[i], wf);
                uint32_t o[8];
#pragma unroll
                for (int j = 0; j < 8; ++j) o[j] = f2bf((f[8 * i + j] * r) * (1.0f + wf[j]));
                v[i] = make_uint4(o[0] | (o[1] << 16), o[2] | (o[3] << 16), o[4] | (o[5] << 16), o[6] | (o[7] << 16));
            }
        }
        uint4* dst = reinterpret_cast<uint4*>(x_lds + t * kXStride + 32 * lane);
#pragma unroll
        for (int i = 0; i < 4; ++i) dst[i] = v[i];
        if (a.shared_expert_gate != nullptr) {
            const float z = rbf(wave_butterfly_sum(lane_dot32(w_sg, x_lds + t * kXStride, lane)));
            if (lane == 0) P.sg[t] = rbf(1.0f / (1.0f + lr_exp(-z)));
        }
    };
    auto stage_rows = [&]() {
        if (has_lo) stage_row(t_lo, x_lo);
        if (has_hi) stage_row(t_hi, x_hi);
    };

    // ---- 2. router rows (workgroups 0..31, one row per wave) ----
    // The router needs the token rows first; with caller logits the rows are
    // staged later, while the first weights are already streaming.
    if (a.router != nullptr) {
        stage_rows();
        __syncthreads();
        TL(122, 0);
        resolve_call();
        if (early) {
            // The shared-expert A tile first_item, exactly as the item loop
            // runs an A item of slot 0 (columns = tokens 0..T-1, pairs from
            // kTopK * T).
            const int m = lane & 15;
            const int g = lane >> 4;
            const uint16_t* bp = x_lds + (m < T ? m : 0) * kXStride + kInner * (wave & 3) + 8 * g;
            f32x4 acc0 = {0.0f, 0.0f, 0.0f, 0.0f}, acc1 = {0.0f, 0.0f, 0.0f, 0.0f};
            staged_mfmas(b0, stage, bp, lane, acc0, acc1);  // (the early path runs the raw kernel only)
            part[wave * kWave + lane] = acc0 + acc1;
            __syncthreads();
            if ((wave & 3) == 0) {
                const f32x4* pp = part + wave * kWave + lane;
                const f32x4 sum = ((pp[0] + pp[kWave]) + pp[2 * kWave]) + pp[3 * kWave];
                f32x4 up;
#pragma unroll
                for (int i = 0; i < 4; ++i) up[i] = __shfl_xor(sum[i], 32, kWave);
                if (g < 2 && m < T) {
                    uint32_t act[4];
#pragma unroll
                    for (int i = 0; i < 4; ++i) act[i] = swiglu_bf16(rbf(sum[i]), rbf(up[i]));
                    uint64_t* dst = a.act + static_cast<size_t>(kTopK * T + m) * (kInner / 2) +
                                    (16 * first_item + 8 * (wave >> 2) + 4 * g) / 2;
                    st_agent64(dst, tag_bits | (act[0] | (act[1] << 16)));
                    st_agent64(dst + 1, tag_bits | (act[2] | (act[3] << 16)));
                }
            }
        }
        if (router_wg) {
            for (int t = 0; t < T; ++t) {
                const float s = wave_butterfly_sum(lane_dot32(w_router, x_lds + t * kXStride, lane));
                if (lane == 0) P.lg[t][wave] = static_cast<uint16_t>(f2bf(s));
            }
            __syncthreads();
            // This workgroup's 8 logits of token t as 4 tagged words (logits
            // 2k and 2k+1 in word k of the token's row), in every copy.
            if (tid < 4 * T) {
                const int t = tid >> 2;
                const int q = tid & 3;
                const uint32_t pair = static_cast<uint32_t>(P.lg[t][2 * q]) | (static_cast<uint32_t>(P.lg[t][2 * q + 1]) << 16);
                uint64_t* dst = a.logits + static_cast<size_t>(t) * (kExperts / 2) + (kWaves / 2) * block + q;
#pragma unroll
                for (int c = 0; c < kDecodeLogitCopies; ++c) st_agent64(dst + c * kDecodeLogitCopyWords, tag_bits | pair);
            }
            TL(123, 0);
        }
    }

    // ---- 4. the route plan ----
    if (a.router != nullptr) {
        // Each wave reloads its tokens' logit rows (bounded) until every word
        // carries this call's tag; lane l ends with logits 4l..4l+3.  The
        // rows come from copy b % 8, and a wave without a token loads none.
        const uint64_t* copy = a.logits + static_cast<size_t>(blockIdx.x % kDecodeLogitCopies) * kDecodeLogitCopyWords;
        const uint64_t* row_lo = copy + static_cast<size_t>(has_lo ? t_lo : 0) * (kExperts / 2) + 2 * lane;
        const uint64_t* row_hi = copy + static_cast<size_t>(has_hi ? t_hi : 0) * (kExperts / 2) + 2 * lane;
        uint64_t lw[4] = {0ull, 0ull, 0ull, 0ull};
        auto fetch = [&]() {
            if (has_lo) {
                lw[0] = ld_agent64(row_lo);
                lw[1] = ld_agent64(row_lo + 1);
            }
            if (has_hi) {
                lw[2] = ld_agent64(row_hi);
                lw[3] = ld_agent64(row_hi + 1);
            }
            return (has_lo && (tag_of(lw[0]) != tag || tag_of(lw[1]) != tag)) ||
                   (has_hi && (tag_of(lw[2]) != tag || tag_of(lw[3]) != tag));
        };
        if (block_or(fetch(), P, vote_row, wave, lane)) {
            const uint64_t start = now_ticks();
            while (true) {
                if (block_or(now_ticks() - start > kSpinTicks, P, vote_row, wave, lane)) {
                    if (tid == 0) P.status |= kStatusTimeout;
                    break;
                }
                __builtin_amdgcn_s_sleep(2);
                if (!block_or(fetch(), P, vote_row, wave, lane)) break;
            }
        }
        TL(124, 0);
        lg_lo = (lw[0] & 0xffffffffull) | (lw[1] << 32);
        lg_hi = (lw[2] & 0xffffffffull) | (lw[3] << 32);
    }
    if (a.indices_in == nullptr) {
        int e_lo, e_hi;
        uint32_t w_lo, w_hi;
        if (T > kWaves) {
            // Two tokens per wave: both selections in one block, so that
            // each fills the other's wave-maximum chains (an absent second
            // token selects over a dummy row and is dropped).
            const uint64_t both[2] = {lg_lo, lg_hi};
            int e2[2];
            uint32_t w2[2];
            topk8_waves<2>(both, e2, w2, lane);
            e_lo = e2[0];
            e_hi = e2[1];
            w_lo = w2[0];
            w_hi = w2[1];
            if (lane < kTopK) {
                P.ids[t_lo][lane] = e_lo;
                P.wts[t_lo][lane] = static_cast<uint16_t>(w_lo);
                if (has_hi) {
                    P.ids[t_hi][lane] = e_hi;
                    P.wts[t_hi][lane] = static_cast<uint16_t>(w_hi);
                }
            }
        } else if (has_lo) {
            topk8_wave(lg_lo, e_lo, w_lo, lane);
            TL(118, 0);
            if (lane < kTopK) {
                P.ids[t_lo][lane] = e_lo;
                P.wts[t_lo][lane] = static_cast<uint16_t>(w_lo);
            }
        }
    } else if (tid < T * kTopK) {
        const int t = tid / kTopK;
        const int r = tid % kTopK;
        const int64_t e = a.indices_in[tid];
        int32_t bad = (e < 0 || e >= kExperts) ? kStatusBadExpert : 0;
        for (int q = 0; q < r; ++q) bad |= (a.indices_in[t * kTopK + q] == e) ? kStatusRepeatedExpert : 0;
        P.ids[t][r] = bad ? 0 : static_cast<int32_t>(e);
        P.wts[t][r] = a.weights_in[tid];
        if (bad) atomicOr(&P.status, bad);
    }
    if (tid < kExperts) P.eptr[tid] = eptr;
    if constexpr (kCodec) {
        if (a.codec != nullptr && tid <= kExperts) {
#pragma unroll
            for (int i = 0; i < 5; ++i) P.ecodec[tid][i] = ec[i];
        }
    }
    __syncthreads();

    TL(1, 0);
    // ---- the first item's weights, first half (raw kernel) ----
    // A workgroup's first item is an A tile of slot s < 9: the shared
    // expert (slot 0) or token 0's route of rank s - 1 (slots are numbered
    // in discovery order), known once top-8 is done.  Half of its loads
    // are issued here, before the rest of the plan (64 KiB per CU, which the
    // load path accepts without stalling the waves); the other half after
    // it.  With bad routes no item runs and these loads are only reads of
    // expert 0's rows.
    int cur = early ? first_item + G : first_item;
    const uint16_t* first_rows[4] = {a.x, a.x, a.x, a.x};
    if constexpr (!kCodec) {
        const int slot = (a.sh_down != nullptr ? 0 : 1) + cur / kATiles;
        SlotInfo s0;
        s0.gate = a.sh_gate;
        s0.up = a.sh_up;
        if (slot > 0) {
            const uint4 pe = P.eptr[P.ids[0][slot - 1]];
            const uint16_t* gate_up = reinterpret_cast<const uint16_t*>(static_cast<uintptr_t>(pe.x) |
                                                                        (static_cast<uintptr_t>(pe.y) << 32));
            s0.gate = gate_up;
            s0.up = gate_up + static_cast<size_t>(kInner) * kHidden;
        }
        item_rows(s0, Item{0, slot, cur % kATiles}, wave, lane, first_rows);
        asm volatile("" ::"v"(warm0), "v"(warm1));  // the warming loads are complete
#pragma unroll
        for (int i = 0; i < kLoads / 2; ++i) b0[i] = ldg16_nt(first_rows[i & 3] + 128 * (i >> 2));
        TL(125, 0);
    }
    // Prefetch target of an item without weights (C items): 1 KiB of token
    // row 0, in cache after the first read.
    const uint16_t* const idle_rows = a.x + 8 * (lane >> 4);
    // Which of the lane's two tiles of an item it reads packed: bit t of
    // `dec`.  A workgroup's first item is read raw; its second takes the
    // choice from the codec table's per-(item, wave) flags (both tiles packed
    // when every tile of the wave's share fits; wave-uniform), later items
    // from their tile bases, loaded one step before the item's own loads
    // (tile_choice).
    auto unit_choice = [&](const Item& it) __attribute__((always_inline)) -> uint32_t {
        if (it.kind > 1) return 0u;
        const SlotCodec& s = P.scodec[it.slot];
        if (s.pk_gu == nullptr) return 0u;
        const uint8_t* flags = reinterpret_cast<const uint8_t*>(&P.ecodec[s.crow][2]);
        return ((flags[(it.kind == 1 ? 32 : 0) + it.tile] >> wave) & 1u) == 0u ? 3u : 0u;
    };
    // The bases of an item's two tiles of this lane (tile 0 in bits 0..7,
    // tile 1 in bits 8..15), loaded (2 bytes) for the A/B items of codec
    // slots; other items load kBothMisfit (both tiles raw).  The load is
    // issued for every item, so that its register is never merged at a join
    // before the wait.
    auto load_bases = [&](const Item& it) __attribute__((always_inline)) -> uint32_t {
        const void* at = &kBothMisfit;
        if (it.kind == 0 || it.kind == 1) {
            const SlotCodec& s = P.scodec[it.slot];
            if (s.pk_gu != nullptr) at = packed_lane(s, it, wave, lane).bases2;
        }
        return ldg_u16(at);
    };
    auto tile_choice = [](uint32_t bases) -> uint32_t {
        return ((bases & 0xffu) != kCodecMisfit ? 1u : 0u) | ((bases >> 8) != kCodecMisfit ? 2u : 0u);
    };
    // One load sequence for every kind of item (only the addresses differ),
    // so that no loaded register is copied at a join, which would wait for
    // the loads.  Without codec tables: load i at the item's base + 64i (C
    // items: cached token rows).  With them, tile t, register 8t + j:
    // packed, block j of the tile (j < 6) or its bases block (j = 6, 7); raw,
    // k-step kRawStep[j] of the tile.
    auto issue_item = [&](const Item& it, uint4* buf, uint32_t dec) __attribute__((always_inline)) {
        if constexpr (!kCodec) {
            // (row pointers selected, not loads branched: a join after the
            // loads would make the compiler wait for them)
            const uint16_t* rows[4];
            item_rows(P.slot[it.slot], it, wave, lane, rows);
            const bool weights = it.kind == 0 || it.kind == 1;
#pragma unroll
            for (int r = 0; r < 4; ++r) rows[r] = weights ? rows[r] : idle_rows + 8 * (lane & 15) - 8 * (lane >> 4);
            issue_rows(rows, buf);
            return;
        }
        const uint8_t* raw = reinterpret_cast<const uint8_t*>(idle_rows);
        const uint8_t* pk = raw;
        const uint8_t* bases = raw;
        if (it.kind == 0 || it.kind == 1) {
            raw = reinterpret_cast<const uint8_t*>(item_base(P.slot[it.slot], it, wave, lane));
            const SlotCodec& s = P.scodec[it.slot];
            if (s.pk_gu != nullptr) {
                const PackedLane p = packed_lane(s, it, wave, lane);
                pk = p.tile0 + 16 * (lane >> 4);
                bases = p.bases16;
            }
        }
#pragma unroll
        for (int t = 0; t < 2; ++t) {
            const bool packed = ((dec >> t) & 1u) != 0u;
            const uint8_t* pt = pk + t * kCodecTileBytes;
            const uint8_t* rt = raw + 512 * t;
#pragma unroll
            for (int j = 0; j < 8; ++j) {
                buf[8 * t + j] = ldg16(packed ? (j < 6 ? pt + 64 * j : bases) : rt + 64 * kRawStep[j]);
            }
        }
    };
    // The tile-codec addresses of an expert (kExperts: the shared one), or
    // null when the call has no codec table or the expert's row does not
    // give all four addresses (then it is read raw).
    auto codec_of = [&](int row) -> const uint4* {
        if (!kCodec || a.codec == nullptr) return nullptr;
        const uint4* c = P.ecodec[row];
        const bool all = (c[0].x | c[0].y) != 0u && (c[0].z | c[0].w) != 0u && (c[1].x | c[1].y) != 0u &&
                         (c[1].z | c[1].w) != 0u;
        return all ? c : nullptr;
    };
    if (block == 0 && tid < T * kTopK) {
        if (a.indices_out != nullptr) a.indices_out[tid] = P.ids[tid / kTopK][tid % kTopK];
        if (a.weights_out != nullptr) a.weights_out[tid] = P.wts[tid / kTopK][tid % kTopK];
    }
    const bool routes_ok = (P.status & ~kStatusTimeout) == 0;
    if (routes_ok && tid < T * kTopK) atomicOr(&P.tokmask[P.ids[tid / kTopK][tid % kTopK]], 1u << (tid / kTopK));
    __syncthreads();
    TL(119, 0);
    {
        // Route i = tid (token i / 8, rank i % 8) opens a slot when its token
        // is the first routed to the expert.  A new expert's slot is the
        // number of routes before it that open one, its first pair the sum
        // of their token counts: ballots over the (at most 128) routes, the
        // counts bit-sliced, so that no block scan is needed.  Waves 0 and 1
        // (the routes' threads) both evaluate all routes.
        auto route_opens = [&](int i, int& e_out, uint32_t& mask_out) -> uint32_t {
            e_out = 0;
            mask_out = 0u;
            if (!routes_ok || i >= T * kTopK) return 0u;
            const int t = i / kTopK;
            e_out = P.ids[t][i % kTopK];
            mask_out = P.tokmask[e_out];
            return (mask_out & ((1u << t) - 1u)) == 0u ? static_cast<uint32_t>(__popc(mask_out)) : 0u;
        };
        const bool route_thread = tid < 2 * kWave;
        const int own = route_thread ? tid : 0;
        int e = 0, e_other = 0;
        uint32_t mask = 0u, mask_other = 0u;
        const uint32_t count = route_opens(own, e, mask);                              // 0 or 1..16
        const uint32_t count_other = route_opens(own ^ kWave, e_other, mask_other);   // the other wave's route
        const uint32_t opens = route_thread && count != 0u ? (1u << 16) | count : 0u;
        // lanes of this route's wave below it, and the routes of wave 0 when
        // this is wave 1
        const uint64_t below = (1ull << lane) - 1ull;
        const bool second = own >= kWave;
        uint32_t rank = 0u, pair0 = 0u, unique = 0u;
        {
            const uint64_t o_own = __ballot(count != 0u);
            const uint64_t o_oth = __ballot(count_other != 0u);
            const uint64_t o_first = second ? o_oth : o_own;
            rank = static_cast<uint32_t>(__popcll(o_own & below)) + (second ? static_cast<uint32_t>(__popcll(o_first)) : 0u);
            unique = static_cast<uint32_t>(__popcll(o_own) + __popcll(o_oth));
#pragma unroll
            for (int b = 0; b < 5; ++b) {
                const uint64_t c_own = __ballot(((count >> b) & 1u) != 0u);
                const uint64_t c_oth = __ballot(((count_other >> b) & 1u) != 0u);
                const uint64_t c_first = second ? c_oth : c_own;
                pair0 += (static_cast<uint32_t>(__popcll(c_own & below)) +
                          (second ? static_cast<uint32_t>(__popcll(c_first)) : 0u)) << b;
            }
        }
        // (thread 0, which numbers the shared expert's slot below, is in wave
        // 0, whose ballots cover every route)
        (void)e_other;
        (void)mask_other;
        if (opens) {
            P.poff[e] = pair0;
            SlotInfo& s = P.slot[1 + rank];
            SlotCodec* sc = kCodec ? &P.scodec[1 + rank] : nullptr;
            const uint4 ptrs = P.eptr[e];
            const uint16_t* gate_up = reinterpret_cast<const uint16_t*>(static_cast<uintptr_t>(ptrs.x) |
                                                                        (static_cast<uintptr_t>(ptrs.y) << 32));
            set_slot_weights(s, sc, gate_up, gate_up + static_cast<size_t>(kInner) * kHidden,
                             reinterpret_cast<const uint16_t*>(static_cast<uintptr_t>(ptrs.z) |
                                                               (static_cast<uintptr_t>(ptrs.w) << 32)),
                             codec_of(e), e);
            uint32_t tok[4] = {0u, 0u, 0u, 0u};
            uint32_t m = mask;
#pragma unroll
            for (int j = 0; j < kMaxT; ++j) {
                const int t = m ? __ffs(m) - 1 : 0;
                const uint32_t v = m ? static_cast<uint32_t>(t) << (8 * (j & 3)) : 0u;
                tok[0] |= (j >> 2) == 0 ? v : 0u;
                tok[1] |= (j >> 2) == 1 ? v : 0u;
                tok[2] |= (j >> 2) == 2 ? v : 0u;
                tok[3] |= (j >> 2) == 3 ? v : 0u;
                m &= m - 1u;
            }
#pragma unroll
            for (int i = 0; i < 4; ++i) s.tok[i] = tok[i];
            s.count = static_cast<int32_t>(opens & 0xffffu);
            s.pair0 = static_cast<int32_t>(pair0);
        }
        if (tid == 0) {
            const bool shared = a.sh_down != nullptr && routes_ok;
            SlotInfo& s = P.slot[0];
            set_slot_weights(s, kCodec ? &P.scodec[0] : nullptr, a.sh_gate, a.sh_up, a.sh_down, codec_of(kExperts),
                             kExperts);
            uint32_t tok[4] = {0u, 0u, 0u, 0u};
#pragma unroll
            for (int j = 0; j < kMaxT; ++j) {
                const uint32_t v = j < T ? static_cast<uint32_t>(j) << (8 * (j & 3)) : 0u;
                tok[0] |= (j >> 2) == 0 ? v : 0u;
                tok[1] |= (j >> 2) == 1 ? v : 0u;
                tok[2] |= (j >> 2) == 2 ? v : 0u;
                tok[3] |= (j >> 2) == 3 ? v : 0u;
            }
#pragma unroll
            for (int i = 0; i < 4; ++i) s.tok[i] = tok[i];
            s.count = T;
            s.pair0 = kTopK * T;
            P.first_slot = shared ? 0 : 1;
            P.n_slots = routes_ok ? static_cast<int32_t>(unique) + (shared ? 1 : 0) : 0;
        }
    }
    __syncthreads();
    TL(120, 0);
    // The route status of a launch's first layer replaces the previous
    // launch's; later layers add theirs (timeouts are OR-ed in at the end).
    if (block == 0 && tid == 0) {
        const int32_t route_status = P.status & ~kStatusTimeout;
        if (layer == 0) {
            st_agent32(a.status, static_cast<uint32_t>(route_status));
        } else if (route_status != 0) {
            atomicOr(a.status, route_status);
        }
    }
    TL(3, 0);
    const int n_slots = P.n_slots;
    const int first_slot = P.first_slot;
    const int total = (kATiles + kBTiles) * n_slots;          // A and B items
    const int end = n_slots > 0 ? total + kCombineItems : 0;  // and the C items

    if (a.router == nullptr) resolve_call();

    // ---- the first item's weights (the codec kernel), or their second half ----
    // Issued as soon as the slots are numbered; the first step then issues
    // the second item's at once, so that two items are in flight from the
    // start.  The token rows (with caller logits) and the combine order are
    // worked out while they stream.
    uint32_t dec = 0u;  // tile choice of the item being run (the first is read raw)
    if constexpr (!kCodec) {
        // the same rows as the plan's slot gives
#pragma unroll
        for (int i = kLoads / 2; i < kLoads; ++i) b0[i] = ldg16_nt(first_rows[i & 3] + 128 * (i >> 2));
    } else {
        issue_item(item_at(cur, total, n_slots, first_slot), b0, 0u);
    }
    TL(2, 0);
    TL(5, 7 * kWave);
    if (a.router == nullptr) {
        stage_rows();
        TL(6, 0);
        TL(121, 7 * kWave);
    }
    if (routes_ok && tid < T * kTopK) {
        const int t = tid / kTopK;
        const int k = tid % kTopK;
        const int e = P.ids[t][k];
        const int p = static_cast<int>(P.poff[e]) + __popc(P.tokmask[e] & ((1u << t) - 1u));
        int order = 0;
#pragma unroll
        for (int q = 0; q < kTopK; ++q) order += P.ids[t][q] < e ? 1 : 0;
        P.comb_pair[t][order] = static_cast<int16_t>(p);
        P.comb_w[t][order] = bf2f(P.wts[t][k]);
    }
    __syncthreads();

    // Bad routes: the output is the residual (or zeros); no expert runs.
    if (!routes_ok) {
        if (block == 0) {
            for (int i = tid; i < T * kHidden / 4; i += kThreads) {
                uint64_t v = 0;
                if (a.residual) v = ld_row8<kChained>(a.x + 4 * static_cast<size_t>(i));
                st_row8<kChained>(a.out + 4 * static_cast<size_t>(i), v);
            }
        }
    }

    // ---- 4. work items ----
    // B staging: thread tid loads words 8*(tid%32)..+7 of act row tid/32.
    uint64_t stg[8];
    const int stg_row = tid >> 5;
    const uint32_t stg_off = static_cast<uint32_t>(stg_row * (kInner / 2) * 8 + (tid & 31) * 64);
    // Lanes of the claiming atomic: lane 0 of wave 0.
    const uint32_t claim_lanes = wave == 0 ? 1u : 0u;
    int par = 0;              // A partial-sum buffer
    int cpar = 0;             // claim buffer
    [[maybe_unused]] int tl_step = 0;  // timeline build: steps taken

    auto stale_word = [&](uint64_t w) { return tag_of(w) != tag; };

    // The MFMAs of an item of a codec slot (B operand rows at bp, bb = the
    // byte of the lane's first tile base in its bases block): per tile the
    // decoded packed values or the raw row's.  (A second copy without the
    // pick for waves that read every tile packed needs more registers than
    // the kernel has.)
    auto codec_mfmas = [&](const uint4* buf, const uint16_t* bp, uint32_t dec, int bb, f32x4& acc0,
                           f32x4& acc1) __attribute__((always_inline)) {
        const uint32_t base0 = byte_of(buf[6], bb) * 0x01010101u;
        const uint32_t base1 = byte_of(buf[14], bb + 1) * 0x01010101u;
#pragma unroll
        for (int q = 0; q < kLoads; q += 2) {
            const uint32_t base = q < kLoads / 2 ? base0 : base1;
            const uint32_t pk = 0u - ((dec >> (q >> 3)) & 1u);
            acc0 = mfma16x16x32(pick(pk, packed_operand(buf, q, base), buf[raw_reg(q)]),
                                *reinterpret_cast<const uint4*>(bp + 32 * q), acc0);
            acc1 = mfma16x16x32(pick(pk, packed_operand(buf, q + 1, base), buf[raw_reg(q + 1)]),
                                *reinterpret_cast<const uint4*>(bp + 32 * (q + 1)), acc1);
        }
    };
    // The MFMAs of an A or B item whose weights are in buf (B operand rows
    // at bp): raw items of the raw kernel through the wave's stage; codec
    // kernel items per tile packed or raw (raw loads in kRawStep order).
    auto item_mfmas = [&](const Item& it, const uint4* buf, const uint16_t* bp, uint32_t dec, f32x4& acc0,
                          f32x4& acc1) __attribute__((always_inline)) {
        if constexpr (!kCodec) {
            staged_mfmas(buf, stage, bp, lane, acc0, acc1);
        } else if (P.scodec[it.slot].pk_gu != nullptr) {
            codec_mfmas(buf, bp, dec, packed_lane(P.scodec[it.slot], it, wave, lane).base_byte, acc0, acc1);
        } else {
#pragma unroll
            for (int q = 0; q < kLoads; q += 2) {
                acc0 = mfma16x16x32(buf[raw_reg(q)], *reinterpret_cast<const uint4*>(bp + 32 * q), acc0);
                acc1 = mfma16x16x32(buf[raw_reg(q + 1)], *reinterpret_cast<const uint4*>(bp + 32 * (q + 1)), acc1);
            }
        }
    };
    // Runs item kk, whose weights are in buf (tile choice `dec`), prefetches
    // item kn into nbuf (tile choice from `bases`, its tile bases, which
    // become those of kn2) and loads the tile bases of kn2.  Returns the item
    // claimed for the step after kn2; ndec receives kn's tile choice.
    auto step = [&](int kk, int kn, int kn2, uint4* buf, uint4* nbuf, uint32_t dec, uint32_t& ndec,
                    uint32_t& bases) __attribute__((always_inline)) -> int {
        [[maybe_unused]] const int tl_at = 8 + 5 * tl_step;
        TL(tl_at, 0);
        const Item it = item_at(kk, total, n_slots, first_slot);
        const Item nx = item_at(kn, total, n_slots, first_slot);
        const Item nx2 = item_at(kn2, total, n_slots, first_slot);
        const SlotInfo& s = P.slot[it.slot];
        // Uniform base of the slot's 16 act rows (rows past its count are
        // padding, loaded but never used).
        const char* stg_base = reinterpret_cast<const char*>(a.act) +
                               static_cast<size_t>(__builtin_amdgcn_readfirstlane(s.pair0)) * (kInner / 2) * 8;
        // (a) staging loads (B), the claim of the item after next, then the
        //     next item's weights: a wait for everything but the newest 16
        //     loads covers this item's weights, staging and claim.
        // Only the slot's count rows are loaded: the other threads issue
        // fewer loads, which the wait below (an upper bound) allows.
        if (it.kind == 1 && stg_row < s.count) {
            ld_agent64x4_async(stg, stg_base, stg_off);
            ld_agent64x4_async(stg + 4, stg_base, stg_off + 32);
        }
        const uint32_t claimed = claim_async(&cnt->claim, claim_lanes);
        uint32_t next_bases = 0u;
        ndec = 0u;
        if constexpr (kCodec) {
            next_bases = load_bases(nx2);
            ndec = tile_choice(bases);
        }
        __builtin_amdgcn_sched_barrier(0);
        issue_item(nx, nbuf, ndec);
        __builtin_amdgcn_sched_barrier(0);
        // s_waitcnt vmcnt(16) (expcnt and lgkmcnt left at their maximum)
        // as a builtin, so that the compiler's own wait insertion knows
        // what it completed.
        __builtin_amdgcn_s_waitcnt(kWaitVm16);
        __builtin_amdgcn_sched_barrier(0);
        TL(tl_at + 1, 0);
        bases = next_bases;
        if (tid == 0) P.claim[cpar] = static_cast<int32_t>(claimed) + (kCodec ? 3 * G : 2 * G + (early_path ? kATiles : 0));
        const int m = lane & 15;
        const int g = lane >> 4;
        if (it.kind == 1) {
            // (b) the slot's act rows, once every word used carries this
            //     call's tag; a slot whose A items are still being written is
            //     reloaded (bounded).  The first barrier also means every wave
            //     is past the previous item's reads of act_lds.
            const bool used = stg_row < s.count;
            bool stale = false;
#pragma unroll
            for (int i = 0; i < 8; ++i) stale |= used && stale_word(stg[i]);
            if (block_or(stale, P, vote_row, wave, lane)) {
                const uint64_t start = now_ticks();
                while (true) {
                    if (block_or(now_ticks() - start > kSpinTicks, P, vote_row, wave, lane)) {
                        if (tid == 0) P.status |= kStatusTimeout;
                        break;
                    }
                    __builtin_amdgcn_s_sleep(2);
                    stale = false;
#pragma unroll
                    for (int i = 0; i < 8; ++i) {
                        stg[i] = ld_agent64(stg_base + stg_off + 8 * i);
                        stale |= used && stale_word(stg[i]);
                    }
                    if (!block_or(stale, P, vote_row, wave, lane)) break;
                }
            }
            uint4* dst = reinterpret_cast<uint4*>(act_lds + stg_row * kActStride + 16 * (tid & 31));
            dst[0] = make_uint4(static_cast<uint32_t>(stg[0]), static_cast<uint32_t>(stg[1]),
                                static_cast<uint32_t>(stg[2]), static_cast<uint32_t>(stg[3]));
            dst[1] = make_uint4(static_cast<uint32_t>(stg[4]), static_cast<uint32_t>(stg[5]),
                                static_cast<uint32_t>(stg[6]), static_cast<uint32_t>(stg[7]));
            __syncthreads();
        }
        TL(tl_at + 2, 0);
        // (c) the item itself.
        if (it.kind == 0) {
            const int tok = column_token(s, m < s.count ? m : 0);
            const uint16_t* bp = x_lds + tok * kXStride + kInner * (wave & 3) + 8 * g;
            f32x4 acc0 = {0.0f, 0.0f, 0.0f, 0.0f}, acc1 = {0.0f, 0.0f, 0.0f, 0.0f};
            item_mfmas(it, buf, bp, dec, acc0, acc1);
            part[(par * kWaves + wave) * kWave + lane] = acc0 + acc1;
            __syncthreads();
            if ((wave & 3) == 0) {
                const f32x4* pp = part + (par * kWaves + wave) * kWave + lane;
                const f32x4 sum = ((pp[0] + pp[kWave]) + pp[2 * kWave]) + pp[3 * kWave];
                f32x4 up;
#pragma unroll
                for (int i = 0; i < 4; ++i) up[i] = __shfl_xor(sum[i], 32, kWave);
                if (g < 2 && m < s.count) {
                    uint32_t act[4];
#pragma unroll
                    for (int i = 0; i < 4; ++i) act[i] = swiglu_bf16(rbf(sum[i]), rbf(up[i]));
                    uint64_t* dst = a.act + static_cast<size_t>(s.pair0 + m) * (kInner / 2) +
                                    (16 * it.tile + 8 * (wave >> 2) + 4 * g) / 2;
                    st_agent64(dst, tag_bits | (act[0] | (act[1] << 16)));
                    st_agent64(dst + 1, tag_bits | (act[2] | (act[3] << 16)));
                }
            }
            par ^= 1;
        } else if (it.kind == 1) {
            const uint16_t* bp = act_lds + (m < s.count ? m : 0) * kActStride + 8 * g;
            f32x4 acc0 = {0.0f, 0.0f, 0.0f, 0.0f}, acc1 = {0.0f, 0.0f, 0.0f, 0.0f};
            item_mfmas(it, buf, bp, dec, acc0, acc1);
            const f32x4 y = acc0 + acc1;
            if (m < s.count) {
                uint32_t o[4];
#pragma unroll
                for (int i = 0; i < 4; ++i) o[i] = f2bf(y[i]);
                uint64_t* dst = a.y + static_cast<size_t>(s.pair0 + m) * (kHidden / 2) +
                                (kBRows * it.tile + 16 * wave + 4 * g) / 2;
                st_agent64(dst, tag_bits | (o[0] | (o[1] << 16)));
                st_agent64(dst + 1, tag_bits | (o[2] | (o[3] << 16)));
            }
        } else if (it.kind == 2) {
            combine_tile<kChained>(a, P, tid, it.tile, T, first_slot == 0, tag, vote_row);
            // Wave 0's claim above is visible to every wave after this.
            __syncthreads();
        } else {
            // No item; the barrier publishes the claim.
            __syncthreads();
        }
        TL(tl_at + 3, 0);
        TL_WORD(tl_at + 4, static_cast<unsigned long long>((it.kind + 1) * 1000000 + it.slot * 1000 + it.tile));
        ++tl_step;
        const int after = P.claim[cpar];
        cpar ^= 1;
        return after;
    };

    // The first three items of a workgroup are fixed (the first one's
    // weights are already in flight); the rest are claimed.
    if (cur < end) {
        int nxt = early ? 2 * G + first_item : cur + G;
        int nxt2 = cur + 2 * G;  // (codec: no early items)
        // Everything but the first item's 16 loads is complete by now; the
        // wait tells the compiler so, which keeps it from draining the
        // first item's loads where the loop reuses the prologue's
        // registers.
        __builtin_amdgcn_s_waitcnt(kWaitVm16);
        // Two steps per iteration (the register sets swap roles) and one
        // exit, at the bottom.  A workgroup with an odd number of items ends
        // with a step of no item: a prefetch of cached rows and one more
        // claim, of a number past the end like all of its later claims.
        // (With an exit after each step, the compiler's control-flow
        // structuring adds a path from the first step straight back to the
        // top, on which that step's prefetch is still in flight; every
        // iteration then waits for all loads before issuing the next
        // prefetch.)
        if constexpr (kCodec) {
            // Items are claimed three ahead, so that each item's tile bases
            // are loaded a step before its weights.  The second item's tile
            // choice comes from the per-(item, wave) flags (as a bases value:
            // 0 packs both tiles, 0xffff reads both raw).
            uint32_t bases = unit_choice(item_at(nxt, total, n_slots, first_slot)) == 3u ? 0u : 0xffffu;
            do {
                uint32_t ndec;
                int after = step(cur, nxt, nxt2, b0, b1, dec, ndec, bases);
                cur = nxt;
                nxt = nxt2;
                nxt2 = after;
                dec = ndec;
                after = step(cur, nxt, nxt2, b1, b0, dec, ndec, bases);
                cur = nxt;
                nxt = nxt2;
                nxt2 = after;
                dec = ndec;
            } while (cur < end);
        } else {
            // Items are claimed two ahead (claims number items from 2G on).
            uint32_t bases = 0u;
            do {
                uint32_t ndec;
                int after = step(cur, nxt, 0, b0, b1, 0u, ndec, bases);
                cur = nxt;
                nxt = after;
                after = step(cur, nxt, 0, b1, b0, 0u, ndec, bases);
                cur = nxt;
                nxt = after;
            } while (cur < end);
        }
    }

    TL(4, 0);
    TL_FLUSH(layer);
    // ---- 5. this workgroup's share of the layer is done ----
    __builtin_amdgcn_s_waitcnt(0);  // also the first-item loads of a call without items
    __syncthreads();
    return P.status & kStatusTimeout;
}

template <bool kCodec>
__global__ __launch_bounds__(kThreads, 1) void moe_decode(DecodeArgs args) {
    // A local copy: the helpers take it by reference, which must not force
    // the kernel-argument block into private memory.
    const DecodeArgs a = args;
    extern __shared__ __attribute__((aligned(16))) uint8_t dyn[];
    __shared__ Plan<kCodec> P;
    // This call's number, from the count of finished workgroups (DecodeSync).
    const unsigned long long finished = ld_agent64(&a.sync->finished);
    const int32_t timeout = decode_layer<false, kCodec>(a, P, dyn, finished, 0, [] {});
    if (threadIdx.x == 0) {
        if (timeout) atomicOr(a.status, kStatusTimeout);
        __hip_atomic_fetch_add(&a.sync->finished, 1ull, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    }
}

// Launch-wide values of a chain, kept in LDS: only the layer index stays
// in registers across layers.
struct ChainState {
    unsigned long long finished;  // DecodeSync::finished at the start
    unsigned long long arrived;   // chain_arrive at the start, rounded down to a multiple of G
    int32_t timeout;
};

// Several decode layers in one launch, with a grid barrier between layers
// (every workgroup is resident).  Layer l is decode call c + l, with c the
// call number read at the start (DecodeSync).
template <bool kCodec>
__global__ __launch_bounds__(kThreads, 1) void moe_chain(ChainArgs args) {
    extern __shared__ __attribute__((aligned(16))) uint8_t dyn[];
    __shared__ Plan<kCodec> P;
    __shared__ ChainState S;
    const unsigned long long G = gridDim.x;
    if (threadIdx.x == 0) {
        S.finished = ld_agent64(&args.base.sync->finished);
        S.arrived = ld_agent64(&args.base.sync->chain_arrive) / G * G;
        S.timeout = 0;
    }
    __syncthreads();
    for (int layer = 0;; ++layer) {
        const int l = __builtin_amdgcn_readfirstlane(layer);
        // The arguments are read again for every layer (an opaque copy of
        // their address), so that they are not held in registers across
        // the layer.
        typedef const __attribute__((address_space(4))) ChainArgs KernelArgs;
        KernelArgs* cp = (KernelArgs*)(__builtin_amdgcn_kernarg_segment_ptr());
        asm volatile("" : "+s"(cp));
        KernelArgs& c = *cp;
        if (l >= c.layers) break;
        const int T = c.base.tokens;
        DecodeArgs a{};
        a.eps = c.base.eps;
        a.logits = c.base.logits;
        a.act = c.base.act;
        a.y = c.base.y;
        a.sync = c.base.sync;
        a.status = c.base.status;
        a.tokens = T;
        const auto& w = c.layer[l];
        a.router = w.router;
        a.expert_ptrs = w.expert_ptrs;
        a.sh_gate = w.sh_gate;
        a.sh_up = w.sh_up;
        a.sh_down = w.sh_down;
        a.shared_expert_gate = w.shared_expert_gate;
        a.norm = w.norm;
        a.codec = w.codec;
        // The chain always routes with the layer's router.
        a.logits_in = nullptr;
        a.indices_in = nullptr;
        a.weights_in = nullptr;
        a.residual = w.norm != nullptr;
        a.x = l == 0 ? c.hidden : c.inner + static_cast<size_t>((l - 1) & 1) * T * kHidden;
        a.out = l == c.layers - 1 ? c.out : c.inner + static_cast<size_t>(l & 1) * T * kHidden;
        a.indices_out = c.base.indices_out != nullptr ? c.base.indices_out + static_cast<size_t>(l) * T * kTopK : nullptr;
        a.weights_out = c.base.weights_out != nullptr ? c.base.weights_out + static_cast<size_t>(l) * T * kTopK : nullptr;
        const unsigned long long finished = uniform64(S.finished);
        DecodeSync* const sync = c.base.sync;
        // Arrivals completed by the barrier before layer l.
        const unsigned long long target = S.arrived + G * static_cast<unsigned long long>(l);
        auto wait_input = [&] {
            // Grid barrier before every layer but the first: the previous
            // layer's output rows are all written.
            if (l > 0) {
                if (threadIdx.x == 0) {
                    const uint64_t start = now_ticks();
                    while (ld_agent64(&sync->chain_release) < target) {
                        if (now_ticks() - start > kSpinTicks) {
                            S.timeout = kStatusTimeout;
                            break;
                        }
                        __builtin_amdgcn_s_sleep(1);
                    }
                }
                __syncthreads();
            }
        };
        const int32_t timeout = decode_layer<true, kCodec>(a, P, dyn, finished, l, wait_input);
        if (threadIdx.x == 0) {
            S.timeout |= timeout;
            if (l + 1 < c.layers) {
                // Arrival: this workgroup's output rows are written (agent
                // scope, waited for at the end of the layer).  The arrival
                // that completes the barrier releases the others.
                const unsigned long long next = target + G;
                const unsigned long long before =
                    __hip_atomic_fetch_add(&sync->chain_arrive, 1ull, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
                if (before + 1 == next) st_agent64(&sync->chain_release, next);
            }
        }
        __syncthreads();
    }
    if (threadIdx.x == 0) {
        if (S.timeout) atomicOr(args.base.status, kStatusTimeout);
        __hip_atomic_fetch_add(&args.base.sync->finished, static_cast<unsigned long long>(args.layers),
                               __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    }
}

}  // namespace

size_t decode_lds_bytes(int tokens, bool codec) {
    return static_cast<size_t>(tokens) * kXStride * 2 + static_cast<size_t>(kMaxT) * kActStride * 2 +
           2 * kWaves * kWave * sizeof(f32x4) + (codec ? 0 : static_cast<size_t>(kWaves) * kStageBytes);
}

namespace {

// Below this many tokens a workgroup runs one or two items per layer, which
// the codec's tile choice (one step ahead) does not reach; its pipeline then
// only costs (T=1 chain: 35 instead of 30 us per layer).
constexpr int kCodecMinTokens = 8;

// Per device and kernel: the CU count, and whether the LDS limit was raised
// and the occupancy checked.
struct LaunchSetup {
    int cus = 0;
    bool ready = false;
};

// Grid size of a persistent decode launch on the current device (one
// workgroup per CU, all resident at once, which the cross-workgroup waits
// rely on).
template <typename Kernel>
hipError_t persistent_grid(Kernel kernel, bool codec, LaunchSetup (&setup)[64], int* grid) {
    int device = 0;
    hipError_t err = hipGetDevice(&device);
    if (err != hipSuccess) return err;
    if (device < 0 || device >= 64) return hipErrorInvalidDevice;
    LaunchSetup& d = setup[device];
    if (d.cus == 0) {
        err = hipDeviceGetAttribute(&d.cus, hipDeviceAttributeMultiprocessorCount, device);
        if (err != hipSuccess) return err;
    }
    if (!d.ready) {
        err = hipFuncSetAttribute(reinterpret_cast<const void*>(kernel), hipFuncAttributeMaxDynamicSharedMemorySize,
                                  static_cast<int>(decode_lds_bytes(kMaxT, codec)));
        if (err != hipSuccess) return err;
        int blocks = 0;
        err = hipOccupancyMaxActiveBlocksPerMultiprocessor(&blocks, kernel, kThreads, decode_lds_bytes(kMaxT, codec));
        if (err != hipSuccess) return err;
        if (blocks < 1) return hipErrorLaunchOutOfResources;
        d.ready = true;
    }
    // The first items name at most 8 slots (G <= 256).
    if (d.cus > kExperts) return hipErrorNotSupported;
    *grid = d.cus;
    return hipSuccess;
}

}  // namespace

hipError_t launch_moe_decode(const DecodeArgs& a, hipStream_t stream) {
    if (a.tokens <= 0) return hipSuccess;
    if (a.tokens > kMaxT) return hipErrorInvalidValue;
    // The codec kernel carries the tile-choice pipeline; calls without codec
    // tables, and calls of fewer than kCodecMinTokens tokens, run the kernel
    // without it (the codec is lossless and the raw rows are always given,
    // so either gives the same results).
    static LaunchSetup setup[2][64];
    const bool codec = a.codec != nullptr && a.tokens >= kCodecMinTokens;
    int grid = 0;
    const hipError_t err = codec ? persistent_grid(moe_decode<true>, true, setup[1], &grid)
                                 : persistent_grid(moe_decode<false>, false, setup[0], &grid);
    if (err != hipSuccess) return err;
    const StageEvents ev = timing_events(kStageLayer);
    if (codec) {
        LRMOE_LAUNCH(moe_decode<true>, dim3(grid), dim3(kThreads), decode_lds_bytes(a.tokens, codec), stream, ev.start,
                     ev.stop, a);
    } else {
        LRMOE_LAUNCH(moe_decode<false>, dim3(grid), dim3(kThreads), decode_lds_bytes(a.tokens, codec), stream, ev.start,
                     ev.stop, a);
    }
    return hipGetLastError();
}

hipError_t launch_moe_chain(const ChainArgs& a, hipStream_t stream) {
    if (a.base.tokens <= 0 || a.layers <= 0) return hipSuccess;
    if (a.base.tokens > kMaxT) return hipErrorInvalidValue;
    static LaunchSetup setup[2][64];
    bool codec = false;
    for (int l = 0; l < a.layers; ++l) codec |= a.layer[l].codec != nullptr;
    codec = codec && a.base.tokens >= kCodecMinTokens;  // as in launch_moe_decode
    int grid = 0;
    const hipError_t err = codec ? persistent_grid(moe_chain<true>, true, setup[1], &grid)
                                 : persistent_grid(moe_chain<false>, false, setup[0], &grid);
    if (err != hipSuccess) return err;
    const StageEvents ev = timing_events(kStageLayer);
    if (codec) {
        LRMOE_LAUNCH(moe_chain<true>, dim3(grid), dim3(kThreads), decode_lds_bytes(a.base.tokens, codec), stream, ev.start,
                     ev.stop, a);
    } else {
        LRMOE_LAUNCH(moe_chain<false>, dim3(grid), dim3(kThreads), decode_lds_bytes(a.base.tokens, codec), stream, ev.start,
                     ev.stop, a);
    }
    return hipGetLastError();
}

}  // namespace lrmoe
