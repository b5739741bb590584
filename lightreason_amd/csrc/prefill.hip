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
// Experts (cpu_experts.c:54-69 rounding points; the shared expert is slot 0):
//   pf_gateup one workgroup per (unit, 128-row tile): 128 gate + 128 up rows
//             of one expert against up to 128 tokens.  Each of the 8 waves
//             streams its 32 weight rows (16 gate, 16 up) from HBM straight
//             into MFMA A operands, two K-chunks ahead; the same waves stage
//             the unit's token rows in LDS chunk by chunk (three chunks ahead
//             in registers), shared by all 8 waves, so a weight byte is read
//             once per 128 tokens and feeds up to 8 16x16x32 MFMAs.  SwiGLU
//             in the epilogue, act rows out.
//   pf_down   one workgroup per (unit, 128-row tile): the tile's down rows over
//             k = 512 stay in registers while the unit's act rows pass through
//             LDS 64 at a time; y rows out (bf16).
//   The ordered combine is experts.hip's combine_kernel.
//
// The 8 (or 16) tiles of a unit run on one XCD (workgroup b runs on XCD
// b % 8), so the unit's token or act rows are fetched into that XCD's L2 once.
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
constexpr int kDnTok = 64;                 // act rows per LDS pass
constexpr int kDnPieces = kDnTok * (kInner / 8) / kDnThreads;  // 16-byte act pieces per thread per pass
constexpr int kActStride = kInner + 8;     // LDS act row stride (bf16)

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
        return;
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

__device__ __forceinline__ bool load_unit(const ExpertArgs& a, int u, Unit& w) {
    if (u >= a.ws.control->n_units) return false;
    const int4 unit = a.ws.units[u];
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
    const uint16_t* gate_up = reinterpret_cast<const uint16_t*>(a.expert_ptrs[2 * e]);
    w.gate = gate_up;
    w.up = gate_up + static_cast<size_t>(kInner) * kHidden;
    w.down = reinterpret_cast<const uint16_t*>(a.expert_ptrs[2 * e + 1]);
    w.tokens = a.plan.pair_token + unit.y;
    return true;
}

// XCD-aware placement: the `tiles` workgroups of one unit run on XCD unit % 8.
__device__ __forceinline__ void unit_tile(int b, int tiles, int& unit, int& tile) {
    const int group = b / (8 * tiles);
    const int within = b % (8 * tiles);
    unit = 8 * group + within % 8;
    tile = within / 8;
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
                *reinterpret_cast<uint2*>((r ? act1 : act0) + static_cast<size_t>(16 * b) * kInner) =
                    make_uint2(v[0] | (v[1] << 16), v[2] | (v[3] << 16));
            }
        }
    }
}

__global__ __launch_bounds__(kGuThreads, 1) void pf_gateup(ExpertArgs a) {
    extern __shared__ __attribute__((aligned(16))) uint16_t xs[];  // [2][kPassTok][kXsStride]
    int ui, tile;
    unit_tile(blockIdx.x, kGuTiles, ui, tile);
    Unit w;
    if (!load_unit(a, ui, w)) return;
    const int tid = threadIdx.x;
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
        gateup_mfma<2>(arow0, arow1, xrow, xrow_row, piece, xs, act0, act1, w.count);
    } else if (nblk <= 4) {
        gateup_mfma<4>(arow0, arow1, xrow, xrow_row, piece, xs, act0, act1, w.count);
    } else {
        gateup_mfma<8>(arow0, arow1, xrow, xrow_row, piece, xs, act0, act1, w.count);
    }
}

__global__ __launch_bounds__(kDnThreads, 1) void pf_down(ExpertArgs a) {
    extern __shared__ __attribute__((aligned(16))) uint16_t as[];  // [kDnTok][kActStride]
    int ui, tile;
    unit_tile(blockIdx.x, kDnTiles, ui, tile);
    Unit w;
    if (!load_unit(a, ui, w)) return;
    const int tid = threadIdx.x;
    const int wave = tid >> 6;
    const int lane = tid & 63;
    const int m = lane & 15;
    const int g = lane >> 4;
    const int h0 = kDnRows * tile + 16 * wave;
    // The tile's 16 rows x 512 of this wave, kept in registers for every pass.
    const uint16_t* arow = w.down + static_cast<size_t>(h0 + m) * kInner + 8 * g;
    uint4 ab[kInner / 32];
#pragma unroll
    for (int s = 0; s < kInner / 32; ++s) ab[s] = ldg16(arow + 32 * s);
    for (int q0 = 0; q0 < w.count; q0 += kDnTok) {
        const int nt = min(kDnTok, w.count - q0);
        // Stage act rows q0..q0+kDnTok-1 (1 KiB each, 64 pieces of 16 bytes).
        uint4 st[kDnPieces];
#pragma unroll
        for (int j = 0; j < kDnPieces; ++j) {
            const int idx = tid + kDnThreads * j;
            const int r = idx / 64;
            const int rr = r < nt ? r : 0;
            st[j] = ldg16(a.ws.act + static_cast<size_t>(w.pair0 + q0 + rr) * kInner + 8 * (idx % 64));
        }
        if (q0 > 0) __syncthreads();  // previous pass done with the LDS rows
#pragma unroll
        for (int j = 0; j < kDnPieces; ++j) {
            const int idx = tid + kDnThreads * j;
            *reinterpret_cast<uint4*>(as + (idx / 64) * kActStride + 8 * (idx % 64)) = st[j];
        }
        __syncthreads();
        const int nb = (nt + 15) / 16;
        for (int b = 0; b < nb; ++b) {
            const uint16_t* bp = as + (16 * b + m) * kActStride + 8 * g;
            f32x4 acc0 = {0.0f, 0.0f, 0.0f, 0.0f}, acc1 = {0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
            for (int s = 0; s < kInner / 32; s += 2) {
                acc0 = mfma16x16x32(ab[s], *reinterpret_cast<const uint4*>(bp + 32 * s), acc0);
                acc1 = mfma16x16x32(ab[s + 1], *reinterpret_cast<const uint4*>(bp + 32 * (s + 1)), acc1);
            }
            const f32x4 y = acc0 + acc1;
            const int col = 16 * b + m;
            if (col < nt) {
                uint16_t* dst = a.ws.y + static_cast<size_t>(w.pair0 + q0 + col) * kHidden + h0 + 4 * g;
                *reinterpret_cast<uint2*>(dst) = make_uint2(f2bf(y[0]) | (f2bf(y[1]) << 16), f2bf(y[2]) | (f2bf(y[3]) << 16));
            }
        }
    }
}

int max_units(int tokens) {
    return (tokens + kPassTok - 1) / kPassTok + kExperts + (kTopK * tokens + kPassTok - 1) / kPassTok;
}

}  // namespace

size_t prefill_gateup_lds() { return static_cast<size_t>(2) * kPassTok * kXsStride * sizeof(uint16_t); }
size_t prefill_down_lds() { return static_cast<size_t>(kDnTok) * kActStride * sizeof(uint16_t); }

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
    hipError_t dev_err = hipGetDevice(&device);
    if (dev_err != hipSuccess) return dev_err;
    if (device < 0 || device >= 64) return hipErrorInvalidDevice;
    static bool attrs[64] = {false};  // per device: dynamic LDS limits raised
    if (!attrs[device]) {
        hipError_t err = hipFuncSetAttribute(reinterpret_cast<const void*>(pf_gateup),
                                             hipFuncAttributeMaxDynamicSharedMemorySize,
                                             static_cast<int>(prefill_gateup_lds()));
        if (err != hipSuccess) return err;
        err = hipFuncSetAttribute(reinterpret_cast<const void*>(pf_down), hipFuncAttributeMaxDynamicSharedMemorySize,
                                  static_cast<int>(prefill_down_lds()));
        if (err != hipSuccess) return err;
        attrs[device] = true;
    }
    const int units = (max_units(a.tokens) + 7) / 8 * 8;
    const StageEvents gate_ev = timing_events(kStageGateUp);
    LRMOE_LAUNCH(pf_gateup, dim3(units * kGuTiles), dim3(kGuThreads), prefill_gateup_lds(), stream, gate_ev.start,
                 gate_ev.stop, a);
    const StageEvents down_ev = timing_events(kStageDown);
    LRMOE_LAUNCH(pf_down, dim3(units * kDnTiles), dim3(kDnThreads), prefill_down_lds(), stream, down_ev.start,
                 down_ev.stop, a);
    return hipGetLastError();
}

}  // namespace lrmoe
