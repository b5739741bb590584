// Full-attention decode step of the 35B model (10 of its 40 decoder layers):
// [HF] Qwen3_5MoeAttention.forward for 1..16 tokens that follow `length`
// cached positions -- q_proj (query and output gate per head), k_proj,
// v_proj, per-head RMSNorm of query and key, the rotary embedding of the
// first 64 of each head's 256 dims, the key/value cache append, causal
// attention of 16 query heads over 2 key/value heads, the sigmoid output
// gate and o_proj.  The reference runs this module stock
// (Transformers SDPA); edge35b/delta_decode.py replaces only the
// linear-attention layers.
//
// Four launches on the caller's stream:
//
//   at_project<36, 2048>  q/gate, k and v rows of x (9216 rows in 256
//        workgroups of 36 rows, one per CU): each wave streams
//        its k range of every row, 4 rows x 256 B per load instruction,
//        through its own LDS stage into the MFMA layout; the T <= 16 tokens
//        are the MFMA's 16 columns; bf16 out (proj).
//   at_attend  one workgroup per (key/value head g, chunk of whole
//        32-position sub-blocks), and above 8 tokens per token half of it
//        (up to 64 query rows per workgroup, so that the 130 chunks of 4096
//        cached positions become 256 workgroups on 256 CUs):
//        the query rows of heads 8g..8g+7 normalised and rotated into LDS,
//        the chunk's new positions (those >= length) normalised, rotated
//        and appended to the caches, then per 32-position sub-block: key
//        and value rows into LDS, scores by MFMA
//        (bf16-rounded, / 16), an online softmax per query row, P.V by MFMA
//        into per-wave accumulators; the chunk's (max, sum, unnormalised
//        rows) go to the partial buffers, the rows as bf16 (half the bytes
//        of fp32: at 16 tokens the partials outweigh the 8 MB of cached
//        keys and values read).
//   at_combine  per (token, head, eighth or quarter of the dims): the
//        chunks' partials merged, the sigmoid gate applied (att, bf16).
//   at_project<8, 4096>  o_proj rows of att (2048 rows in 256 workgroups).
//
// Rounding points follow the Transformers forward in bf16: projections,
// normed and rotated q/k, scores (then / 16, exact) and the attention
// output are bf16; the softmax is fp32 (its probabilities enter P.V as
// bf16 values relative to the chunk's running maximum), and so are the
// chunks' maxima, sums and the merge; the unnormalised chunk rows are
// rounded to bf16 once (2^-9 of each chunk's row, the size of the output's
// own rounding).
#include "lrmoe_device.h"
#include "lrmoe_internal.h"

// Timeline build (-DLRMOE_TIMELINE, liblrmoe_timeline.so; the product
// library has none of it): thread 0 of every workgroup stamps the 100 MHz
// wall clock into the buffer given by lrmoe_attn_timeline_set, 8192 words
// per launch: at_project (q/gate/k/v) words 8192 + 4 b: 0 entry, 1 end;
// at_attend words 16 b: 0 entry, 1 first barrier passed (query rows,
// norm weights, cos, sin landed), 2 query rows normed and rotated, 3 new
// positions appended, 4 + n sub-block n done (n < 3), 7 partials stored;
// at_combine words 16384 + 4 b and o_proj words 24576 + 4 b: 0 entry, 1 end.
#ifdef LRMOE_TIMELINE
__device__ unsigned long long* g_attn_timeline;
extern "C" int lrmoe_attn_timeline_set(void* p) {
    return static_cast<int>(hipMemcpyToSymbol(HIP_SYMBOL(g_attn_timeline), &p, sizeof(p)));
}
#define AT_TL(base, stride, k)                                                                   \
    do {                                                                                         \
        if (threadIdx.x == 0 && g_attn_timeline != nullptr)                                      \
            g_attn_timeline[(base) + blockIdx.x * (stride) + (k)] = wall_clock64();               \
    } while (0)
#else
#define AT_TL(base, stride, k)
#endif

namespace lrmoe {
namespace {

constexpr int kAtHeads = 16;                       // query heads
constexpr int kAtKv = 2;                           // key/value heads
constexpr int kAtGroup = kAtHeads / kAtKv;         // query heads per key/value head
constexpr int kAtD = 256;                          // head width
constexpr int kAtRot = 64;                         // rotary width
constexpr int kAtQg = kAtHeads * 2 * kAtD;         // 8192 q_proj rows (256 query, 256 gate per head)
constexpr int kAtKRow = kAtQg;                     // first k_proj row of proj
constexpr int kAtVRow = kAtQg + kAtKv * kAtD;      // first v_proj row of proj
constexpr int kAtProj = kAtQg + 2 * kAtKv * kAtD;  // 9216 projected rows
constexpr int kAtO = kAtHeads * kAtD;              // 4096 o_proj inputs
constexpr int kAtThreads = 512;
constexpr int kAtWaves = kAtThreads / 64;
constexpr int kAtSub = 32;                          // positions per sub-block
constexpr int kAtQStride = kAtD + 8;                // LDS row strides (bf16 / fp32 elements)
constexpr int kAtVStride = kAtSub + 8;
constexpr int kAtSStride = kAtSub + 4;  // (rows 4 apart 16 banks apart: the score stores conflict 2-way)
constexpr float kAtScale = 0.0625f;                 // 256^-0.5, exact

// ---- projections: y[t][row] = bf16(sum_k W[row][k] x[t][k]) ---------------

// Rows [0, split1) come from w0, [split1, split2) from w1 (row - split1),
// the rest from w2 (row - split2): the q/gate, k and v matrices in one grid.
// Fused decoder glue: with kNorm, x is the raw residual stream and its rows
// are put through the input RMSNorm (weights `norm`, `eps`) on the way into
// the MFMA operands, bit for bit as a separate norm would write them
// (workgroup 0 stores them in norm_out when it is not null); with
// kResidual, sum_out also receives bf16(residual + y).
struct ProjectGlue {
    const uint16_t* norm;
    float eps;
    uint16_t* norm_out;
    const uint16_t* residual;
    uint16_t* sum_out;
};

// A workgroup projects kRows rows (8 waves, one workgroup per CU, every CU
// the same rows: 36 of q/gate/k/v, 8 of o_proj): wave w takes the k range
// [kKw w, kKw (w + 1)) of every row.  Its weight loads, all issued at once
// (non-temporal), cover 4 rows x 256 B each (lanes 16 j .. 16 j + 15: one
// row's 256 contiguous bytes, so an instruction reads whole 128-byte
// lines) and pass per 16-row MFMA tile through the wave's own LDS stage
// into the MFMA layout (lane (m, g) of step s: row m, elements 32 s + 8 g
// ..; stage rows past a short tile hold stale values, their outputs are
// dropped); the T <= 16 tokens are the MFMA's 16 columns, and the waves'
// sums meet in LDS in wave order.  A row's matrix is chosen per row: rows
// [0, split1) from w0, [split1, split2) from w1 (row - split1), the rest
// from w2 (row - split2), splits and row0 multiples of 4.
template <int kRows>
__device__ constexpr int at_tile_parts(int a) {  // 4-row loads of tile a per span
    return (kRows - 16 * a) >= 16 ? 4 : (kRows - 16 * a) / 4;
}

template <int kRows, int kK, bool kNorm = false, bool kResidual = false>
__global__ __launch_bounds__(kAtThreads, 2) void at_project(
    const uint16_t* __restrict__ w0, const uint16_t* __restrict__ w1, const uint16_t* __restrict__ w2, int split1,
    int split2, const uint16_t* __restrict__ x, int tokens, uint16_t* __restrict__ y, int y_stride, ProjectGlue glue) {
    constexpr int kTiles = (kRows + 15) / 16;
    constexpr int kKw = kK / kAtWaves;              // k range of a wave
    constexpr int kSpans = kKw / 128;               // 128-element spans per row
    constexpr int kLoads = kSpans * kRows / 4;      // 16-byte weight loads per lane
    constexpr int kSteps = kKw / 32;
    constexpr int kStageRow = 256 + 16;             // bytes per staged row (+16: conflict-free both ways)
    static_assert(kKw % 128 == 0 && kRows % 4 == 0 && kLoads <= 24, "whole spans and 4-row loads");
    __shared__ __attribute__((aligned(16))) uint8_t stage[kAtWaves][16 * kStageRow];
    __shared__ float red[kAtWaves][16 * kTiles][17];
    const int tid = threadIdx.x;
    const int lane = tid & 63;
    const int wave = tid >> 6;
    const int t = lane & 15;
    const int g = lane >> 4;
    const int row0 = blockIdx.x * kRows;
    [[maybe_unused]] constexpr int kTl = kK == kHidden ? 8192 : 24576;  // (timeline words of this launch)
    AT_TL(kTl, 4, 0);
    // token rows first (columns t >= T read token 0: their outputs are
    // dropped) and what the fused norm needs, then the weights, tile by
    // tile: load (tile a, span j, part p) is row 16 a + 4 p + lane / 16,
    // bytes 256 j + 16 (lane % 16) of the wave's range
    uint4 xb[kSteps];
    const uint16_t* xrow = x + static_cast<int64_t>(t < tokens ? t : 0) * kK + kKw * wave + 8 * g;
#pragma unroll
    for (int s = 0; s < kSteps; ++s) xb[s] = ldg16(xrow + 32 * s);
    // the fused input norm: wave w's rows w and w + 8 in the norm's layout
    // (lane l: elements 32 l ..); its weights (4 KiB) pass through LDS
    [[maybe_unused]] uint4 nrow[2][4], wn = make_uint4(0, 0, 0, 0);
    [[maybe_unused]] uint32_t res[(16 * kRows + kAtThreads - 1) / kAtThreads] = {};
    static_assert(!kNorm || (kK == kHidden && kHidden == 8 * 256), "the input norm runs over hidden rows");
    if constexpr (kNorm) {
#pragma unroll
        for (int h = 0; h < 2; ++h) {
            const int r = wave + 8 * h;
            const uint16_t* src = x + static_cast<int64_t>(r < tokens ? r : 0) * kK + 32 * lane;
#pragma unroll
            for (int i = 0; i < 4; ++i) nrow[h][i] = ldg16(src + 8 * i);
        }
        wn = ldg16(glue.norm + 8 * (tid & 255));
    }
    const uint16_t* wsrc[kRows / 4];  // the lane's row of each 4-row group, at the wave's range
#pragma unroll
    for (int q = 0; q < kRows / 4; ++q) {
        const int r = row0 + 4 * q + (lane >> 4);
        wsrc[q] = (r < split1   ? w0 + static_cast<int64_t>(r) * kK
                   : r < split2 ? w1 + static_cast<int64_t>(r - split1) * kK
                                : w2 + static_cast<int64_t>(r - split2) * kK) +
                  kKw * wave + 8 * (lane & 15);
    }
    uint4 wv[kLoads];
#pragma unroll
    for (int a = 0; a < kTiles; ++a)
#pragma unroll
        for (int j = 0; j < kSpans; ++j)
#pragma unroll
            for (int p = 0; p < 4; ++p)
                if (p < at_tile_parts<kRows>(a))
                    wv[4 * kSpans * a + at_tile_parts<kRows>(a) * j + p] = ldg16_nt(wsrc[4 * a + p] + 128 * j);
    if constexpr (kResidual) {
        // output (row row0 + i / 16, token i % 16) for i = tid, tid + 512, ..
        // (tokens clamped where none is stored)
#pragma unroll
        for (int k = 0; k < (16 * kRows + kAtThreads - 1) / kAtThreads; ++k) {
            const int i = tid + kAtThreads * k < 16 * kRows ? tid + kAtThreads * k : 0;
            const int rt = (i & 15) < tokens ? (i & 15) : 0;
            res[k] = ldg_u16(glue.residual + static_cast<int64_t>(rt) * y_stride + row0 + (i >> 4));
        }
    }
    if constexpr (kNorm) {
        __shared__ float rscale[16];
        __shared__ __attribute__((aligned(16))) uint16_t nw[kHidden];
        if (tid < 256) *reinterpret_cast<uint4*>(&nw[8 * tid]) = wn;
#pragma unroll
        for (int h = 0; h < 2; ++h) {
            const float r = row_rms_scale(nrow[h], glue.eps);
            if (lane == 0) rscale[wave + 8 * h] = r;
        }
        __syncthreads();
        const float r = rscale[t < tokens ? t : 0];
#pragma unroll
        for (int s = 0; s < kSteps; ++s)
            xb[s] = rms_apply8(xb[s], *reinterpret_cast<const uint4*>(&nw[kKw * wave + 32 * s + 8 * g]), r);
        if (blockIdx.x == 0 && glue.norm_out != nullptr && t < tokens) {
#pragma unroll
            for (int s = 0; s < kSteps; ++s)
                *reinterpret_cast<uint4*>(glue.norm_out + static_cast<int64_t>(t) * kK + kKw * wave + 32 * s + 8 * g) = xb[s];
        }
    }
    // per tile: the steps in order into one accumulator (per span: the
    // tile's loads into the stage, four operands back out in the MFMA layout)
    uint8_t* st = stage[wave];
#pragma unroll
    for (int a = 0; a < kTiles; ++a) {
        f32x4 acc = {0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
        for (int j = 0; j < kSpans; ++j) {
#pragma unroll
            for (int p = 0; p < 4; ++p)
                if (p < at_tile_parts<kRows>(a))
                    *reinterpret_cast<uint4*>(st + (4 * p + (lane >> 4)) * kStageRow + 16 * (lane & 15)) =
                        wv[4 * kSpans * a + at_tile_parts<kRows>(a) * j + p];
            // (the stage is the wave's own: in-order LDS access within the
            // wave, and no reordering by the compiler across these fences)
            __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
            __builtin_amdgcn_wave_barrier();
            __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
            uint4 op[4];
#pragma unroll
            for (int s = 0; s < 4; ++s) op[s] = *reinterpret_cast<const uint4*>(st + t * kStageRow + 16 * (4 * s + g));
            __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
            __builtin_amdgcn_wave_barrier();
            __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
#pragma unroll
            for (int s = 0; s < 4; ++s) acc = mfma16x16x32(op[s], xb[4 * j + s], acc);
        }
#pragma unroll
        for (int i = 0; i < 4; ++i) red[wave][16 * a + 4 * g + i][t] = acc[i];
    }
    __syncthreads();
#pragma unroll
    for (int k = 0; k < (16 * kRows + kAtThreads - 1) / kAtThreads; ++k) {
        const int i = tid + kAtThreads * k;
        if (i < 16 * kRows) {
            const int r = i >> 4;
            const int tt = i & 15;
            float p = 0.0f;
#pragma unroll
            for (int ww = 0; ww < kAtWaves; ++ww) p += red[ww][r][tt];
            const uint32_t o = f2bf(p);
            if (tt < tokens) {
                y[static_cast<int64_t>(tt) * y_stride + row0 + r] = static_cast<uint16_t>(o);
                if constexpr (kResidual)
                    glue.sum_out[static_cast<int64_t>(tt) * y_stride + row0 + r] =
                        static_cast<uint16_t>(f2bf(bf2f(res[k]) + bf2f(o)));
            }
        }
    }
    AT_TL(kTl, 4, 1);
}

// ---- attention partials ------------------------------------------------------

// exp(x) for the softmax with the hardware base-2 exponential (x <= 0 here;
// exp(-inf) = 0).  The attention parity is a float tolerance, not bits.
__device__ __forceinline__ float fast_exp(float x) { return __builtin_amdgcn_exp2f(x * 1.4426950408889634f); }

// A lane's value moved by DPP control kCtrl (rows outside kRowMask get
// `old`): a VALU cross-lane move, no LDS round trip.
template <int kCtrl, int kRowMask = 0xf>
__device__ __forceinline__ float dpp_f(float v, float old = 0.0f) {
    return __int_as_float(
        __builtin_amdgcn_update_dpp(__float_as_int(old), __float_as_int(v), kCtrl, kRowMask, 0xf, false));
}

// Sum and maximum over the 64 lanes, returned to every lane: quads (quad_perm
// [1,0,3,2], [2,3,0,1]), the other quad of each 8 (row_half_mirror), the
// other 8 of each row (row_mirror), then rows 0+1 and 2+3 (row_bcast15 into
// rows 1, 3) and all four (row_bcast31 into rows 2, 3): lane 63 holds the
// result.  The attention's sums need float accuracy, not a fixed order.
__device__ __forceinline__ float wave_sum_dpp(float v) {
    v += dpp_f<0xB1>(v);
    v += dpp_f<0x4E>(v);
    v += dpp_f<0x141>(v);
    v += dpp_f<0x140>(v);
    v += dpp_f<0x142, 0xa>(v);
    v += dpp_f<0x143, 0xc>(v);
    return __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), 63));
}

__device__ __forceinline__ float wave_max_dpp(float v) {
    v = fmaxf(v, dpp_f<0xB1>(v));
    v = fmaxf(v, dpp_f<0x4E>(v));
    v = fmaxf(v, dpp_f<0x141>(v));
    v = fmaxf(v, dpp_f<0x140>(v));
    v = fmaxf(v, dpp_f<0x142, 0xa>(v, v));  // (rows the broadcast skips keep their own)
    v = fmaxf(v, dpp_f<0x143, 0xc>(v, v));
    return __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), 63));
}

// The norm factors 1 + w of a lane's 4 dims (dims 4 lane .. 4 lane + 3).
__device__ __forceinline__ void norm_scale(const uint16_t* w, int lane, float (&w1)[4]) {
    const uint2 wr = *reinterpret_cast<const uint2*>(w + 4 * lane);
    const float wf[4] = {lo_bf(wr.x), hi_bf(wr.x), lo_bf(wr.y), hi_bf(wr.y)};
#pragma unroll
    for (int i = 0; i < 4; ++i) w1[i] = 1.0f + wf[i];
}

// One head row (256 dims, 4 per lane) normalised: x rsqrt(mean x^2 + eps)
// (1 + w) in fp32, not yet rounded (v_rsq_f32: the attention's bar is a
// float tolerance).  Every lane of the wave calls it.
__device__ __forceinline__ void rms_norm_row(uint2 raw, const float (&w1)[4], float eps, float (&n)[4]) {
    const float x[4] = {lo_bf(raw.x), hi_bf(raw.x), lo_bf(raw.y), hi_bf(raw.y)};
    const float ss = wave_sum_dpp(x[0] * x[0] + x[1] * x[1] + x[2] * x[2] + x[3] * x[3]);
    const float r = __builtin_amdgcn_rsqf(ss / static_cast<float>(kAtD) + eps);
#pragma unroll
    for (int i = 0; i < 4; ++i) n[i] = (x[i] * r) * w1[i];
}

// The rotary embedding of one element: bf16(bf16(x cos) + bf16(rot sin)),
// rot = -x[d + 32] for d < 32, x[d - 32] for 32 <= d < 64.
__device__ __forceinline__ float rope1(float x, float rot, float c, float s) {
    return rbf(rbf(x * c) + rbf(rot * s));
}

// A head row normalised and rotated on dims 0..63 (lanes 0..15 hold them;
// lane l pairs with lane l ^ 8, the row rotation by 8), as packed bf16.
// Every lane of the wave calls it.
__device__ __forceinline__ uint2 norm_rope(uint2 raw, const uint16_t* w, float eps, const uint16_t* cos_r,
                                          const uint16_t* sin_r, int lane) {
    float w1[4], n[4];
    norm_scale(w, lane, w1);
    rms_norm_row(raw, w1, eps, n);
#pragma unroll
    for (int i = 0; i < 4; ++i) n[i] = rbf(n[i]);
    const int d0 = 4 * (lane & 15);
    const uint2 cr = *reinterpret_cast<const uint2*>(cos_r + d0);
    const uint2 sr = *reinterpret_cast<const uint2*>(sin_r + d0);
    const float cf[4] = {lo_bf(cr.x), hi_bf(cr.x), lo_bf(cr.y), hi_bf(cr.y)};
    const float sf[4] = {lo_bf(sr.x), hi_bf(sr.x), lo_bf(sr.y), hi_bf(sr.y)};
    float o[4];
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        const float partner = dpp_f<0x128>(n[i]);  // row_ror:8
        const float v = rope1(n[i], (lane & 8) ? partner : -partner, cf[i], sf[i]);
        o[i] = lane < 16 ? v : n[i];
    }
    return make_uint2(pack_bf2(o[0], o[1]), pack_bf2(o[2], o[3]));
}

// kRows query rows (8 per token), kTok tokens' rotary rows and new-position
// key/value rows (all of the call's tokens: a workgroup of one token half
// still appends, and attends over, every new position).
template <int kRows, int kTok>
struct AttendLds {
    static constexpr int kMaxT = kTok;
    __attribute__((aligned(16))) uint16_t qs[kRows][kAtQStride];  // normed, rotated query rows
    __attribute__((aligned(16))) uint16_t ks[kAtSub][kAtQStride];  // a sub-block's key rows
    __attribute__((aligned(16))) uint16_t vs[kAtSub][kAtQStride];  // its value rows
    float sc[kRows][kAtSStride];                                   // its scores
    __attribute__((aligned(16))) uint16_t es[kRows][kAtVStride];   // its exp(score - max), bf16
    __attribute__((aligned(16))) float mrow[kRows];
    __attribute__((aligned(16))) float lrow[kRows];
    __attribute__((aligned(16))) float frow[kRows];
    __attribute__((aligned(16))) uint16_t nw[2][kAtD];             // q_norm, k_norm
    __attribute__((aligned(16))) uint16_t cs[2][kMaxT][kAtRot];    // cos, sin
    __attribute__((aligned(16))) uint16_t fk[kMaxT][kAtD];         // the new positions' key rows
    __attribute__((aligned(16))) uint16_t fv[kMaxT][kAtD];         // and value rows
};

// Key and value rows of the sub-block at q0 into kb[parity] / vb[parity]
// (16-byte piece j = tid + 512 i: row j / 32, dims 8 (j % 32) ..; rows at or
// past p1 read zeros: the buffer range ends there).
__device__ __forceinline__ void attend_issue(uint4 (&kb)[2][2], uint4 (&vb)[2][2], int parity, const uint16_t* kc,
                                             const uint16_t* vc, int q0, uint32_t range, int tid) {
#pragma unroll
    for (int i = 0; i < 2; ++i) {
        const int j = tid + kAtThreads * i;
        const uint32_t off = static_cast<uint32_t>(((q0 + (j >> 5)) * kAtD + 8 * (j & 31)) * 2);
        kb[parity][i] = ld_agent16(kc, off, range);
        vb[parity][i] = ld_agent16(vc, off, range);
    }
}

// Cached positions before the call: the host's value or, for a call whose
// launches are replayed as the cache grows, the value at length_dev (read
// at kernel start), clamped to [0, capacity - tokens] so that no read leaves
// the caches; for a value outside that range at_attend writes no cache row
// and at_combine writes NaN rows.
__device__ __forceinline__ int attn_length(const AttnArgs& a) {
    if (a.length_dev == nullptr) return a.length;
    const int v = *a.length_dev;
    return v < 0 ? 0 : (v > a.capacity - a.tokens ? a.capacity - a.tokens : v);
}
__device__ __forceinline__ bool attn_length_bad(const AttnArgs& a) {
    if (a.length_dev == nullptr) return false;
    const int v = *a.length_dev;
    return v < 0 || v > a.capacity - a.tokens;
}

// The attention partials of chunk c of key/value head g, for 8 T <= kRows
// query rows (512 threads): the query rows normed and rotated, the chunk's
// new positions appended, then per 32-position sub-block scores, online
// softmax and P.V; (max, sum, unnormalised rows) to the partial buffers.
// kb / vb carry the key and value rows of two sub-blocks in flight.
template <int kRows, int kTok, bool kHalves>
__device__ __forceinline__ void attend_chunk(const AttnArgs& a, AttendLds<kRows, kTok>& S, int g, int c, int half,
                                             uint4 (&kb)[2][2], uint4 (&vb)[2][2]) {
    constexpr int kMaxT = kRows / kAtGroup;  // query tokens per workgroup
    constexpr int kRowTiles = kRows / 16;
    auto& qs = S.qs;
    auto& ks = S.ks;
    auto& vs = S.vs;
    auto& sc = S.sc;
    auto& es = S.es;
    auto& mrow = S.mrow;
    auto& lrow = S.lrow;
    auto& frow = S.frow;
    auto& nw = S.nw;
    auto& cs = S.cs;
    auto& fk = S.fk;
    auto& fv = S.fv;

    const int tid = threadIdx.x;
    const int lane = tid & 63;
    const int wave = tid >> 6;
    const int m = lane & 15;
    const int gq = lane >> 4;
    const int T = a.tokens;
    // this workgroup's query tokens t0 .. t0 + Tq - 1 (its rows r = 8 (t - t0)
    // + local head; rows 8 t0 .. of the chunk's partials)
    const int t0 = kHalves ? half * a.t_half : 0;
    const int Tq = kHalves ? (half == 0 ? a.t_half : T - a.t_half) : T;
    const int R = kAtGroup * Tq;
    const int RT = (R + 15) / 16;
    const int L = attn_length(a);  // (chunks past L + T read and write nothing: empty partials)
    const int total = L + T;
    // chunk c: sub-blocks c per .. (c + 1) per - 1, the last chunk to the end
    const int p0 = kAtSub * c * a.per;
    const int last = c + 1 == a.chunks ? 1 : 0;  // (arithmetic, not a branch ahead of the first loads)
    const int p1 = min(kAtSub * ((c + 1) * a.per + last * (a.sub_blocks - (c + 1) * a.per)), total);
    uint16_t* kc = a.k_cache + static_cast<int64_t>(g) * a.capacity * kAtD;
    uint16_t* vc = a.v_cache + static_cast<int64_t>(g) * a.capacity * kAtD;
    AT_TL(0, 16, 0);

    // Every load below is issued by every lane (dummy addresses where a lane
    // needs none), in the order of need, so that the compiler's in-order
    // waits for one cover only what is older.
    // (1) wave w's query rows: head 8g + w, tokens t0 .. t0 + Tq - 1 (rows w + 8 j)
    uint2 raw[kMaxT];
    const uint16_t* qsrc = a.proj + (kAtGroup * g + wave) * 2 * kAtD + 4 * lane;
#pragma unroll
    for (int j = 0; j < kMaxT; ++j)
        raw[j] = *reinterpret_cast<const uint2*>(qsrc + static_cast<int64_t>(t0 + (j < Tq ? j : 0)) * kAtProj);
    // (2) norm weights, cos, sin: 8-byte pieces; piece i < 128 a norm
    // weight's, then T x 16 pieces of cos and of sin
    const int pieces = 128 + 32 * T;
    uint2 pc[2];
#pragma unroll
    for (int k = 0; k < 2; ++k) {
        const int i = tid + kAtThreads * k < pieces ? tid + kAtThreads * k : 0;
        const uint16_t* src = i < 64 ? a.q_norm + 4 * i
                            : i < 128 ? a.k_norm + 4 * (i - 64)
                            : ((i - 128) < 16 * T ? a.cos : a.sin) + 4 * ((i - 128) % (16 * T));
        pc[k] = *reinterpret_cast<const uint2*>(src);
    }
    // (2b) the chunk's new positions (p >= length): their projected key and
    // value rows, wave w taking positions p_new + w + 8 i (token 0's rows
    // where there is none), loaded here so that the chunk holding them
    // does not wait for a second round trip below
    const int p_new = attn_length_bad(a) ? p1 : max(p0, L);  // (no cache row written for a bad length)
    constexpr int kNew = (kTok + kAtWaves - 1) / kAtWaves;
    uint2 kraw[kNew], vraw[kNew];
#pragma unroll
    for (int i = 0; i < kNew; ++i) {
        const int p = p_new + wave + kAtWaves * i;
        const uint16_t* pr = a.proj + static_cast<int64_t>(p < p1 ? p - L : 0) * kAtProj + g * kAtD + 4 * lane;
        kraw[i] = *reinterpret_cast<const uint2*>(pr + kAtKRow);
        vraw[i] = *reinterpret_cast<const uint2*>(pr + kAtVRow);
    }
    // (3) key and value rows of sub-blocks 0 and 1 (16-byte piece j of a
    // sub-block: row j / 32, dims 8 (j % 32) ..; rows past the chunk read
    // zeros: the buffer range ends at p1).  Rows of new positions read
    // whatever the cache held; the staging below takes them from fk / fv.
    const uint32_t range = static_cast<uint32_t>(p1) * kAtD * 2;
    attend_issue(kb, vb, 0, kc, vc, p0, range, tid);
    attend_issue(kb, vb, 1, kc, vc, p0 + kAtSub, range, tid);
#pragma unroll
    for (int k = 0; k < 2; ++k) {
        const int i = tid + kAtThreads * k;
        if (i < pieces) {
            uint16_t* dst = i < 128 ? &nw[i >> 6][4 * (i & 63)]
                                    : &cs[(i - 128) / (16 * T)][((i - 128) % (16 * T)) >> 4][4 * ((i - 128) & 15)];
            *reinterpret_cast<uint2*>(dst) = pc[k];
        }
    }
    if (tid < kRows) {
        mrow[tid] = -__builtin_inff();
        lrow[tid] = 0.0f;
        frow[tid] = 1.0f;
    }
    __syncthreads();
    AT_TL(0, 16, 1);
    // (4) the query rows normed and rotated into qs: one row when T = 1;
    // else (a) every row of the wave normalised, up to 8 rows per pass (rows
    // past T repeat token 0 and are not stored) so that their independent
    // reductions interleave, then (b) the rotary dims of the wave's rows
    // rotated in place, lane l taking row l / 4, dims 16 (l % 4) .. + 15
    if (T == 1) {
        *reinterpret_cast<uint2*>(&qs[wave][4 * lane]) = norm_rope(raw[0], nw[0], a.eps, cs[0][0], cs[1][0], lane);
    } else {
        constexpr int kPass = kMaxT < 8 ? kMaxT : 8;
        float w1[4];
        norm_scale(nw[0], lane, w1);
#pragma unroll
        for (int j0 = 0; j0 < kMaxT; j0 += kPass) {
            if (j0 < Tq) {
                float n[kPass][4];
#pragma unroll
                for (int j = 0; j < kPass; ++j) rms_norm_row(raw[j0 + j], w1, a.eps, n[j]);
#pragma unroll
                for (int j = 0; j < kPass; ++j)
                    if (j0 + j < Tq)
                        *reinterpret_cast<uint2*>(&qs[wave + kAtGroup * (j0 + j)][4 * lane]) =
                            make_uint2(pack_bf2(n[j][0], n[j][1]), pack_bf2(n[j][2], n[j][3]));
            }
        }
        // (the wave's LDS stores above are complete before its loads below)
        __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
        __builtin_amdgcn_wave_barrier();
        __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
        const int j = lane >> 2;
        const int qd = lane & 3;
        if (j < Tq) {
            uint16_t* row = &qs[wave + kAtGroup * j][0];
            const uint4* own = reinterpret_cast<const uint4*>(row + 16 * qd);
            const uint4* mate = reinterpret_cast<const uint4*>(row + 16 * (qd ^ 2));
            const uint4* cp = reinterpret_cast<const uint4*>(&cs[0][t0 + j][16 * qd]);
            const uint4* sp = reinterpret_cast<const uint4*>(&cs[1][t0 + j][16 * qd]);
            const uint4 xv[2] = {own[0], own[1]};
            const uint4 pv[2] = {mate[0], mate[1]};
            const uint4 cv[2] = {cp[0], cp[1]};
            const uint4 sv[2] = {sp[0], sp[1]};
            const float sign = qd < 2 ? -1.0f : 1.0f;
            uint4 out[2];
#pragma unroll
            for (int h = 0; h < 2; ++h) {
                const uint32_t xw[4] = {xv[h].x, xv[h].y, xv[h].z, xv[h].w};
                const uint32_t pw[4] = {pv[h].x, pv[h].y, pv[h].z, pv[h].w};
                const uint32_t cw[4] = {cv[h].x, cv[h].y, cv[h].z, cv[h].w};
                const uint32_t sw[4] = {sv[h].x, sv[h].y, sv[h].z, sv[h].w};
                uint32_t ow[4];
#pragma unroll
                for (int e = 0; e < 4; ++e)
                    ow[e] = pack_bf2(rope1(lo_bf(xw[e]), sign * lo_bf(pw[e]), lo_bf(cw[e]), lo_bf(sw[e])),
                                     rope1(hi_bf(xw[e]), sign * hi_bf(pw[e]), hi_bf(cw[e]), hi_bf(sw[e])));
                out[h] = make_uint4(ow[0], ow[1], ow[2], ow[3]);
            }
            // (a lane's own dims are read by it and by its mate, lane l ^ 2;
            // the stores use every value loaded, so they follow both reads)
            reinterpret_cast<uint4*>(row + 16 * qd)[0] = out[0];
            reinterpret_cast<uint4*>(row + 16 * qd)[1] = out[1];
        }
    }
    AT_TL(0, 16, 2);
    // (5) new positions of this chunk: keys normed and rotated, values as
    // projected, into fk / fv for this call and appended to the caches for
    // later ones (no other workgroup reads them in this call)
#pragma unroll
    for (int i = 0; i < kNew; ++i) {
        const int p = p_new + wave + kAtWaves * i;
        if (p < p1) {
            const int t = p - L;
            const uint2 k = norm_rope(kraw[i], nw[1], a.eps, cs[0][t], cs[1][t], lane);
            *reinterpret_cast<uint2*>(&fk[t][4 * lane]) = k;
            *reinterpret_cast<uint2*>(&fv[t][4 * lane]) = vraw[i];
            st_agent64(kc + static_cast<int64_t>(p) * kAtD + 4 * lane,
                       static_cast<uint64_t>(k.x) | (static_cast<uint64_t>(k.y) << 32));
            st_agent64(vc + static_cast<int64_t>(p) * kAtD + 4 * lane,
                       static_cast<uint64_t>(vraw[i].x) | (static_cast<uint64_t>(vraw[i].y) << 32));
        }
    }
    __syncthreads();
    AT_TL(0, 16, 3);

    // The 64-row variants keep each wave's query operands (row tile w / 2 of
    // the scores) in registers for every sub-block: half the LDS reads of
    // the score phase.
    static_assert(kRowTiles <= 4, "one score row tile per wave");
    constexpr bool kQReg = kRows == 64;
    [[maybe_unused]] uint4 qa[kQReg ? kAtD / 32 : 1];
    if constexpr (kQReg) {
        const int rt = wave >> 1;
#pragma unroll
        for (int s = 0; s < kAtD / 32; ++s)
            qa[s] = rt < RT ? *reinterpret_cast<const uint4*>(&qs[16 * rt + m][32 * s + 8 * gq]) : make_uint4(0, 0, 0, 0);
    }

    // P.V accumulators: wave w owns dim tiles 2w, 2w + 1 of every row tile
    f32x4 acc[kRowTiles][2];
#pragma unroll
    for (int rt = 0; rt < kRowTiles; ++rt)
#pragma unroll
        for (int j = 0; j < 2; ++j) acc[rt][j] = f32x4{0.0f, 0.0f, 0.0f, 0.0f};

    // One sub-block: its rows from registers into ks / vs (16-byte stores
    // along a row), the registers refilled with the sub-block two ahead,
    // then scores, softmax, P.V.
    auto sub_block = [&](int parity, int q0) __attribute__((always_inline)) {
#pragma unroll
        for (int i = 0; i < 2; ++i) {
            const int j = tid + kAtThreads * i;
            const int row = j >> 5;
            const int col = 8 * (j & 31);
            const int t = q0 + row - L;  // a new position: its rows from fk / fv
            const bool fresh = t >= 0 && q0 + row < p1;
            // (both read, then selected: a select of addresses would put the
            // register rows in memory)
            const uint4 nk = *reinterpret_cast<const uint4*>(&fk[fresh ? t : 0][col]);
            const uint4 nv = *reinterpret_cast<const uint4*>(&fv[fresh ? t : 0][col]);
            const uint4 ok = kb[parity][i];
            const uint4 ov = vb[parity][i];
            *reinterpret_cast<uint4*>(&ks[row][col]) =
                make_uint4(fresh ? nk.x : ok.x, fresh ? nk.y : ok.y, fresh ? nk.z : ok.z, fresh ? nk.w : ok.w);
            *reinterpret_cast<uint4*>(&vs[row][col]) =
                make_uint4(fresh ? nv.x : ov.x, fresh ? nv.y : ov.y, fresh ? nv.z : ov.z, fresh ? nv.w : ov.w);
        }
        attend_issue(kb, vb, parity, kc, vc, q0 + 2 * kAtSub, range, tid);
        __syncthreads();
        // scores: wave w takes column tile w & 1 of row tile w / 2
        {
            const int ct = wave & 1;
            {
                const int rt = wave >> 1;
                if (rt < RT) {
                    f32x4 s4 = {0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
                    for (int s = 0; s < kAtD / 32; ++s) {
                        uint4 qop;
                        if constexpr (kQReg) qop = qa[s];
                        else qop = *reinterpret_cast<const uint4*>(&qs[16 * rt + m][32 * s + 8 * gq]);
                        s4 = mfma16x16x32(qop, *reinterpret_cast<const uint4*>(&ks[16 * ct + m][32 * s + 8 * gq]), s4);
                    }
                    const int pos = q0 + 16 * ct + m;
#pragma unroll
                    for (int i = 0; i < 4; ++i) {
                        const int r = 16 * rt + 4 * gq + i;
                        const bool ok = r < R && pos < p1 && pos <= L + t0 + (r >> 3);
                        sc[r][16 * ct + m] = ok ? rbf(s4[i]) * kAtScale : -__builtin_inff();
                    }
                }
            }
        }
        __syncthreads();
        // online softmax: four threads per row, eight positions each.  P.V's
        // k-slot 8 q + j (the A operand's lane group q) holds position
        // 2 q + 8 (j / 2) + j % 2, the same in the probabilities (es) and
        // in the value rows gathered below: the gather's four lane groups
        // then read rows 2 apart, in disjoint banks.
        {
            const int r = tid >> 2;
            const int q = tid & 3;
            if (r < R) {  // (R is a multiple of 8: whole quads take part)
                float s8[8];
                float mx = -__builtin_inff();
#pragma unroll
                for (int j = 0; j < 8; j += 2) {
                    const float2 pr = *reinterpret_cast<const float2*>(&sc[r][2 * q + 8 * (j >> 1)]);
                    s8[j] = pr.x;
                    s8[j + 1] = pr.y;
                    mx = fmaxf(mx, fmaxf(pr.x, pr.y));
                }
                mx = fmaxf(mx, dpp_f<0xB1>(mx));
                mx = fmaxf(mx, dpp_f<0x4E>(mx));
                const float m_old = mrow[r];
                const float m_new = fmaxf(m_old, mx);
                const bool none = m_new == -__builtin_inff();
                float sum = 0.0f;
                uint32_t e2[4];
#pragma unroll
                for (int j = 0; j < 8; j += 2) {
                    const uint32_t e = pack_bf2(none ? 0.0f : fast_exp(s8[j] - m_new),
                                                none ? 0.0f : fast_exp(s8[j + 1] - m_new));
                    sum += lo_bf(e) + hi_bf(e);
                    e2[j / 2] = e;
                }
                *reinterpret_cast<uint4*>(&es[r][8 * q]) = make_uint4(e2[0], e2[1], e2[2], e2[3]);
                sum += dpp_f<0xB1>(sum);
                sum += dpp_f<0x4E>(sum);
                const float f = none ? 1.0f : (m_old == -__builtin_inff() ? 0.0f : fast_exp(m_old - m_new));
                if (q == 0) {
                    mrow[r] = m_new;
                    lrow[r] = lrow[r] * f + sum;
                    frow[r] = f;
                }
            }
        }
        __syncthreads();
        // P.V: rescale, then one k-step of 32 positions per tile; the B
        // operand (k-slots 8 gq .. 8 gq + 7: positions 2 gq + 8 e, 2 gq +
        // 8 e + 1 of dim 16 dt + m) gathered from vs, once per dim tile
        uint4 vop[2];
#pragma unroll
        for (int j = 0; j < 2; ++j) {
            const int d = 16 * (2 * wave + j) + m;
            uint32_t w[4];
#pragma unroll
            for (int e = 0; e < 4; ++e)
                w[e] = static_cast<uint32_t>(vs[2 * gq + 8 * e][d]) | (static_cast<uint32_t>(vs[2 * gq + 8 * e + 1][d]) << 16);
            vop[j] = make_uint4(w[0], w[1], w[2], w[3]);
        }
#pragma unroll
        for (int rt = 0; rt < kRowTiles; ++rt) {
            if (rt < RT) {
                const uint4 ea = *reinterpret_cast<const uint4*>(&es[16 * rt + m][8 * gq]);
                const float4 f4 = *reinterpret_cast<const float4*>(&frow[16 * rt + 4 * gq]);
                const float f[4] = {f4.x, f4.y, f4.z, f4.w};
#pragma unroll
                for (int j = 0; j < 2; ++j) {
#pragma unroll
                    for (int i = 0; i < 4; ++i) acc[rt][j][i] *= f[i];
                    acc[rt][j] = mfma16x16x32(ea, vop[j], acc[rt][j]);
                }
            }
        }
        __syncthreads();
    };
    [[maybe_unused]] int n_sub = 0;  // (timeline words)
    for (int q0 = p0; q0 < p1; q0 += 2 * kAtSub) {
        sub_block(0, q0);
        AT_TL(0, 16, 4 + min(n_sub++, 2));
        if (q0 + kAtSub < p1) {
            sub_block(1, q0 + kAtSub);
            AT_TL(0, 16, 4 + min(n_sub++, 2));
        }
    }

    // the chunk's partials: unnormalised rows (bf16), running max and sum
    // per row (fp32).  Lanes m and m ^ 1 hold columns m and m ^ 1 of rows
    // 4 gq .. 4 gq + 3: one exchange, then the even lane stores rows 4 gq and
    // 4 gq + 1, the odd lane rows 4 gq + 2 and 4 gq + 3, as column pairs.
    const int Rall = kAtGroup * T;  // the chunk's partial rows
    uint16_t* po = a.part_o + ((static_cast<int64_t>(g) * a.chunks + c) * Rall + kAtGroup * t0) * kAtD;
    const bool odd = (m & 1) != 0;
#pragma unroll
    for (int rt = 0; rt < kRowTiles; ++rt) {
        if (rt < RT) {
#pragma unroll
            for (int j = 0; j < 2; ++j) {
                const uint32_t w01 = f2bf(acc[rt][j][0]) | (f2bf(acc[rt][j][1]) << 16);
                const uint32_t w23 = f2bf(acc[rt][j][2]) | (f2bf(acc[rt][j][3]) << 16);
                const uint32_t x = static_cast<uint32_t>(lane_xor<1>(static_cast<int>(odd ? w01 : w23)));
                const uint32_t own = odd ? w23 : w01;
                const uint32_t lo = odd ? (x & 0xffffu) | (own << 16) : (own & 0xffffu) | (x << 16);
                const uint32_t hi = odd ? (x >> 16) | (own & 0xffff0000u) : (own >> 16) | (x & 0xffff0000u);
                const int r = 16 * rt + 4 * gq + (odd ? 2 : 0);  // (R is a multiple of 8: r + 1 < R with r)
                if (r < R) {
                    uint16_t* dst = po + r * kAtD + 16 * (2 * wave + j) + (m & ~1);
                    *reinterpret_cast<uint32_t*>(dst) = lo;
                    *reinterpret_cast<uint32_t*>(dst + kAtD) = hi;
                }
            }
        }
    }
    if (tid < R) {
        float* pm = a.part_ml + ((static_cast<int64_t>(g) * a.chunks + c) * Rall + kAtGroup * t0 + tid) * 2;
        pm[0] = mrow[tid];
        pm[1] = lrow[tid];
    }
    AT_TL(0, 16, 7);
}

// kRows: the query rows of a workgroup (8 per token): 32 up to 4 tokens
// (about 63 KB of LDS), 64 above (103 KB).  Above 8
// tokens a chunk's rows take two workgroups, one per token half, on the
// same XCD (workgroups b and b + 8 of each group of 16), so they share the
// chunk's key and value rows through its L2.
template <int kRows, int kTok, bool kHalves>
__global__ __launch_bounds__(kAtThreads, kRows <= 32 ? 2 : 1) void at_attend(AttnArgs a) {
    __shared__ AttendLds<kRows, kTok> S;
    uint4 kb[2][2], vb[2][2];  // [sub-block parity][piece]
    if constexpr (kHalves) {
        const int b = blockIdx.x;
        const int i = (b >> 4) * 8 + (b & 7);  // (key/value head, chunk) index
        if (i >= kAtKv * a.chunks) return;     // (the grid is rounded up to whole groups of 16)
        attend_chunk<kRows, kTok, true>(a, S, i / a.chunks, i % a.chunks, (b >> 3) & 1, kb, vb);
    } else {
        attend_chunk<kRows, kTok, false>(a, S, blockIdx.x / a.chunks, blockIdx.x % a.chunks, 0, kb, vb);
    }
}

// ---- merge and gate: att[t][h][d] = bf16(bf16(o) bf16(sigmoid(gate))) -------
// kSplit workgroups per (token, head), each merging 256 / kSplit dims: the
// chunks' (max, sum) pairs into LDS, the weights exp(m_c - M) (every
// workgroup of the row computes them); thread group q (eight dims per
// thread) sums chunks q, q + kGroups, ... (every load issued at once: the
// gate, the pairs and the thread's partial rows); the groups' rows meet in
// LDS, summed in group order in two steps.
template <int kGroups, int kDims>
struct CombineLds {
    float wc[kAttnMaxChunks];
    float lc[kAttnMaxChunks];
    __attribute__((aligned(16))) float part[kGroups][kDims];
    __attribute__((aligned(16))) uint16_t out[kDims];
    float den;
};

template <int kThreads, int kSplit>
using CombineLdsOf = CombineLds<kThreads * kSplit / 32, kAtD / kSplit>;

template <int kThreads, int kSplit>
__device__ __forceinline__ void combine_row(const AttnArgs& a, CombineLdsOf<kThreads, kSplit>& S, int t, int h,
                                            int piece) {
    constexpr int kDims = kAtD / kSplit;        // dims of this workgroup
    constexpr int kRowThreads = kDims / 8;      // threads per partial row
    constexpr int kGroups = kThreads / kRowThreads;
    constexpr int kBatch = kAttnMaxChunks / kGroups;  // chunks per thread
    constexpr int kSets = kThreads / kDims;           // first summing step: kSets sets of kGroups / kSets groups
    static_assert(kThreads >= kAttnMaxChunks && kThreads >= 2 * kDims, "pairs and stores one per thread");
    static_assert(kBatch * kGroups == kAttnMaxChunks && kBatch <= 8 && kGroups % kSets == 0, "one batch of rows");
    auto& wc = S.wc;
    auto& lc = S.lc;
    auto& part = S.part;
    float& den_s = S.den;
    const int tid = threadIdx.x;
    const int g = h / kAtGroup;
    const int R = kAtGroup * a.tokens;
    const int r = kAtGroup * t + (h % kAtGroup);
    const int C = a.chunks;
    const int64_t chunk_rows = static_cast<int64_t>(g) * C;  // first chunk of head g
    // every load at once: the gate (threads < 256), the chunks' (max, sum)
    // pairs, the thread's partial rows (chunks q + kGroups k < C)
    const int q = tid / kRowThreads;
    const int dbase = kDims * piece;
    const int d0 = 8 * (tid % kRowThreads);
    const uint16_t* po = a.part_o + (chunk_rows * R + r) * kAtD + dbase + d0;
    const int64_t cstride = static_cast<int64_t>(R) * kAtD;
    // (the gate as the 4-byte word holding it)
    const int64_t gi = static_cast<int64_t>(t) * kAtProj + h * 2 * kAtD + kAtD + dbase + (tid % kDims);
    const uint32_t gword = *reinterpret_cast<const uint32_t*>(a.proj + (gi & ~1ll));
    const float* pml = a.part_ml + ((chunk_rows + (tid < C ? tid : 0)) * R + r) * 2;
    const float2 ml = *reinterpret_cast<const float2*>(pml);
    uint4 v[kBatch];
#pragma unroll
    for (int k = 0; k < kBatch; ++k) {
        const int c = q + kGroups * k;
        v[k] = c < C ? *reinterpret_cast<const uint4*>(po + static_cast<int64_t>(c) * cstride) : make_uint4(0, 0, 0, 0);
    }
    if (tid < C) {
        wc[tid] = ml.x;
        lc[tid] = ml.y;
    }
    __syncthreads();
    if (tid < 64) {  // wave 0: the maximum, the weights, the denominator
        float M = -__builtin_inff();
        for (int c = tid; c < C; c += 64) M = fmaxf(M, wc[c]);
        M = wave_max_dpp(M);
        float den = 0.0f;
        float wv[kAttnMaxChunks / 64];
#pragma unroll
        for (int k = 0; k < kAttnMaxChunks / 64; ++k) {
            const int c = tid + 64 * k;
            const float mc = c < C ? wc[c] : -__builtin_inff();
            wv[k] = mc == -__builtin_inff() ? 0.0f : lr_exp(mc - M);  // a chunk this token sees nothing of: 0
            if (c < C) den += lc[c] * wv[k];
        }
        den = wave_sum_dpp(den);
#pragma unroll
        for (int k = 0; k < kAttnMaxChunks / 64; ++k) {
            const int c = tid + 64 * k;
            if (c < C) wc[c] = wv[k];
        }
        if (tid == 0) den_s = den;
    }
    __syncthreads();
    float acc[8] = {0.0f, 0.0f, 0.0f, 0.0f, 0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
    for (int k = 0; k < kBatch; ++k) {
        const int c = q + kGroups * k;
        const float wk = c < C ? wc[c] : 0.0f;
        const uint32_t u[4] = {v[k].x, v[k].y, v[k].z, v[k].w};
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            acc[2 * i] += bf2f(u[i] & 0xffffu) * wk;
            acc[2 * i + 1] += bf2f(u[i] >> 16) * wk;
        }
    }
    *reinterpret_cast<float4*>(&part[q][d0]) = make_float4(acc[0], acc[1], acc[2], acc[3]);
    *reinterpret_cast<float4*>(&part[q][d0 + 4]) = make_float4(acc[4], acc[5], acc[6], acc[7]);
    __syncthreads();
    // groups s kGroups / kSets .. into part[s] (each thread one dim of one set)
    {
        const int d = tid % kDims;
        const int s0 = tid / kDims;
        constexpr int kPer = kGroups / kSets;
        float num = part[kPer * s0][d];
#pragma unroll
        for (int k = 1; k < kPer; ++k) num += part[kPer * s0 + k][d];
        __syncthreads();
        part[s0][d] = num;
    }
    __syncthreads();
    if (tid < kDims) {
        const int d = tid;
        float num = part[0][d];
#pragma unroll
        for (int k = 1; k < kSets; ++k) num += part[k][d];
        const float o = rbf(num / den_s);
        const float gate = bf2f((gi & 1) ? gword >> 16 : gword & 0xffffu);
        const float sg = rbf(1.0f / (1.0f + lr_exp(-gate)));
        S.out[d] = attn_length_bad(a) ? static_cast<uint16_t>(0x7fc0u) : static_cast<uint16_t>(f2bf(o * sg));
    }
    __syncthreads();
    // the row as 4-byte words
    if (tid < kDims / 2) {
        const uint32_t w = static_cast<uint32_t>(S.out[2 * tid]) | (static_cast<uint32_t>(S.out[2 * tid + 1]) << 16);
        uint16_t* dst = a.att + static_cast<int64_t>(t) * kAtO + h * kAtD + dbase + 2 * tid;
        *reinterpret_cast<uint32_t*>(dst) = w;
    }
}

constexpr int kAtCombineThreads = 256;

// kSplit workgroups per (token, head): 8 up to 4 tokens, 4 above.
template <int kSplit>
__global__ __launch_bounds__(kAtCombineThreads) void at_combine(AttnArgs a) {
    __shared__ CombineLdsOf<kAtCombineThreads, kSplit> S;
    AT_TL(16384, 4, 0);
    const int row = blockIdx.x / kSplit;
    combine_row<kAtCombineThreads, kSplit>(a, S, row / kAtHeads, row % kAtHeads, blockIdx.x % kSplit);
    AT_TL(16384, 4, 1);
}

}  // namespace

void attn_geometry(AttnArgs& a, int tokens, int span) {
    // Chunks of `per` whole 32-position sub-blocks: one per chunk up to 4
    // tokens (the partials of 8 T rows per chunk stay small), two above
    // unless chunks of one make at most 128 workgroups (short caches: then
    // the extra workgroups gain more than the extra partials cost, 0.6-1.5
    // us a step at 300 and 1000 positions; at 1900 positions and 12-16
    // tokens, 240 workgroups of one sub-block lost 0.5-0.7 us),
    // more only when the chunks would exceed the cap: 128 per head up to 8
    // tokens, 64 above (two workgroups per chunk), so that the launch is at
    // most 256 workgroups, one per CU.  (Up to 4 tokens a cap of 256, two
    // 32-row workgroups on some or all CUs, was slower at every length past
    // 128 sub-blocks: 0.8 us at one token and 4096 positions, 5.2 us at four
    // tokens and 8100.)
    // The last chunk takes what the cap leaves (at most 2 per): 4096 cached
    // positions and 16 new ones make 64 chunks of 2 sub-blocks and one of 3,
    // not 43 of 3.  A chunk's bounds depend on the span only through `per`,
    // so a call sized for a cache's capacity and one sized for its length
    // split the valid positions alike while `per` is the same.
    const int S = (span + kAtSub - 1) / kAtSub;
    const int halves = tokens > 8 ? 2 : 1;
    const int floor_per = tokens <= 4 || kAtKv * halves * S <= 128 ? 1 : 2;
    const int cap = kAttnMaxChunks / halves;
    const int per = max(floor_per, (S + cap) / (cap + 1));
    a.sub_blocks = S;
    a.per = per;
    a.chunks = min((S + per - 1) / per, cap);
    a.halves = halves;
    a.t_half = (tokens + 1) / 2;
}

size_t attn_workspace_bytes(int tokens) {
    return carve_attn(nullptr, tokens).bytes;
}

AttnWorkspace carve_attn(void* base, int tokens) {
    AttnWorkspace w{};
    uint8_t* p = static_cast<uint8_t*>(base);
    size_t off = 0;
    auto take = [&](size_t bytes) {
        const size_t at = off;
        off += (bytes + 255) & ~static_cast<size_t>(255);
        return p + at;
    };
    const size_t T = static_cast<size_t>(tokens);
    w.proj = reinterpret_cast<uint16_t*>(take(T * kAtProj * 2));
    w.att = reinterpret_cast<uint16_t*>(take(T * kAtO * 2));
    const size_t rows = static_cast<size_t>(kAtGroup) * T;
    w.part_o = reinterpret_cast<uint16_t*>(take(static_cast<size_t>(kAtKv) * kAttnMaxChunks * rows * kAtD * 2));
    w.part_ml = reinterpret_cast<float*>(take(static_cast<size_t>(kAtKv) * kAttnMaxChunks * rows * 2 * 4));
    w.bytes = off;
    return w;
}

hipError_t launch_attn_decode(AttnArgs a, const uint16_t* x, const uint16_t* w_q, const uint16_t* w_k,
                              const uint16_t* w_v, const uint16_t* w_o, uint16_t* out, const AttnGlue& fused,
                              hipStream_t stream) {
    static_assert(kAtProj % 36 == 0 && kAtQg % 4 == 0 && kAtVRow % 4 == 0 && kHidden % 8 == 0, "projection grids");
    const int T = a.tokens;
    const StageEvents ev = timing_events(kStageAttention);
    // q/gate, k and v rows: the three weight matrices in one grid
    const ProjectGlue in_glue{fused.in_norm, fused.in_eps, fused.norm_out, nullptr, nullptr};
    const ProjectGlue out_glue{nullptr, 0.0f, nullptr, x, fused.sum_out};
    if (fused.in_norm != nullptr) {
        LRMOE_LAUNCH((at_project<36, kHidden, true, false>), dim3(kAtProj / 36), dim3(kAtThreads), 0, stream, ev.start,
                     nullptr, w_q, w_k, w_v, kAtKRow, kAtVRow, x, T, a.proj, kAtProj, in_glue);
    } else {
        LRMOE_LAUNCH((at_project<36, kHidden>), dim3(kAtProj / 36), dim3(kAtThreads), 0, stream, ev.start, nullptr,
                     w_q, w_k, w_v, kAtKRow, kAtVRow, x, T, a.proj, kAtProj, in_glue);
    }
    if (T <= 4) {
        LRMOE_LAUNCH((at_attend<32, 4, false>), dim3(kAtKv * a.chunks), dim3(kAtThreads), 0, stream, nullptr, nullptr,
                     a);
    } else if (a.halves == 1) {
        LRMOE_LAUNCH((at_attend<64, 8, false>), dim3(kAtKv * a.chunks), dim3(kAtThreads), 0, stream, nullptr, nullptr,
                     a);
    } else {
        LRMOE_LAUNCH((at_attend<64, kAttnMaxTokens, true>), dim3((2 * kAtKv * a.chunks + 15) / 16 * 16),
                     dim3(kAtThreads), 0, stream, nullptr, nullptr, a);
    }
    if (T <= 4) {
        LRMOE_LAUNCH(at_combine<8>, dim3(T * kAtHeads * 8), dim3(kAtCombineThreads), 0, stream, nullptr, nullptr, a);
    } else {
        LRMOE_LAUNCH(at_combine<4>, dim3(T * kAtHeads * 4), dim3(kAtCombineThreads), 0, stream, nullptr, nullptr, a);
    }
    if (fused.sum_out != nullptr) {
        LRMOE_LAUNCH((at_project<8, kAtO, false, true>), dim3(kHidden / 8), dim3(kAtThreads), 0, stream, nullptr,
                     ev.stop, w_o, w_o, w_o, kHidden, kHidden, a.att, T, out, kHidden, out_glue);
    } else {
        LRMOE_LAUNCH((at_project<8, kAtO>), dim3(kHidden / 8), dim3(kAtThreads), 0, stream, nullptr, ev.stop, w_o, w_o,
                     w_o, kHidden, kHidden, a.att, T, out, kHidden, out_glue);
    }
    return hipGetLastError();
}

}  // namespace lrmoe
