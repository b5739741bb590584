// Gated DeltaNet decode on gfx950: the gated delta rule over a short block
// of tokens (edge35b/delta_decode.py:11-55, _delta and _run: dn_rule), and
// the whole cached-decode step of the 35B model's linear-attention mixer
// ([HF] Qwen3_5MoeGatedDeltaNet.forward 430-543: 16 key heads and 32 value
// heads of width 128, conv kernel 4) as one persistent launch (dn_mixer):
// in_proj with the causal conv + SiLU, the conv-state update, beta and
// G = exp(g); the delta rule; the gated RMSNorm; out_proj.
//
// Rounding points follow the Transformers forward in bf16: projections and
// conv outputs rounded to bf16, SiLU of the rounded conv output rounded,
// beta = bf16(sigmoid(b)), g in fp32, l2norm with every step rounded, the
// state rounded to its dtype after every token, the output rounded to bf16,
// then n = bf16(o rsqrt(mean o^2 + eps)), bf16(bf16(w n) silu(z)).  The
// recurrence multiplies and adds separately (no fused multiply-add), as the
// reference's kernel does (enable_fp_fusion=False).
#include "lrmoe_device.h"
#include "lrmoe_internal.h"

// Timeline build (-DLRMOE_TIMELINE, liblrmoe_timeline.so; the product
// library has none of it): thread 0 of every dn_mixer workgroup stamps the
// 100 MHz wall clock at its phases into the buffer given by
// lrmoe_mixer_timeline_set (16 words per workgroup): 0 entry, 1 unit 0
// multiplied, 2 unit 0's epilogue done, 3 unit 1 and beta/G done, 4 phase A
// end, 5 first barrier passed, 11 the rule's inputs staged, 13 q and k
// l2norm'd, 14 wave 0's token loop done, 6 rule done, 7 z unit done and
// counted in, 8 gated norm done (word 12: 1 on the head's last workgroup),
// 9 second barrier passed, 10 out_proj done.
#ifdef LRMOE_TIMELINE
__device__ unsigned long long* g_mixer_timeline;
extern "C" int lrmoe_mixer_timeline_set(void* p) {
    return static_cast<int>(hipMemcpyToSymbol(HIP_SYMBOL(g_mixer_timeline), &p, sizeof(p)));
}
#define MX_WORD(k, v)                                                                        \
    do {                                                                                     \
        if (threadIdx.x == 0 && g_mixer_timeline != nullptr) g_mixer_timeline[blockIdx.x * 16 + (k)] = (v); \
    } while (0)
#else
#define MX_WORD(k, v)
#endif
#define MX_TL(k) MX_WORD(k, wall_clock64())

namespace lrmoe {
namespace {

constexpr int kDnKeyHeads = 16;
constexpr int kDnValueHeads = 32;
constexpr int kDnWidth = 128;
constexpr int kDnKey = kDnKeyHeads * kDnWidth;      // 2048
constexpr int kDnValue = kDnValueHeads * kDnWidth;  // 4096
constexpr int kDnConv = 2 * kDnKey + kDnValue;      // 8192
constexpr int kDnTaps = 4;
constexpr int kDnZRow = kDnConv;                    // first in_proj_z row
constexpr int kDnBRow = kDnZRow + kDnValue;         // first in_proj_b row

__device__ __forceinline__ float silu(float x) { return x / (1.0f + lr_exp(-x)); }

__device__ __forceinline__ float softplus(float x) { return x > 20.0f ? x : log1pf(lr_exp(x)); }

// Sum over the 16 lanes of a DPP row, the same total in every lane: xor
// butterflies 1 and 2 (quad permutes), then the half-row and row mirrors,
// which pair each lane with one of the other quad (half-row) whose lanes
// already hold equal partial sums.
__device__ __forceinline__ float row_sum16(float v) {
    v = v + __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), 0xB1, 0xf, 0xf, false));   // quad_perm [1,0,3,2]
    v = v + __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), 0x4E, 0xf, 0xf, false));   // quad_perm [2,3,0,1]
    v = v + __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), 0x141, 0xf, 0xf, false));  // row_half_mirror
    v = v + __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), 0x140, 0xf, 0xf, false));  // row_mirror
    return v;
}

template <bool BF16, int C>
__device__ __forceinline__ void load_state(const void* base, int64_t idx, float* s) {
    if constexpr (BF16) {
        const uint16_t* p = static_cast<const uint16_t*>(base) + idx;
#pragma unroll
        for (int c = 0; c < C; ++c) s[c] = bf2f(p[c]);
    } else {
        const float* p = static_cast<const float*>(base) + idx;
#pragma unroll
        for (int c = 0; c < C; ++c) s[c] = p[c];
    }
}

template <bool BF16, int C>
__device__ __forceinline__ void store_state(void* base, int64_t idx, const float* s) {
    if constexpr (BF16) {
        uint16_t* p = static_cast<uint16_t*>(base) + idx;
#pragma unroll
        for (int c = 0; c < C; ++c) p[c] = static_cast<uint16_t>(f2bf(s[c]));
    } else {
        float* p = static_cast<float*>(base) + idx;
#pragma unroll
        for (int c = 0; c < C; ++c) p[c] = s[c];
    }
}

constexpr int kRuleStage = 16;  // tokens staged in LDS at a time

// The gated delta rule for value head blockIdx.x, state columns
// 4C blockIdx.y .. 4C blockIdx.y + 4C - 1, one wave.  Lane (row group
// rg = lane % 16, column slot cq = lane / 16) holds state rows
// rg R .. rg R + R - 1 (R = D / 16) of columns 4C blockIdx.y + C cq .. +C-1
// in registers for all T tokens.  Per block of up to 16 tokens, q and k
// (l2norm'd, q scaled by D^-1/2), the wave's v columns, G and beta are
// staged in LDS first, so the serial token loop reads only LDS.  Per token:
// state *= G; mem = state^T k; delta = (v - mem) beta; state += k delta^T;
// out = state^T q; the state rounded to its dtype (a no-op for fp32).
// Column sums over the D rows: in-lane, then across the row group's DPP row
// (row_sum16).  C = 1 spreads the 32 heads of the 35B mixer over 1024 waves,
// so that a token's serial step is short.
template <int D, bool BF16, int C>
__global__ __launch_bounds__(64) void dn_rule(DnRuleArgs a) {
    constexpr int R = D / 16;
    constexpr int kCols = 4 * C;
    __shared__ float qs[kRuleStage][D];
    __shared__ float ks[kRuleStage][D];
    __shared__ float vs[kRuleStage][kCols];
    __shared__ float gs[kRuleStage];
    __shared__ float bs[kRuleStage];

    const int lane = threadIdx.x;
    const int rg = lane & 15;
    const int cq = lane >> 4;
    const int h = blockIdx.x;
    const int H = a.heads;
    const int E = a.width;
    const int T = a.tokens;
    const int col0 = blockIdx.y * kCols;
    const int col = col0 + C * cq;
    const int64_t slab = static_cast<int64_t>(h) * D * E;
    const int kh = h >> a.kv_shift;

    float S[R][C];
#pragma unroll
    for (int i = 0; i < R; ++i) load_state<BF16, C>(a.initial, slab + static_cast<int64_t>(rg * R + i) * E + col, S[i]);

    const float scale = 1.0f / __builtin_sqrtf(static_cast<float>(D));
    for (int t0 = 0; t0 < T; t0 += kRuleStage) {
        const int n = min(kRuleStage, T - t0);
        if (t0 > 0) __syncthreads();  // the previous block's tokens have been read
        for (int i = lane; i < n * (D / 8); i += 64) {
            const int tt = i / (D / 8);
            const int ch = i % (D / 8);
            const int64_t src = static_cast<int64_t>(t0 + tt) * a.qk_stride + static_cast<int64_t>(kh) * D + ch * 8;
            unpack8(ldg16(a.q + src), &qs[tt][ch * 8]);
            unpack8(ldg16(a.k + src), &ks[tt][ch * 8]);
        }
        for (int i = lane; i < n * kCols; i += 64) {
            const int tt = i / kCols;
            vs[tt][i % kCols] = bf2f(ldg_u16(a.v + static_cast<int64_t>(t0 + tt) * a.v_stride +
                                             static_cast<int64_t>(h) * E + col0 + i % kCols));
        }
        if (lane < n) {
            gs[lane] = a.G[(t0 + lane) * H + h];
            bs[lane] = bf2f(a.beta[(t0 + lane) * H + h]);
        }
        __syncthreads();
        // l2norm of q and k (torch on bf16: every step rounded), q scaled;
        // token tt on DPP row tt % 4, R values per lane
        for (int tt = cq; tt < n; tt += 4) {
            float* qrow = &qs[tt][rg * R];
            float* krow = &ks[tt][rg * R];
            if (a.normalize) {
                float sq = 0.0f, sk = 0.0f;
#pragma unroll
                for (int i = 0; i < R; ++i) {
                    sq += rbf(qrow[i] * qrow[i]);
                    sk += rbf(krow[i] * krow[i]);
                }
                sq = row_sum16(sq);
                sk = row_sum16(sk);
                const float iq = rbf(1.0f / __builtin_sqrtf(rbf(rbf(sq) + 1e-6f)));
                const float ik = rbf(1.0f / __builtin_sqrtf(rbf(rbf(sk) + 1e-6f)));
#pragma unroll
                for (int i = 0; i < R; ++i) {
                    qrow[i] = rbf(qrow[i] * iq) * scale;
                    krow[i] = rbf(krow[i] * ik);
                }
            } else {
#pragma unroll
                for (int i = 0; i < R; ++i) qrow[i] = qrow[i] * scale;
            }
        }
        __syncthreads();

        for (int tt = 0; tt < n; ++tt) {
            const int t = t0 + tt;
            float q[R], k[R], v[C];
#pragma unroll
            for (int i = 0; i < R; ++i) {
                q[i] = qs[tt][rg * R + i];
                k[i] = ks[tt][rg * R + i];
            }
#pragma unroll
            for (int c = 0; c < C; ++c) v[c] = vs[tt][C * cq + c];
            const float G = gs[tt];
            const float beta = bs[tt];

            float mem[C];
#pragma unroll
            for (int c = 0; c < C; ++c) mem[c] = 0.0f;
#pragma unroll
            for (int i = 0; i < R; ++i)
#pragma unroll
                for (int c = 0; c < C; ++c) {
                    S[i][c] = S[i][c] * G;
                    mem[c] = mem[c] + S[i][c] * k[i];
                }
            float delta[C], o[C];
#pragma unroll
            for (int c = 0; c < C; ++c) {
                delta[c] = (v[c] - row_sum16(mem[c])) * beta;
                o[c] = 0.0f;
            }
#pragma unroll
            for (int i = 0; i < R; ++i)
#pragma unroll
                for (int c = 0; c < C; ++c) {
                    S[i][c] = S[i][c] + k[i] * delta[c];
                    o[c] = o[c] + S[i][c] * q[i];
                }
#pragma unroll
            for (int c = 0; c < C; ++c) o[c] = row_sum16(o[c]);
            if (rg == 0) {
                uint16_t* dst = a.out + (static_cast<int64_t>(t) * H + h) * E + col;
#pragma unroll
                for (int c = 0; c < C; ++c) dst[c] = static_cast<uint16_t>(f2bf(o[c]));
            }
            if constexpr (BF16) {
#pragma unroll
                for (int i = 0; i < R; ++i)
#pragma unroll
                    for (int c = 0; c < C; ++c) S[i][c] = rbf(S[i][c]);
            }
            if (a.record) {
                const int64_t rec = static_cast<int64_t>(t) * H * D * E + slab;
#pragma unroll
                for (int i = 0; i < R; ++i)
                    store_state<BF16, C>(a.record, rec + static_cast<int64_t>(rg * R + i) * E + col, S[i]);
            }
        }
    }
    if (a.final_state) {
#pragma unroll
        for (int i = 0; i < R; ++i) store_state<BF16, C>(a.final_state, slab + static_cast<int64_t>(rg * R + i) * E + col, S[i]);
    }
}

template <int D>
hipError_t launch_rule_d(const DnRuleArgs& a, bool bf16, hipStream_t stream) {
    const StageEvents ev = timing_events(kStageDeltaRule);
    const dim3 grid(a.heads, a.width / 4);
    if (bf16) {
        LRMOE_LAUNCH((dn_rule<D, true, 1>), grid, dim3(64), 0, stream, ev.start, ev.stop, a);
    } else {
        LRMOE_LAUNCH((dn_rule<D, false, 1>), grid, dim3(64), 0, stream, ev.start, ev.stop, a);
    }
    return hipGetLastError();
}

// ---- the mixer step in one persistent launch (dn_mixer) ---------------------
//
// 256 workgroups of 8 waves, one per CU, all resident (the workgroups wait
// for each other's flags).  The rule waits only for the rows it reads (q, k
// and v); the rest of the workgroup's HBM stream (in_proj's z unit and
// out_proj's rows) is requested after the rule's inputs and lands while the
// rule runs:
//
//   start    A_log and dt_bias, the head's counter, the rule's state slab,
//            the token rows, then in_proj units b and b + 256 (q, k and v
//            rows: 768 units of 16 rows in all, 128 KiB per CU), every load
//            unconditional (clamped dummy addresses where a lane needs
//            none) so that the compiler's in-order waits cover only what
//            is consumed; each load instruction reads 1 KiB of one row
//            (5.4 TB/s on this part, against 3.9 TB/s when an instruction
//            gathers the MFMA layout's 64 bytes from each of 16 rows);
//   phase A  a unit passes through LDS into the MFMA layout, wave w
//            multiplying k in [256 w, 256 w + 256); per unit the causal
//            conv + SiLU and the conv-state update, written with
//            agent-scope stores; into unit 0's registers, head b / 8's
//            in_proj_b and in_proj_a rows (its beta and G go to LDS: no
//            other workgroup needs them); then the workgroup's "staged"
//            flag;
//   wait     for the staged flags of the 16 workgroups whose unit 0 holds
//            key head (b / 16)'s q and k rows (its own unit 1 holds its v
//            rows);
//   phase B  the rule's inputs; the rule for (head b / 8, columns
//            16 (b % 8) .. +15): q and k staged and l2norm'd by the
//            workgroup, waves 0-3 four columns each (dn_rule's
//            arithmetic); outputs through LDS to agent-scope rows; then
//            unit b + 512 (z) and out_proj rows 8b .. 8b + 7 (A operands of
//            phase D) requested, and the z unit; the last of a head's 8
//            workgroups to count itself in (a monotonic counter, 8 per
//            call) forms the head's gated RMSNorm (phase C: o, z and the
//            norm weights in one round trip) and sets the head's "normed"
//            flag;
//   wait     per wave, for the normed flags of the 4 heads whose rows it
//            multiplies (wave w: heads 4w .. 4w + 3);
//   phase D  out_proj rows 8b .. 8b + 7 from the registers and the normed
//            rows, each wave's requested as soon as its heads are normed.
//
// Flags hold the number of the last call that set them (the head counter at
// the start, divided by 8, plus 1), so nothing is ever reset; each sits in a
// 128-byte line of its own and takes plain agent-scope stores, no atomics.
// (A grid barrier on one counter serialises 256 atomics: ~4 us back to
// back; the flags let a workgroup wait only for its producers.)
// Waits are bounded (50 ms); on expiry the launch still ends and sets
// LRMOE_STATUS_TIMEOUT in the status word.

constexpr int kMixGrid = 256;
constexpr int kMixWaves = 8;
constexpr int kMixThreads = 64 * kMixWaves;
constexpr int kMixRows = 8;                                        // out_proj rows per workgroup
constexpr int kMixInRows = 16;                                     // rows per in_proj unit
constexpr int kMixInUnits = kDnBRow / kMixInRows;                  // 768: qkv and z rows
constexpr int kMixUnitsPerWg = kMixInUnits / 256;                   // 3, all in flight at once
constexpr int kMixRuleWaves = 4;
constexpr int kMixHeadGroups = kDnWidth / (4 * kMixRuleWaves);    // 8 workgroups per head
constexpr uint64_t kMixSpinTicks = 5000000;                        // 50 ms of the 100 MHz wall clock
static_assert(kMixGrid == kDnValueHeads * kMixHeadGroups, "one rule unit per workgroup");
static_assert(kMixGrid == kHidden / kMixRows, "one out_proj unit per workgroup");
static_assert(kMixUnitsPerWg * kMixGrid == kMixInUnits && kMixUnitsPerWg == 3, "three in_proj units each");

__device__ __forceinline__ const uint16_t* mix_row_ptr(const DnProjectArgs& a, int n) {
    return n < kDnZRow ? a.w_qkv + static_cast<int64_t>(n) * kHidden : a.w_z + static_cast<int64_t>(n - kDnZRow) * kHidden;
}

template <bool BF16>
__device__ __forceinline__ float state_at(const void* base, int64_t i) {
    if constexpr (BF16) return bf2f(static_cast<const uint16_t*>(base)[i]);
    else return static_cast<const float*>(base)[i];
}

template <bool BF16>
__device__ __forceinline__ void state_put(void* base, int64_t i, float v) {
    if constexpr (BF16) static_cast<uint16_t*>(base)[i] = static_cast<uint16_t>(f2bf(v));
    else static_cast<float*>(base)[i] = v;
}

template <bool BF16, bool kNorm>
__global__ __launch_bounds__(kMixThreads, 1) void dn_mixer(DnMixerArgs m) {
    const DnProjectArgs& a = m.p;
    __shared__ __attribute__((aligned(16))) uint16_t tile[kMixInRows][kHidden + 8];  // one in_proj unit, row-major
    __shared__ float red[kMixWaves][16][17];
    __shared__ float red_ba[kMixWaves][2][16];
    __shared__ uint16_t seq[kMixInRows][kDnTaps + 16];
    __shared__ uint2 conv_lds[2][2][kMixInRows];  // [unit parity] per unit row: conv weights, cached conv inputs
    __shared__ float gate_lds[2][kDnValueHeads];  // A_log, dt_bias
    __shared__ float qs[kRuleStage][kDnWidth];
    __shared__ float ks[kRuleStage][kDnWidth];
    __shared__ float vs[kMixRuleWaves][kRuleStage][4];
    __shared__ float gs[kRuleStage];
    __shared__ float bs[kRuleStage];
    __shared__ uint16_t os[kRuleStage][4 * kMixRuleWaves];
    __shared__ unsigned long long base_s;
    __shared__ int timeout_s;
    __shared__ int last_s;
    __shared__ float rscale[kDeltaMaxTokens];  // the fused input norm's 1 / rms per token row

    const int tid = threadIdx.x;
    const int lane = tid & 63;
    const int wave = tid >> 6;
    const int t = lane & 15;
    const int g = lane >> 4;
    const int T = a.tokens;
    const int b = blockIdx.x;
    const bool live = t < kMixRows;  // this lane's MFMA row holds a weight row
    MX_TL(0);

    // conv weights and cached inputs of a unit's rows (threads 0-31 of a
    // unit below the z rows keep them; every other thread loads conv row
    // tid % 16 and drops it, so that no branch makes the compiler wait for
    // the load before the units behind it are issued)
    auto load_conv = [&](int v) -> uint2 {
        const int n0 = kMixInRows * v;
        const bool kept = tid < 2 * kMixInRows && n0 < kDnZRow;
        return *reinterpret_cast<const uint2*>(((tid & 16) ? a.conv_state : a.conv_w) + ((kept ? n0 : 0) + (tid & 15)) * kDnTaps);
    };
    // A unit's rows as the memory system streams them best: each load
    // instruction of a wave reads 1 KiB of one row (wave w: rows 2w, 2w + 1;
    // load i: row 2w + i / 4, k from 512 (i % 4) + 8 lane).
    auto load_unit = [&](uint4 (&w)[8], uint2& cv, int v) {
        const uint16_t* row0 = mix_row_ptr(a, kMixInRows * v + 2 * wave) + 8 * lane;
#pragma unroll
        for (int i = 0; i < 8; ++i) w[i] = ldg16(row0 + (i >> 2) * kHidden + 512 * (i & 3));
        cv = load_conv(v);
    };
    // The small inputs first -- A_log and dt_bias, the head's counter, the
    // rule's state slab, the token rows -- then in_proj units 0 (q, k) and 1
    // (v).  The memory counter retires in order: waiting for a small input
    // then never waits for a unit, and unit 0 is multiplied as soon as it
    // arrives.  (Every thread issues every one of these loads, with valid
    // dummy addresses where it needs none, so that no branch blurs the
    // waits.)  Unit 2 (z, needed only by the gated norm) is requested behind
    // the rule's inputs, after the first barrier, which would otherwise wait
    // for it.
    const uint16_t gate_raw = static_cast<uint16_t>(ldg_u16(((tid >> 5) & 1 ? a.dt_bias : a.A_log) + (tid & 31)));
    // (this call's number: each call counts 8 workgroups in on every head's
    // counter, and none of this head's can count in 8 before this one has)
    const unsigned long long counted = ld_agent64(m.heads + kDeltaWsStride * (b / kMixHeadGroups));
    // the rule's state: head rh, column rc, rows 8 rg .. 8 rg + 7 (waves 0-3;
    // waves 4-7 load the same words as waves 0-3 and drop them)
    const int rg = lane & 15;
    const int cq = lane >> 4;
    const int rh = b / kMixHeadGroups;
    const int rc0 = 16 * (b % kMixHeadGroups);
    const int rc = rc0 + 4 * (wave % kMixRuleWaves) + cq;
    const int64_t slab = static_cast<int64_t>(rh) * kDnWidth * kDnWidth;
    float S[8];
#pragma unroll
    for (int i = 0; i < 8; ++i) S[i] = state_at<BF16>(m.state, slab + static_cast<int64_t>(8 * rg + i) * kDnWidth + rc);
    // token rows (columns t >= T load token 0: their results are dropped)
    uint4 xb[8];
    {
        const uint16_t* xrow = a.x + static_cast<int64_t>(t < T ? t : 0) * kHidden + 256 * wave + 8 * g;
#pragma unroll
        for (int s = 0; s < 2; ++s)
#pragma unroll
            for (int j = 0; j < 4; ++j) xb[4 * s + j] = ldg16(xrow + 128 * s + 32 * j);
    }
    // The fused input RMSNorm: wave w's rows w and w + 8 in the norm's
    // layout (lane l: elements 32 l ..), and the weights of the lane's xb
    // pieces (rows past T load row 0)
    [[maybe_unused]] uint4 nrow[2][4], wn[8];
    if constexpr (kNorm) {
#pragma unroll
        for (int h = 0; h < 2; ++h) {
            const int r = wave + 8 * h;
            const uint16_t* src = a.x + static_cast<int64_t>(r < T ? r : 0) * kHidden + 32 * lane;
#pragma unroll
            for (int i = 0; i < 4; ++i) nrow[h][i] = ldg16(src + 8 * i);
        }
        const uint16_t* wsrc = a.in_norm + 256 * wave + 8 * g;
#pragma unroll
        for (int i = 0; i < 8; ++i) wn[i] = ldg16(wsrc + 32 * i);
    }
    uint4 w0[8], w1[8], w2[8];
    uint2 c0, c1;
    const int v0 = b, v1 = b + kMixGrid, v2 = b + 2 * kMixGrid;
    load_unit(w0, c0, v0);
    // Unit 1 is requested once unit 0's rows have landed: with no unit 1
    // in the memory system, every CU's unit 0 arrives ~0.9 us earlier and is
    // multiplied while unit 1 streams (requesting it when half of unit 0
    // had landed gained ~0.3 us).  (s_waitcnt vmcnt(1): unit 0's conv word
    // may still be in flight.)
    __builtin_amdgcn_s_waitcnt((1 & 15) | (7 << 4) | (15 << 8));
    load_unit(w1, c1, v1);
    if (tid == 0) {
        base_s = counted / kMixHeadGroups + 1;
        timeout_s = 0;
    }
    if (tid < 2 * kDnValueHeads) gate_lds[tid >> 5][tid & 31] = bf2f(gate_raw);
    // Take the state slab here, behind only the gate rows: its first use is
    // in the rule's token loop, where the compiler would otherwise wait for
    // every load in flight (the z unit and the out_proj rows) before the loop.
    asm volatile("" ::"v"(S[0]), "v"(S[1]), "v"(S[2]), "v"(S[3]), "v"(S[4]), "v"(S[5]), "v"(S[6]), "v"(S[7]));

    // The fused input RMSNorm (the decoder layer's input_layernorm): each
    // wave takes rows w and w + 8 in the norm's own layout and order, then
    // every lane scales its token-row pieces in place, so the operands equal
    // a separate norm's rows bit for bit; workgroup 0 stores them when asked.
    if constexpr (kNorm) {
#pragma unroll
        for (int h = 0; h < 2; ++h) {
            const float r = row_rms_scale(nrow[h], a.in_eps);
            if (lane == 0) rscale[wave + 8 * h] = r;
        }
        __syncthreads();
        const float r = rscale[t < T ? t : 0];
#pragma unroll
        for (int i = 0; i < 8; ++i) xb[i] = rms_apply8(xb[i], wn[i], r);
        if (b == 0 && a.norm_out != nullptr && t < T) {
#pragma unroll
            for (int i = 0; i < 8; ++i)
                *reinterpret_cast<uint4*>(a.norm_out + static_cast<int64_t>(t) * kHidden + 256 * wave + 32 * i + 8 * g) = xb[i];
        }
    }

    // ---- phase A: in_proj (wave w multiplies k in [256 w, 256 w + 256)) ----
    // MFMA A rows from row0 (every lane loads: an output row depends on its
    // own A row only, so rows the caller drops may hold anything)
    auto load_rows = [&](uint4 (&w)[8], const uint16_t* row0) {
        const uint16_t* wrow = row0 + 256 * wave + 8 * g;
#pragma unroll
        for (int s = 0; s < 2; ++s)
#pragma unroll
            for (int j = 0; j < 4; ++j) w[4 * s + j] = ldg16(wrow + 128 * s + 32 * j);
    };
    // The unit's rows through LDS into the MFMA layout, its partial tile
    // into red (rows 4 g + i, token t).  The caller's next barrier (the
    // epilogue's first) ends the reads of `tile`.
    auto unit_mfma = [&](const uint4 (&w)[8], uint2 cv, int v, int slot) {
#pragma unroll
        for (int i = 0; i < 8; ++i) *reinterpret_cast<uint4*>(&tile[2 * wave + (i >> 2)][512 * (i & 3) + 8 * lane]) = w[i];
        __syncthreads();
        f32x4 acc = {0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
        for (int s = 0; s < 2; ++s)
#pragma unroll
            for (int j = 0; j < 4; ++j)
                acc = mfma16x16x32(*reinterpret_cast<const uint4*>(&tile[t][256 * wave + 128 * s + 32 * j + 8 * g]),
                                   xb[4 * s + j], acc);
#pragma unroll
        for (int i = 0; i < 4; ++i) red[wave][4 * g + i][t] = acc[i];
        if (tid < 2 * kMixInRows && kMixInRows * v < kDnZRow) conv_lds[slot][tid >> 4][tid & 15] = cv;
    };
    auto unit_epilogue = [&](int v, int slot) {
        const int n0 = kMixInRows * v;
        __syncthreads();
        if (tid < 16 * kMixInRows) {
            const int row = tid >> 4;
            const int tt = tid & 15;
            float p = 0.0f;
#pragma unroll
            for (int ww = 0; ww < kMixWaves; ++ww) p += red[ww][row][tt];
            seq[row][kDnTaps + tt] = static_cast<uint16_t>(f2bf(p));
            if (n0 < kDnZRow && tt < kDnTaps) {
                const uint2 old = conv_lds[slot][1][row];
                seq[row][tt] = static_cast<uint16_t>(((tt < 2 ? old.x : old.y) >> (16 * (tt & 1))) & 0xffffu);
            }
        }
        __syncthreads();
        // waves 0-1: rows in pairs (one 4-byte store per token and pair).
        // The next unit writes red and seq only after its own first barrier,
        // which these waves reach after this, and the other conv_lds slot.
        if (tid < 8 * 16) {
            const int rp = tid >> 4;
            const int tt = tid & 15;
            if (tt < T) {
                if (n0 < kDnZRow) {
                    uint32_t pair = 0;
#pragma unroll
                    for (int r2 = 0; r2 < 2; ++r2) {
                        const int rr = 2 * rp + r2;
                        const uint2 cw = conv_lds[slot][0][rr];
                        const float wv[kDnTaps] = {lo_bf(cw.x), hi_bf(cw.x), lo_bf(cw.y), hi_bf(cw.y)};
                        float c = 0.0f;
#pragma unroll
                        for (int j = 0; j < kDnTaps; ++j) c = __builtin_fmaf(wv[j], bf2f(seq[rr][tt + 1 + j]), c);
                        pair |= f2bf(silu(rbf(c))) << (16 * r2);
                        if (a.conv_record) {
                            uint16_t* rec = a.conv_record + (static_cast<int64_t>(tt) * kDnConv + n0 + rr) * kDnTaps;
#pragma unroll
                            for (int j = 0; j < kDnTaps; ++j) rec[j] = seq[rr][tt + 1 + j];
                        }
                    }
                    st_agent32(a.act + static_cast<int64_t>(tt) * kDnConv + n0 + 2 * rp, pair);
                } else {
                    st_agent32(a.z + static_cast<int64_t>(tt) * kDnValue + (n0 - kDnZRow) + 2 * rp,
                               static_cast<uint32_t>(seq[2 * rp][kDnTaps + tt]) |
                                   (static_cast<uint32_t>(seq[2 * rp + 1][kDnTaps + tt]) << 16));
                }
            }
        }
        if (n0 < kDnZRow && tid >= 128 && tid < 128 + kMixInRows * kDnTaps) {
            const int rr = (tid - 128) >> 2;
            const int j = tid & 3;
            a.conv_state[(n0 + rr) * kDnTaps + j] = seq[rr][T + j];
        }
    };
    uint4 wo[16];  // out_proj rows 8b + t (t < 8), k in [512 wave, 512 wave + 512): phase D's A operands
    {
        unit_mfma(w0, c0, v0, 0);
        // head rh's b row (MFMA row 0) and a row (rows 1-15; only rows 0 and
        // 1 are kept), into w0's registers
        load_rows(w0, (t == 0 ? a.w_b : a.w_a) + static_cast<int64_t>(rh) * kHidden);
        MX_TL(1);
        unit_epilogue(v0, 0);
        MX_TL(2);
        unit_mfma(w1, c1, v1, 1);
        unit_epilogue(v1, 1);
        MX_TL(3);
        {
            // beta and G of head rh for every token, from its b and a rows
            f32x4 acc = {0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
            for (int i = 0; i < 8; ++i) acc = mfma16x16x32(w0[i], xb[i], acc);
            if (g == 0) {
                red_ba[wave][0][t] = acc[0];
                red_ba[wave][1][t] = acc[1];
            }
            __syncthreads();
            if (tid < 2 * 16) {
                const int row = tid >> 4;  // 0: b, 1: a
                const int tt = tid & 15;
                float p = 0.0f;
#pragma unroll
                for (int ww = 0; ww < kMixWaves; ++ww) p += red_ba[ww][row][tt];
                const float pb = rbf(p);
                if (row == 0) bs[tt] = rbf(1.0f / (1.0f + lr_exp(-pb)));
                else gs[tt] = lr_exp(-lr_exp(gate_lds[0][rh]) * softplus(pb + gate_lds[1][rh]));
            }
        }
    }

    // Publish this workgroup's flag (when `flag` is not null) once its
    // agent-scope stores are complete, then wait until the `count` flags
    // named by `flag_of(i)` hold this call's number.
    const unsigned long long call = base_s;
    auto publish_wait = [&](unsigned long long* flag, int count, auto flag_of) {
        __builtin_amdgcn_s_waitcnt(0);  // this wave's agent-scope stores are complete
        __syncthreads();
        if (tid == 0 && flag != nullptr) st_agent64(flag, call);
        if (tid < count) {
            const unsigned long long* f = flag_of(tid);
            const uint64_t start = wall_clock64();
            while (ld_agent64(f) < call) {
                if (wall_clock64() - start > kMixSpinTicks) {
                    timeout_s = 1;
                    break;
                }
                __builtin_amdgcn_s_sleep(1);
            }
        }
        __syncthreads();
    };
    const int kh = rh >> 1;  // value head h reads key head h / 2
    // The rule's inputs: its own v rows (unit 1) and key head kh's q and k
    // rows, units 8 kh .. 8 kh + 7 and 128 + 8 kh .. 128 + 8 kh + 7, which
    // are workgroups' unit 0 of the same numbers.  z (unit 2) is not needed
    // before the gated norm.
    MX_TL(4);
    publish_wait(m.staged + kDeltaWsStride * b, 16, [&](int i) {
        return m.staged + kDeltaWsStride * ((i < 8 ? 0 : 128) + 8 * kh + (i & 7));
    });
    MX_TL(5);

    // ---- phase B: the rule for head rh, columns rc0 .. rc0 + 15 ----
    {
        // The rule's inputs, loaded by every thread (clamped to token 0: no
        // branch around loads, so that the waits below cover only them).
        const bool is_qk = tid < 16 * T;
        const int tq = is_qk ? tid >> 4 : 0;
        const int ch = tid & 15;
        const uint32_t qoff = static_cast<uint32_t>((tq * kDnConv + kh * kDnWidth + ch * 8) * 2);
        const uint4 qraw = ld_agent16(a.act, qoff);
        const uint4 kraw = ld_agent16(a.act, qoff + kDnKey * 2);
        const int vi = tid - 256;
        const bool is_v = vi >= 0 && vi < kMixRuleWaves * T;
        const int vw = is_v ? vi & 3 : 0;
        const int vt = is_v ? vi >> 2 : 0;
        const uint64_t v4 = ld_agent64(a.act + static_cast<int64_t>(vt) * kDnConv + 2 * kDnKey + rh * kDnWidth + rc0 + 4 * vw);
        // (taken on every path: a wait inside only one branch would leave
        // the registers pending at the merge, and the compiler then waits
        // for every load in flight)
        asm volatile("" ::"v"(qraw.x), "v"(kraw.x), "v"(v4));
        if (is_qk) {
            unpack8(qraw, &qs[tq][ch * 8]);
            unpack8(kraw, &ks[tq][ch * 8]);
        }
        if (is_v) {
            const uint32_t lo = static_cast<uint32_t>(v4), hi = static_cast<uint32_t>(v4 >> 32);
            vs[vw][vt][0] = lo_bf(lo); vs[vw][vt][1] = hi_bf(lo); vs[vw][vt][2] = lo_bf(hi); vs[vw][vt][3] = hi_bf(hi);
        }
        __syncthreads();
        MX_TL(11);
        {
            const float scale = 1.0f / __builtin_sqrtf(static_cast<float>(kDnWidth));
            const int tt = tid >> 4;  // one DPP row per token
            if (tt < T) {
                float* qrow = &qs[tt][8 * rg];
                float* krow = &ks[tt][8 * rg];
                float sq = 0.0f, sk = 0.0f;
#pragma unroll
                for (int i = 0; i < 8; ++i) {
                    sq += rbf(qrow[i] * qrow[i]);
                    sk += rbf(krow[i] * krow[i]);
                }
                sq = row_sum16(sq);
                sk = row_sum16(sk);
                const float iq = rbf(1.0f / __builtin_sqrtf(rbf(rbf(sq) + 1e-6f)));
                const float ik = rbf(1.0f / __builtin_sqrtf(rbf(rbf(sk) + 1e-6f)));
#pragma unroll
                for (int i = 0; i < 8; ++i) {
                    qrow[i] = rbf(qrow[i] * iq) * scale;
                    krow[i] = rbf(krow[i] * ik);
                }
            }
        }
        __syncthreads();
        MX_TL(13);
        if (wave < kMixRuleWaves) {
            for (int tt = 0; tt < T; ++tt) {
                float q[8], k[8];
#pragma unroll
                for (int i = 0; i < 8; ++i) {
                    q[i] = qs[tt][8 * rg + i];
                    k[i] = ks[tt][8 * rg + i];
                }
                const float G = gs[tt];
                const float beta = bs[tt];
                float mem = 0.0f;
#pragma unroll
                for (int i = 0; i < 8; ++i) {
                    S[i] = S[i] * G;
                    mem = mem + S[i] * k[i];
                }
                const float delta = (vs[wave][tt][cq] - row_sum16(mem)) * beta;
                float o = 0.0f;
#pragma unroll
                for (int i = 0; i < 8; ++i) {
                    S[i] = S[i] + k[i] * delta;
                    o = o + S[i] * q[i];
                }
                o = row_sum16(o);
                if (rg == 0) os[tt][4 * wave + cq] = static_cast<uint16_t>(f2bf(o));
                if constexpr (BF16) {
#pragma unroll
                    for (int i = 0; i < 8; ++i) S[i] = rbf(S[i]);
                }
                if (m.state_record) {
                    const int64_t rec = static_cast<int64_t>(tt) * kDnValueHeads * kDnWidth * kDnWidth + slab;
#pragma unroll
                    for (int i = 0; i < 8; ++i) state_put<BF16>(m.state_record, rec + static_cast<int64_t>(8 * rg + i) * kDnWidth + rc, S[i]);
                }
            }
#pragma unroll
            for (int i = 0; i < 8; ++i) state_put<BF16>(m.state, slab + static_cast<int64_t>(8 * rg + i) * kDnWidth + rc, S[i]);
        }
        // Then in_proj unit 2 (z rows 16 b .. 16 b + 15) and out_proj rows
        // 8 b .. 8 b + 7 (phase D's A operands): waves 4-7 reach this point
        // as soon as the inputs are normed and stream their rows during the
        // token loop, the rule waves after it.  (Issued before the rule, the
        // 32 MiB of rows every CU requests held up the rule's own input loads
        // behind them for ~6 us.)
        {
            const uint16_t* row0 = mix_row_ptr(a, kMixInRows * v2 + 2 * wave) + 8 * lane;
#pragma unroll
            for (int i = 0; i < 8; ++i) w2[i] = ldg16(row0 + (i >> 2) * kHidden + 512 * (i & 3));
            // (lanes t >= 8 load row 8 b too: MFMA output rows 8-15, which
            // they feed, are dropped)
            const uint16_t* wrow = a.w_out + static_cast<int64_t>(kMixRows * b + (live ? t : 0)) * kDnValue + 512 * wave + 8 * g;
#pragma unroll
            for (int s2 = 0; s2 < 4; ++s2)
#pragma unroll
                for (int j = 0; j < 4; ++j) wo[4 * s2 + j] = ldg16(wrow + 128 * s2 + 32 * j);
        }
        MX_TL(14);
        __syncthreads();
        if (tid < 4 * T) {
            const int tt = tid >> 2;
            const int q4 = tid & 3;
            const uint64_t w4 = static_cast<uint64_t>(os[tt][4 * q4]) | (static_cast<uint64_t>(os[tt][4 * q4 + 1]) << 16) |
                                (static_cast<uint64_t>(os[tt][4 * q4 + 2]) << 32) |
                                (static_cast<uint64_t>(os[tt][4 * q4 + 3]) << 48);
            st_agent64(m.o + static_cast<int64_t>(tt) * kDnValue + rh * kDnWidth + rc0 + 4 * q4, w4);
        }
        // z rows 16 b .. 16 b + 15 (head rh's: its 8 workgroups write all of
        // its z rows), while the rule's stores drain; counted in below with
        // the rule's outputs.
        MX_TL(6);
        unit_mfma(w2, make_uint2(0u, 0u), v2, 0);
        unit_epilogue(v2, 0);
        __builtin_amdgcn_s_waitcnt(0);
        __syncthreads();
        if (tid == 0) {
            const unsigned long long before =
                __hip_atomic_fetch_add(m.heads + kDeltaWsStride * rh, 1ull, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
            last_s = (before + 1) % kMixHeadGroups == 0;
        }
        __syncthreads();
        MX_TL(7);
        // ---- phase C (the head's last workgroup): gated RMSNorm of head rh ----
        if (last_s) {
            const int tt = tid >> 5;
            const int q4 = tid & 31;
            const bool act_t = tt < T;
            // o, z and the norm weights in one round trip (rows t >= T read
            // token 0's and store nothing)
            const int64_t at = static_cast<int64_t>(act_t ? tt : 0) * kDnValue + rh * kDnWidth + 4 * q4;
            const uint64_t o4 = ld_agent64(m.o + at);
            const uint64_t z4 = ld_agent64(a.z + at);
            const uint2 w4 = *reinterpret_cast<const uint2*>(a.norm_w + 4 * q4);
            const float ov[4] = {lo_bf(static_cast<uint32_t>(o4)), hi_bf(static_cast<uint32_t>(o4)),
                                 lo_bf(static_cast<uint32_t>(o4 >> 32)), hi_bf(static_cast<uint32_t>(o4 >> 32))};
            float sq = ov[0] * ov[0] + ov[1] * ov[1] + ov[2] * ov[2] + ov[3] * ov[3];
            sq = sq + __int_as_float(lane_xor<1>(__float_as_int(sq)));
            sq = sq + __int_as_float(lane_xor<2>(__float_as_int(sq)));
            sq = butterfly_step4(sq);
            sq = butterfly_step8(sq);
            sq = sq + __int_as_float(lane_xor<16>(__float_as_int(sq)));
            if (act_t) {
                const float r = 1.0f / __builtin_sqrtf(sq / static_cast<float>(kDnWidth) + a.eps);
                const float zv[4] = {lo_bf(static_cast<uint32_t>(z4)), hi_bf(static_cast<uint32_t>(z4)),
                                     lo_bf(static_cast<uint32_t>(z4 >> 32)), hi_bf(static_cast<uint32_t>(z4 >> 32))};
                const float wv[4] = {lo_bf(w4.x), hi_bf(w4.x), lo_bf(w4.y), hi_bf(w4.y)};
                uint64_t c4 = 0;
#pragma unroll
                for (int i = 0; i < 4; ++i)
                    c4 |= static_cast<uint64_t>(f2bf(rbf(wv[i] * rbf(ov[i] * r)) * silu(zv[i]))) << (16 * i);
                st_agent64(m.core + at, c4);
            }
        }
    }
    MX_TL(8);
    MX_WORD(12, static_cast<unsigned long long>(last_s));
    // Phase D: wave w multiplies the normed rows of heads 4w .. 4w + 3 (k in
    // [512 w, 512 w + 512)), so it waits for those four heads' flags only
    // and requests their rows at once; the waves meet at the reduction.
    // (The head's flag is published once every wave's stores are complete.)
    static_assert(kDnValueHeads == 4 * kMixWaves, "four heads per wave in phase D");
    __builtin_amdgcn_s_waitcnt(0);
    __syncthreads();
    if (tid == 0 && last_s) st_agent64(m.normed + kDeltaWsStride * rh, call);
    if (lane < 4) {
        const unsigned long long* f = m.normed + kDeltaWsStride * (4 * wave + lane);
        const uint64_t start = wall_clock64();
        while (ld_agent64(f) < call) {
            if (wall_clock64() - start > kMixSpinTicks) {
                timeout_s = 1;
                break;
            }
            __builtin_amdgcn_s_sleep(1);
        }
    }
    MX_TL(9);

    // ---- phase D: out_proj rows 8b .. 8b + 7 ----
    {
        // (the residual for the fused add: output row 8b + tid / 16, token
        // tid % 16, clamped for the threads that store none)
        const int res_row = (tid >> 4) & (kMixRows - 1);
        const int res_t = (tid & 15) < T ? (tid & 15) : 0;
        const uint32_t res = ldg_u16(a.x + static_cast<int64_t>(res_t) * kHidden + kMixRows * b + res_row);
        // columns t >= T read token 0's row: their output columns are dropped
        uint4 cb[16];
        const int tc = t < T ? t : 0;
#pragma unroll
        for (int s = 0; s < 4; ++s)
#pragma unroll
            for (int j = 0; j < 4; ++j)
                cb[4 * s + j] = ld_agent16(m.core, static_cast<uint32_t>((tc * kDnValue + 512 * wave + 128 * s + 32 * j + 8 * g) * 2));
        __builtin_amdgcn_sched_barrier(0);  // all 16 loads in flight before the first MFMA
        f32x4 acc = {0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
        for (int i = 0; i < 16; ++i) acc = mfma16x16x32(wo[i], cb[i], acc);
        if (g < 2) {
#pragma unroll
            for (int i = 0; i < 4; ++i) red[wave][4 * g + i][t] = acc[i];
        }
        __syncthreads();
        if (tid < 16 * kMixRows) {
            const int row = tid >> 4;
            const int tt = tid & 15;
            float p = 0.0f;
#pragma unroll
            for (int ww = 0; ww < kMixWaves; ++ww) p += red[ww][row][tt];
            const uint32_t o = f2bf(p);
            if (tt < T) {
                a.out[static_cast<int64_t>(tt) * kHidden + kMixRows * b + row] = static_cast<uint16_t>(o);
                // bf16(x + out), the decoder's residual add
                if (a.sum_out != nullptr)
                    a.sum_out[static_cast<int64_t>(tt) * kHidden + kMixRows * b + row] =
                        static_cast<uint16_t>(f2bf(bf2f(res) + bf2f(o)));
            }
        }
    }
    MX_TL(10);
    if (tid == 0 && timeout_s) atomicOr(m.status, LRMOE_STATUS_TIMEOUT);
}

}  // namespace

hipError_t launch_delta_rule(const DnRuleArgs& a, int key_width, bool state_bf16, hipStream_t stream) {
    switch (key_width) {
        case 64: return launch_rule_d<64>(a, state_bf16, stream);
        case 128: return launch_rule_d<128>(a, state_bf16, stream);
        case 256: return launch_rule_d<256>(a, state_bf16, stream);
        default: return hipErrorInvalidValue;
    }
}

size_t delta_workspace_bytes(int tokens) {
    const DeltaWorkspace w = carve_delta(nullptr, tokens);
    return w.bytes;
}

DeltaWorkspace carve_delta(void* base, int tokens) {
    DeltaWorkspace w{};
    uint8_t* p = static_cast<uint8_t*>(base);
    // control block (fixed offsets whatever the token count; zero at allocation)
    w.status = reinterpret_cast<int32_t*>(p + kDeltaWsStatus);
    w.heads = reinterpret_cast<unsigned long long*>(p + kDeltaWsHeads);
    w.normed = reinterpret_cast<unsigned long long*>(p + kDeltaWsNormed);
    w.staged = reinterpret_cast<unsigned long long*>(p + kDeltaWsStaged);
    size_t off = kDeltaWsControl;
    auto take = [&](size_t bytes) {
        const size_t at = off;
        off += (bytes + 255) & ~static_cast<size_t>(255);
        return p + at;
    };
    const size_t T = static_cast<size_t>(tokens);
    w.act = reinterpret_cast<uint16_t*>(take(T * kDnConv * 2));
    w.z = reinterpret_cast<uint16_t*>(take(T * kDnValue * 2));
    w.beta = reinterpret_cast<uint16_t*>(take(T * kDnValueHeads * 2));
    w.G = reinterpret_cast<float*>(take(T * kDnValueHeads * 4));
    w.o = reinterpret_cast<uint16_t*>(take(T * kDnValue * 2));
    w.core = reinterpret_cast<uint16_t*>(take(T * kDnValue * 2));
    w.bytes = off;
    return w;
}

hipError_t launch_delta_mixer(DnProjectArgs p, void* state, bool state_bf16, void* state_record,
                              const DeltaWorkspace& w, hipStream_t stream) {
    static int cus[64] = {0};
    int device = 0;
    hipError_t err = hipGetDevice(&device);
    if (err != hipSuccess) return err;
    if (device < 0 || device >= 64) return hipErrorInvalidDevice;
    if (cus[device] == 0) {
        err = hipDeviceGetAttribute(&cus[device], hipDeviceAttributeMultiprocessorCount, device);
        if (err != hipSuccess) return err;
    }
    // one workgroup per CU, all resident: the grid barriers need 256 CUs
    if (cus[device] < kMixGrid) return hipErrorNotSupported;
    DnMixerArgs m{};
    p.act = w.act;
    p.z = w.z;
    p.beta = w.beta;
    p.G = w.G;
    m.p = p;
    m.state = state;
    m.state_record = state_record;
    m.o = w.o;
    m.core = w.core;
    m.status = w.status;
    m.heads = w.heads;
    m.normed = w.normed;
    m.staged = w.staged;
    const StageEvents ev = timing_events(kStageDeltaMixer);
    const bool norm = p.in_norm != nullptr;
    if (state_bf16) {
        if (norm) {
            LRMOE_LAUNCH((dn_mixer<true, true>), dim3(kMixGrid), dim3(kMixThreads), 0, stream, ev.start, ev.stop, m);
        } else {
            LRMOE_LAUNCH((dn_mixer<true, false>), dim3(kMixGrid), dim3(kMixThreads), 0, stream, ev.start, ev.stop, m);
        }
    } else {
        if (norm) {
            LRMOE_LAUNCH((dn_mixer<false, true>), dim3(kMixGrid), dim3(kMixThreads), 0, stream, ev.start, ev.stop, m);
        } else {
            LRMOE_LAUNCH((dn_mixer<false, false>), dim3(kMixGrid), dim3(kMixThreads), 0, stream, ev.start, ev.stop, m);
        }
    }
    return hipGetLastError();
}

}  // namespace lrmoe
