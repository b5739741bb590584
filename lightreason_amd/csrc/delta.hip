// Gated DeltaNet decode on gfx950: the gated delta rule over a short block
// of tokens (edge35b/delta_decode.py:11-55, _delta and _run), and the whole
// cached-decode step of the 35B model's linear-attention mixer ([HF]
// Qwen3_5MoeGatedDeltaNet.forward 430-543: 16 key heads and 32 value heads
// of width 128, conv kernel 4) as three kernels on one stream:
//
//   dn_project<kProjIn>   hidden [T, 2048] times in_proj_qkv / _z / _b / _a
//                         (12352 rows, MFMA with the T <= 16 tokens as the
//                         16 columns), with the causal conv + SiLU and the
//                         conv-state update (qkv channels), beta (b rows) and
//                         G = exp(g) (a rows) in the epilogue;
//   dn_rule               per (value head, block of 16 state columns): l2norm
//                         of q and k, the recurrence over the T tokens with
//                         the state slab in registers, the bf16 output and
//                         its per-block sums of squares;
//   dn_project<kProjOut>  out_proj [2048, 4096] whose MFMA operand is the
//                         gated RMSNorm of the rule's output, formed as it is
//                         loaded.
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
constexpr int kDnARow = kDnBRow + kDnValueHeads;    // first in_proj_a row
constexpr int kDnProjRows = kDnARow + kDnValueHeads;  // 12352
constexpr int kDnBlocks = kDnWidth / 16;            // 16-column blocks per value head

enum ProjMode : int { kProjIn = 0, kProjOut = 1 };

// Per mode: workgroup waves (each owns a 512-wide slice of the reduction
// dimension), rows per tile (16: every MFMA row is a weight row; 8: half the
// rows are zero so out_proj still has 256 workgroups).
template <int MODE> struct ProjShape;
template <> struct ProjShape<kProjIn> {
    static constexpr int kWaves = 4, kRows = 16, kK = 2048;
};
template <> struct ProjShape<kProjOut> {
    static constexpr int kWaves = 8, kRows = 8, kK = 4096;
};

__device__ __forceinline__ float silu(float x) { return x / (1.0f + lr_exp(-x)); }

__device__ __forceinline__ float softplus(float x) { return x > 20.0f ? x : log1pf(lr_exp(x)); }

// Eight bf16 values of the gated RMSNorm output for one token and value
// head: o8 the rule's output, z8 the gate, w8 the norm weight, r the
// head's 1/sqrt(mean(o^2) + eps).
__device__ __forceinline__ uint4 gated_norm8(uint4 o8, uint4 z8, uint4 w8, float r) {
    float o[8], z[8], w[8];
    unpack8(o8, o);
    unpack8(z8, z);
    unpack8(w8, w);
    uint32_t b[8];
#pragma unroll
    for (int i = 0; i < 8; ++i) {
        const float n = rbf(o[i] * r);
        const float wn = rbf(w[i] * n);
        b[i] = f2bf(wn * silu(z[i]));
    }
    return make_uint4(b[0] | (b[1] << 16), b[2] | (b[3] << 16), b[4] | (b[5] << 16), b[6] | (b[7] << 16));
}

// out[t][n] = bf16(sum_k X[t][k] W[n][k]) for one tile of kRows weight rows
// (blockIdx.x), T <= 16 tokens.  Wave w multiplies k in [512w, 512w + 512):
// per 128-wide step s, lane l (token l % 16, group g = l / 16) holds the
// eight values at 128s + 32j + 8g for j = 0..3 of its row's weights (A) and
// of its token's input (B), so each load instruction reads 64 contiguous
// bytes per row.  The waves' 16x16 partial tiles are summed in LDS in wave
// order, then the mode's epilogue runs on (row, token) = (tid / 16, tid % 16).
template <int MODE>
__global__ __launch_bounds__(ProjShape<MODE>::kWaves * 64) void dn_project(DnProjectArgs a) {
    constexpr int kWaves = ProjShape<MODE>::kWaves;
    constexpr int kRows = ProjShape<MODE>::kRows;
    constexpr int kK = ProjShape<MODE>::kK;
    __shared__ float red[kWaves][16][17];
    __shared__ uint16_t seq[16][kDnTaps + 16];  // conv: per row the cached context, then the projections

    const int lane = threadIdx.x & 63;
    const int wave = threadIdx.x >> 6;
    const int t = lane & 15;
    const int g = lane >> 4;
    const int T = a.tokens;
    const int n0 = blockIdx.x * kRows;
    const int k0 = 512 * wave + 8 * g;

    // this tile's weight rows
    const uint16_t* W;
    int seg = 0;
    if constexpr (MODE == kProjIn) {
        if (n0 < kDnZRow) {
            W = a.w_qkv + static_cast<int64_t>(n0) * kK;
        } else if (n0 < kDnBRow) {
            W = a.w_z + static_cast<int64_t>(n0 - kDnZRow) * kK;
            seg = 1;
        } else if (n0 < kDnARow) {
            W = a.w_b + static_cast<int64_t>(n0 - kDnBRow) * kK;
            seg = 2;
        } else {
            W = a.w_a + static_cast<int64_t>(n0 - kDnARow) * kK;
            seg = 3;
        }
    } else {
        W = a.w_out + static_cast<int64_t>(n0) * kK;
    }

    uint4 wa[16];
    const bool row_live = t < kRows;
    const uint16_t* wrow = W + static_cast<int64_t>(t) * kK + k0;
#pragma unroll
    for (int s = 0; s < 4; ++s)
#pragma unroll
        for (int j = 0; j < 4; ++j)
            wa[4 * s + j] = row_live ? ldg16(wrow + 128 * s + 32 * j) : make_uint4(0u, 0u, 0u, 0u);

    uint4 xb[16];
    if (t < T) {
        if constexpr (MODE == kProjIn) {
            const uint16_t* xrow = a.x + static_cast<int64_t>(t) * kK + k0;
#pragma unroll
            for (int s = 0; s < 4; ++s)
#pragma unroll
                for (int j = 0; j < 4; ++j) xb[4 * s + j] = ldg16(xrow + 128 * s + 32 * j);
        } else {
            // step s of wave w covers value head 4w + s; the lane's chunks sit
            // at e = 32j + 8g inside it
#pragma unroll
            for (int s = 0; s < 4; ++s) {
                const int head = 4 * wave + s;
                const float* part = a.sumsq + (static_cast<int64_t>(t) * kDnValueHeads + head) * kDnBlocks;
                float sum = 0.0f;
#pragma unroll
                for (int b = 0; b < kDnBlocks; ++b) sum += part[b];
                const float r = 1.0f / __builtin_sqrtf(sum / static_cast<float>(kDnWidth) + a.eps);
                const int64_t base = static_cast<int64_t>(t) * kDnValue + head * kDnWidth + 8 * g;
#pragma unroll
                for (int j = 0; j < 4; ++j)
                    xb[4 * s + j] = gated_norm8(ldg16(a.o + base + 32 * j), ldg16(a.z_in + base + 32 * j),
                                                ldg16(a.norm_w + 8 * g + 32 * j), r);
            }
        }
    } else {
#pragma unroll
        for (int i = 0; i < 16; ++i) xb[i] = make_uint4(0u, 0u, 0u, 0u);
    }

    f32x4 acc = {0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
    for (int i = 0; i < 16; ++i) acc = mfma16x16x32(wa[i], xb[i], acc);
#pragma unroll
    for (int i = 0; i < 4; ++i) red[wave][4 * g + i][t] = acc[i];
    __syncthreads();

    const int tid = threadIdx.x;
    const int row = (tid >> 4) & 15;
    const int tt = tid & 15;
    float p = 0.0f;
    if (tid < 256) {
#pragma unroll
        for (int w = 0; w < kWaves; ++w) p += red[w][row][tt];
    }
    const int n = n0 + row;

    if constexpr (MODE == kProjOut) {
        if (tid < 256 && row < kRows && tt < T) a.out[static_cast<int64_t>(tt) * kHidden + n] = static_cast<uint16_t>(f2bf(p));
        return;
    } else {
        if (seg == 0) {
            // causal conv over [cached 4 inputs, the T projections], SiLU;
            // the cache keeps the last 4 (channel n is owned by this tile)
            seq[row][kDnTaps + tt] = static_cast<uint16_t>(f2bf(p));
            if (tt < kDnTaps) seq[row][tt] = static_cast<uint16_t>(ldg_u16(a.conv_state + n * kDnTaps + tt));
            __syncthreads();
            if (tt < T) {
                float c = 0.0f;
#pragma unroll
                for (int j = 0; j < kDnTaps; ++j)
                    c = __builtin_fmaf(bf2f(ldg_u16(a.conv_w + n * kDnTaps + j)), bf2f(seq[row][tt + 1 + j]), c);
                a.act[static_cast<int64_t>(tt) * kDnConv + n] = static_cast<uint16_t>(f2bf(silu(rbf(c))));
                if (a.conv_record) {
                    uint16_t* rec = a.conv_record + (static_cast<int64_t>(tt) * kDnConv + n) * kDnTaps;
#pragma unroll
                    for (int j = 0; j < kDnTaps; ++j) rec[j] = seq[row][tt + 1 + j];
                }
            }
            if (tt < kDnTaps) a.conv_state[n * kDnTaps + tt] = seq[row][T + tt];
        } else if (tt < T) {
            const uint32_t pb = f2bf(p);
            if (seg == 1) {
                a.z[static_cast<int64_t>(tt) * kDnValue + (n - kDnZRow)] = static_cast<uint16_t>(pb);
            } else if (seg == 2) {
                const int h = n - kDnBRow;
                a.beta[tt * kDnValueHeads + h] = static_cast<uint16_t>(f2bf(1.0f / (1.0f + lr_exp(-bf2f(pb)))));
            } else {
                const int h = n - kDnARow;
                const float gv = -lr_exp(bf2f(ldg_u16(a.A_log + h))) * softplus(bf2f(pb) + bf2f(ldg_u16(a.dt_bias + h)));
                a.G[tt * kDnValueHeads + h] = lr_exp(gv);
            }
        }
    }
}

// Sum over the 16 lanes that share lane % 4 (lane bits 2..5).
__device__ __forceinline__ float sum_rows(float v) {
    v += __shfl_xor(v, 4);
    v += __shfl_xor(v, 8);
    v += __shfl_xor(v, 16);
    v += __shfl_xor(v, 32);
    return v;
}

template <int R>
__device__ __forceinline__ void load_bf16_rows(const uint16_t* p, float* out) {
    if constexpr (R == 4) {
        const uint2 v = *reinterpret_cast<const uint2*>(p);
        out[0] = lo_bf(v.x); out[1] = hi_bf(v.x); out[2] = lo_bf(v.y); out[3] = hi_bf(v.y);
    } else {
#pragma unroll
        for (int i = 0; i < R; i += 8) unpack8(ldg16(p + i), out + i);
    }
}

// l2norm of a D-wide head split over the 16 row groups of a wave (R values
// per lane), every step rounded to bf16 as torch does on bf16 tensors:
// x * bf16(1 / sqrt(bf16(bf16(sum bf16(x^2)) + 1e-6))), rounded.
template <int R>
__device__ __forceinline__ void l2norm_rows(float* x) {
    float s = 0.0f;
#pragma unroll
    for (int i = 0; i < R; ++i) s += rbf(x[i] * x[i]);
    s = sum_rows(s);
    const float inv = rbf(1.0f / __builtin_sqrtf(rbf(rbf(s) + 1e-6f)));
#pragma unroll
    for (int i = 0; i < R; ++i) x[i] = rbf(x[i] * inv);
}

template <bool BF16>
__device__ __forceinline__ void load_state4(const void* base, int64_t idx, float* s) {
    if constexpr (BF16) {
        const uint2 v = *reinterpret_cast<const uint2*>(static_cast<const uint16_t*>(base) + idx);
        s[0] = lo_bf(v.x); s[1] = hi_bf(v.x); s[2] = lo_bf(v.y); s[3] = hi_bf(v.y);
    } else {
        const float4 v = *reinterpret_cast<const float4*>(static_cast<const float*>(base) + idx);
        s[0] = v.x; s[1] = v.y; s[2] = v.z; s[3] = v.w;
    }
}

template <bool BF16>
__device__ __forceinline__ void store_state4(void* base, int64_t idx, const float* s) {
    if constexpr (BF16) {
        *reinterpret_cast<uint2*>(static_cast<uint16_t*>(base) + idx) =
            make_uint2(f2bf(s[0]) | (f2bf(s[1]) << 16), f2bf(s[2]) | (f2bf(s[3]) << 16));
    } else {
        *reinterpret_cast<float4*>(static_cast<float*>(base) + idx) = make_float4(s[0], s[1], s[2], s[3]);
    }
}

// The gated delta rule for value head blockIdx.x, state columns
// 16 blockIdx.y .. +15, one wave: lane (row group rg = lane / 4, column
// quad c4 = lane % 4) holds state rows rg R .. rg R + R - 1 (R = D / 16) of
// columns 16 blockIdx.y + 4 c4 .. +3 in registers for all T tokens.  Per
// token: state *= G; mem = state^T k; delta = (v - mem) beta;
// state += k delta^T; out = state^T (q D^-1/2); the state then rounded to
// its dtype (a no-op for fp32).  Column sums over the D rows: in-lane, then
// across the 16 row groups.
template <int D, bool BF16>
__global__ __launch_bounds__(64) void dn_rule(DnRuleArgs a) {
    constexpr int R = D / 16;
    const int lane = threadIdx.x;
    const int rg = lane >> 2;
    const int c4 = lane & 3;
    const int h = blockIdx.x;
    const int cb = blockIdx.y;
    const int H = a.heads;
    const int E = a.width;
    const int col = cb * 16 + 4 * c4;
    const int64_t slab = static_cast<int64_t>(h) * D * E;

    float S[R][4];
#pragma unroll
    for (int i = 0; i < R; ++i) load_state4<BF16>(a.initial, slab + static_cast<int64_t>(rg * R + i) * E + col, S[i]);

    const float scale = 1.0f / __builtin_sqrtf(static_cast<float>(D));
    const int kh = h >> a.kv_shift;
    for (int t = 0; t < a.tokens; ++t) {
        float q[R], k[R];
        load_bf16_rows<R>(a.q + t * a.qk_stride + static_cast<int64_t>(kh) * D + rg * R, q);
        load_bf16_rows<R>(a.k + t * a.qk_stride + static_cast<int64_t>(kh) * D + rg * R, k);
        if (a.normalize) {
            l2norm_rows<R>(q);
            l2norm_rows<R>(k);
        }
#pragma unroll
        for (int i = 0; i < R; ++i) q[i] = q[i] * scale;
        float v[4];
        {
            const uint2 vv = *reinterpret_cast<const uint2*>(a.v + t * a.v_stride + static_cast<int64_t>(h) * E + col);
            v[0] = lo_bf(vv.x); v[1] = hi_bf(vv.x); v[2] = lo_bf(vv.y); v[3] = hi_bf(vv.y);
        }
        const float G = a.G[t * H + h];
        const float beta = bf2f(a.beta[t * H + h]);

        float mem[4] = {0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
        for (int i = 0; i < R; ++i)
#pragma unroll
            for (int c = 0; c < 4; ++c) {
                S[i][c] = S[i][c] * G;
                mem[c] = mem[c] + S[i][c] * k[i];
            }
        float delta[4];
#pragma unroll
        for (int c = 0; c < 4; ++c) delta[c] = (v[c] - sum_rows(mem[c])) * beta;
        float o[4] = {0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
        for (int i = 0; i < R; ++i)
#pragma unroll
            for (int c = 0; c < 4; ++c) {
                S[i][c] = S[i][c] + k[i] * delta[c];
                o[c] = o[c] + S[i][c] * q[i];
            }
        uint32_t ob[4];
#pragma unroll
        for (int c = 0; c < 4; ++c) ob[c] = f2bf(sum_rows(o[c]));
        const int64_t orow = (static_cast<int64_t>(t) * H + h) * E + col;
        if (rg == 0) *reinterpret_cast<uint2*>(a.out + orow) = make_uint2(ob[0] | (ob[1] << 16), ob[2] | (ob[3] << 16));
        if (a.sumsq) {
            float sq = 0.0f;
#pragma unroll
            for (int c = 0; c < 4; ++c) sq = sq + bf2f(ob[c]) * bf2f(ob[c]);
            sq += __shfl_xor(sq, 1);
            sq += __shfl_xor(sq, 2);
            if (lane == 0) a.sumsq[(static_cast<int64_t>(t) * H + h) * (E / 16) + cb] = sq;
        }
        if constexpr (BF16) {
#pragma unroll
            for (int i = 0; i < R; ++i)
#pragma unroll
                for (int c = 0; c < 4; ++c) S[i][c] = rbf(S[i][c]);
        }
        if (a.record) {
            const int64_t rec = static_cast<int64_t>(t) * H * D * E + slab;
#pragma unroll
            for (int i = 0; i < R; ++i) store_state4<BF16>(a.record, rec + static_cast<int64_t>(rg * R + i) * E + col, S[i]);
        }
    }
    if (a.final_state) {
#pragma unroll
        for (int i = 0; i < R; ++i) store_state4<BF16>(a.final_state, slab + static_cast<int64_t>(rg * R + i) * E + col, S[i]);
    }
}

template <int D>
hipError_t launch_rule_d(const DnRuleArgs& a, bool bf16, hipStream_t stream) {
    const StageEvents ev = timing_events(kStageDeltaRule);
    const dim3 grid(a.heads, a.width / 16);
    if (bf16) {
        LRMOE_LAUNCH((dn_rule<D, true>), grid, dim3(64), 0, stream, ev.start, ev.stop, a);
    } else {
        LRMOE_LAUNCH((dn_rule<D, false>), grid, dim3(64), 0, stream, ev.start, ev.stop, a);
    }
    return hipGetLastError();
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
    size_t off = 0;
    auto take = [&](size_t bytes) {
        const size_t at = off;
        off += (bytes + 255) & ~static_cast<size_t>(255);
        return static_cast<uint8_t*>(base) + at;
    };
    const size_t T = static_cast<size_t>(tokens);
    w.act = reinterpret_cast<uint16_t*>(take(T * kDnConv * 2));
    w.z = reinterpret_cast<uint16_t*>(take(T * kDnValue * 2));
    w.beta = reinterpret_cast<uint16_t*>(take(T * kDnValueHeads * 2));
    w.G = reinterpret_cast<float*>(take(T * kDnValueHeads * 4));
    w.o = reinterpret_cast<uint16_t*>(take(T * kDnValue * 2));
    w.sumsq = reinterpret_cast<float*>(take(T * kDnValueHeads * kDnBlocks * 4));
    w.bytes = off;
    return w;
}

hipError_t launch_delta_mixer(DnProjectArgs p, const void* state, bool state_bf16, void* state_record,
                              const DeltaWorkspace& w, hipStream_t stream) {
    p.act = w.act;
    p.z = w.z;
    p.z_in = w.z;
    p.beta = w.beta;
    p.G = w.G;
    p.o = w.o;
    p.sumsq = w.sumsq;
    {
        const StageEvents ev = timing_events(kStageDeltaIn);
        LRMOE_LAUNCH((dn_project<kProjIn>), dim3(kDnProjRows / ProjShape<kProjIn>::kRows),
                     dim3(ProjShape<kProjIn>::kWaves * 64), 0, stream, ev.start, ev.stop, p);
        const hipError_t err = hipGetLastError();
        if (err != hipSuccess) return err;
    }
    DnRuleArgs r{};
    r.q = w.act;
    r.k = w.act + kDnKey;
    r.v = w.act + 2 * kDnKey;
    r.qk_stride = kDnConv;
    r.v_stride = kDnConv;
    r.kv_shift = 1;  // value head h reads key head h / 2 (repeat_interleave by 2)
    r.G = w.G;
    r.beta = w.beta;
    r.initial = state;
    r.final_state = const_cast<void*>(state);
    r.record = state_record;
    r.out = w.o;
    r.sumsq = w.sumsq;
    r.tokens = p.tokens;
    r.heads = kDnValueHeads;
    r.width = kDnWidth;
    r.normalize = 1;
    hipError_t err = launch_rule_d<kDnWidth>(r, state_bf16, stream);
    if (err != hipSuccess) return err;
    {
        const StageEvents ev = timing_events(kStageDeltaOut);
        LRMOE_LAUNCH((dn_project<kProjOut>), dim3(kHidden / ProjShape<kProjOut>::kRows),
                     dim3(ProjShape<kProjOut>::kWaves * 64), 0, stream, ev.start, ev.stop, p);
    }
    return hipGetLastError();
}

}  // namespace lrmoe
