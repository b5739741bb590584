// Gated DeltaNet decode on gfx950: the gated delta rule over a short block
// of tokens (edge35b/delta_decode.py:11-55, _delta and _run), and the whole
// cached-decode step of the 35B model's linear-attention mixer ([HF]
// Qwen3_5MoeGatedDeltaNet.forward 430-543: 16 key heads and 32 value heads
// of width 128, conv kernel 4) as four kernels on one stream:
//
//   dn_project<kProjIn>   hidden [T, 2048] times in_proj_qkv / _z / _b / _a
//                         (12352 rows, MFMA with the T <= 16 tokens as the
//                         16 columns), with the causal conv + SiLU and the
//                         conv-state update (qkv channels), beta (b rows) and
//                         G = exp(g) (a rows) in the epilogue;
//   dn_rule               per (value head, block of 4 state columns): the
//                         block's q, k, v, g, beta staged in LDS, l2norm of q
//                         and k, the recurrence over the T tokens with the
//                         state slab in registers, the bf16 output;
//   dn_gate_norm          the gated RMSNorm per (token, value head);
//   dn_project<kProjOut>  out_proj [2048, 4096].
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

enum ProjMode : int { kProjIn = 0, kProjOut = 1 };

// Per mode: workgroup waves (each owns a 512-wide slice of the reduction
// dimension), tiles per workgroup (each wave multiplies its slice of every
// tile with the same input fragments) and rows per tile (16: every MFMA row
// is a weight row; 8: half the rows are zero so out_proj still has 256
// workgroups).  in_proj: 386 workgroups of 2 x 16 rows, all resident at
// once (two per CU at 2 waves per SIMD), so no tile waits for a second round.
template <int MODE> struct ProjShape;
template <> struct ProjShape<kProjIn> {
    static constexpr int kWaves = 4, kTiles = 2, kRows = 16, kK = 2048;
};
template <> struct ProjShape<kProjOut> {
    static constexpr int kWaves = 8, kTiles = 1, kRows = 8, kK = 4096;
};

__device__ __forceinline__ float silu(float x) { return x / (1.0f + lr_exp(-x)); }

__device__ __forceinline__ float softplus(float x) { return x > 20.0f ? x : log1pf(lr_exp(x)); }

// out[t][n] = bf16(sum_k X[t][k] W[n][k]) for kTiles tiles of kRows weight
// rows (workgroup blockIdx.x), T <= 16 tokens.  Wave w multiplies k in
// [512w, 512w + 512): per 128-wide step s, lane l (token l % 16, group
// g = l / 16) holds the eight values at 128s + 32j + 8g (j = 0..3) of its
// row's weights (A, per tile) and of its token's input (B, shared by the
// tiles), so each load instruction reads 64 contiguous bytes per row.  The
// waves' 16x16 partial tiles are summed in LDS in wave order, then the
// mode's epilogue runs on (row, token) = (tid / 16 % 16, tid % 16).
template <int MODE>
__global__ __launch_bounds__(ProjShape<MODE>::kWaves * 64) void dn_project(DnProjectArgs a) {
    constexpr int kWaves = ProjShape<MODE>::kWaves;
    constexpr int kTiles = ProjShape<MODE>::kTiles;
    constexpr int kRows = ProjShape<MODE>::kRows;
    constexpr int kK = ProjShape<MODE>::kK;
    __shared__ float red[kTiles][kWaves][16][17];
    __shared__ uint16_t seq[16][kDnTaps + 16];  // conv: per row the cached context, then the projections

    const int lane = threadIdx.x & 63;
    const int wave = threadIdx.x >> 6;
    const int t = lane & 15;
    const int g = lane >> 4;
    const int T = a.tokens;
    const int n0 = blockIdx.x * kRows * kTiles;
    const int k0 = 512 * wave + 8 * g;

    // the weight rows of this workgroup's tiles (no tile pair straddles two
    // matrices: every boundary is a multiple of 32 rows)
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

    // the epilogue's small operands, fetched before the weights stream
    const int tid = threadIdx.x;
    const int row = (tid >> 4) & 15;
    const int tt = tid & 15;
    uint2 conv_w[kTiles] = {};
    uint32_t conv_old[kTiles] = {};
    float A[kTiles] = {}, dt[kTiles] = {};
    if constexpr (MODE == kProjIn) {
        if (seg == 0 && tid < 256) {
#pragma unroll
            for (int u = 0; u < kTiles; ++u) {
                const int n = n0 + u * kRows + row;
                conv_w[u] = *reinterpret_cast<const uint2*>(a.conv_w + n * kDnTaps);
                if (tt < kDnTaps) conv_old[u] = ldg_u16(a.conv_state + n * kDnTaps + tt);
            }
        } else if (seg == 3 && tid < 256) {
#pragma unroll
            for (int u = 0; u < kTiles; ++u) {
                const int h = n0 + u * kRows + row - kDnARow;
                A[u] = bf2f(ldg_u16(a.A_log + h));
                dt[u] = bf2f(ldg_u16(a.dt_bias + h));
            }
        }
    }

    uint4 wa[kTiles][16];
    const bool row_live = t < kRows;
#pragma unroll
    for (int u = 0; u < kTiles; ++u) {
        const uint16_t* wrow = W + static_cast<int64_t>(u * kRows + t) * kK + k0;
#pragma unroll
        for (int s = 0; s < 4; ++s)
#pragma unroll
            for (int j = 0; j < 4; ++j)
                wa[u][4 * s + j] = row_live ? ldg16(wrow + 128 * s + 32 * j) : make_uint4(0u, 0u, 0u, 0u);
    }
    uint4 xb[16];
    const uint16_t* xrow = a.x + static_cast<int64_t>(t) * kK + k0;
#pragma unroll
    for (int s = 0; s < 4; ++s)
#pragma unroll
        for (int j = 0; j < 4; ++j) xb[4 * s + j] = t < T ? ldg16(xrow + 128 * s + 32 * j) : make_uint4(0u, 0u, 0u, 0u);

#pragma unroll
    for (int u = 0; u < kTiles; ++u) {
        f32x4 acc = {0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
        for (int i = 0; i < 16; ++i) acc = mfma16x16x32(wa[u][i], xb[i], acc);
#pragma unroll
        for (int i = 0; i < 4; ++i) red[u][wave][4 * g + i][t] = acc[i];
    }
    __syncthreads();

#pragma unroll
    for (int u = 0; u < kTiles; ++u) {
        float p = 0.0f;
        if (tid < 256) {
#pragma unroll
            for (int w = 0; w < kWaves; ++w) p += red[u][w][row][tt];
        }
        const int n = n0 + u * kRows + row;
        if constexpr (MODE == kProjOut) {
            if (tid < 256 && row < kRows && tt < T) a.out[static_cast<int64_t>(tt) * kHidden + n] = static_cast<uint16_t>(f2bf(p));
        } else {
            if (seg == 0) {
                // causal conv over [cached 4 inputs, the T projections], SiLU;
                // the cache keeps the last 4 (channel n belongs to this tile)
                if (u > 0) __syncthreads();  // the previous tile's conv has read seq
                seq[row][kDnTaps + tt] = static_cast<uint16_t>(f2bf(p));
                if (tt < kDnTaps) seq[row][tt] = static_cast<uint16_t>(conv_old[u]);
                __syncthreads();
                if (tt < T) {
                    const float w[kDnTaps] = {lo_bf(conv_w[u].x), hi_bf(conv_w[u].x), lo_bf(conv_w[u].y), hi_bf(conv_w[u].y)};
                    float c = 0.0f;
#pragma unroll
                    for (int j = 0; j < kDnTaps; ++j) c = __builtin_fmaf(w[j], bf2f(seq[row][tt + 1 + j]), c);
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
                    const float gv = -lr_exp(A[u]) * softplus(bf2f(pb) + dt[u]);
                    a.G[tt * kDnValueHeads + h] = lr_exp(gv);
                }
            }
        }
    }
}

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

// The gated RMSNorm of the mixer ([HF] Qwen3_5MoeRMSNormGated 169-185) for
// token blockIdx.y, value head blockIdx.x, one thread per element e:
// n = bf16(o rsqrt(mean(o^2) + eps)), core = bf16(bf16(w n) silu(z)).  The
// sum of squares: a butterfly per wave, then wave 0's sum plus wave 1's.
__global__ __launch_bounds__(kDnWidth) void dn_gate_norm(const uint16_t* o, const uint16_t* z, const uint16_t* norm_w,
                                                         float eps, uint16_t* core) {
    __shared__ float part[kDnWidth / 64];
    const int e = threadIdx.x;
    const int64_t at = static_cast<int64_t>(blockIdx.y) * kDnValue + blockIdx.x * kDnWidth + e;
    const float ov = bf2f(ldg_u16(o + at));
    const float zv = bf2f(ldg_u16(z + at));
    const float wv = bf2f(ldg_u16(norm_w + e));
    const float s = wave_butterfly_sum(ov * ov);
    if ((e & 63) == 0) part[e >> 6] = s;
    __syncthreads();
    const float r = 1.0f / __builtin_sqrtf((part[0] + part[1]) / static_cast<float>(kDnWidth) + eps);
    core[at] = static_cast<uint16_t>(f2bf(rbf(wv * rbf(ov * r)) * silu(zv)));
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
    w.core = reinterpret_cast<uint16_t*>(take(T * kDnValue * 2));
    w.bytes = off;
    return w;
}

hipError_t launch_delta_mixer(DnProjectArgs p, const void* state, bool state_bf16, void* state_record,
                              const DeltaWorkspace& w, hipStream_t stream) {
    p.act = w.act;
    p.z = w.z;
    p.beta = w.beta;
    p.G = w.G;
    {
        const StageEvents ev = timing_events(kStageDeltaIn);
        LRMOE_LAUNCH((dn_project<kProjIn>), dim3(kDnProjRows / (ProjShape<kProjIn>::kRows * ProjShape<kProjIn>::kTiles)),
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
    r.tokens = p.tokens;
    r.heads = kDnValueHeads;
    r.width = kDnWidth;
    r.normalize = 1;
    hipError_t err = launch_rule_d<kDnWidth>(r, state_bf16, stream);
    if (err != hipSuccess) return err;
    {
        const StageEvents ev = timing_events(kStageDeltaNorm);
        LRMOE_LAUNCH(dn_gate_norm, dim3(kDnValueHeads, p.tokens), dim3(kDnWidth), 0, stream, ev.start, ev.stop, w.o, w.z,
                     p.norm_w, p.eps, w.core);
        err = hipGetLastError();
        if (err != hipSuccess) return err;
    }
    p.x = w.core;
    {
        const StageEvents ev = timing_events(kStageDeltaOut);
        LRMOE_LAUNCH((dn_project<kProjOut>), dim3(kHidden / (ProjShape<kProjOut>::kRows * ProjShape<kProjOut>::kTiles)),
                     dim3(ProjShape<kProjOut>::kWaves * 64), 0, stream, ev.start, ev.stop, p);
    }
    return hipGetLastError();
}

}  // namespace lrmoe
