// Routed-expert SwiGLU on BF16 MFMA, and the ordered weighted combine.
//
// Semantics: edge35b/cpu_experts.c:54-69 (gate and up rounded to bf16,
// bf16 SiLU, bf16 SiLU*up, bf16 down output; fp32 accumulation) and
// edge35b/fused_experts.py:27-37 / block_experts.py:31-49 (per token, routes
// in ascending expert order, acc = bf16(acc + bf16(y * w)) from 0), then the
// shared expert of Qwen3_5MoeSparseMoeBlock.forward
// (out = bf16(routed + bf16(sigmoid_gate * shared))) and, for a decoder layer,
// the residual add.
//
// Layout of the work: a workgroup owns one (expert, 16-row tile) and streams
// that tile's weights exactly once from HBM straight into MFMA A operands;
// every token routed to the expert is a column of the B operand (up to 16
// per MFMA), so a weight byte read from HBM serves all of its tokens.  The
// 16x16x32 bf16 MFMA accumulates in fp32.
#include "lrmoe_device.h"
#include "lrmoe_internal.h"

namespace lrmoe {
namespace {

constexpr int kGateTiles = kInner / 16;      // 32 tiles of 16 gate (and 16 up) rows
constexpr int kDownRowsPerWg = 64;           // 4 waves x 16 output rows
constexpr int kDownTiles = kHidden / kDownRowsPerWg;

__device__ __forceinline__ uint4 zero4() { return make_uint4(0, 0, 0, 0); }

struct Group {
    const uint16_t* gate;   // [512][2048]
    const uint16_t* up;     // [512][2048]
    const uint16_t* down;   // [2048][512]
    const int32_t* tokens;  // token of each column, or null for 0..n-1
    int pair0;              // first act/y row of this group
    int count;              // tokens in the group
};

// slot 0 is the shared expert, slot s >= 1 the (s-1)-th unique routed expert.
__device__ __forceinline__ bool load_group(const ExpertArgs& a, int slot, Group& g) {
    if (slot == 0) {
        if (a.shared_down == nullptr) return false;
        g.gate = a.shared_gate_proj;
        g.up = a.shared_up_proj;
        g.down = a.shared_down;
        g.tokens = nullptr;
        g.pair0 = kTopK * a.tokens;
        g.count = a.tokens;
        return true;
    }
    const int u = slot - 1;
    if (u >= *a.plan.unique) return false;
    const int e = a.plan.expert[u];
    const uint16_t* gate_up = reinterpret_cast<const uint16_t*>(a.expert_ptrs[2 * e]);
    g.gate = gate_up;
    g.up = gate_up + static_cast<size_t>(kInner) * kHidden;
    g.down = reinterpret_cast<const uint16_t*>(a.expert_ptrs[2 * e + 1]);
    g.pair0 = a.plan.offset[u];
    g.count = a.plan.offset[u + 1] - g.pair0;
    g.tokens = a.plan.pair_token + g.pair0;
    return true;
}

// Gate/up + SwiGLU.  Wave w covers k in [512w, 512w+512) of a 16-row tile;
// the four partial tiles meet in LDS in wave order.  Columns beyond 16 tokens
// are handled in successive 16-token blocks that re-read the (now cached)
// weight tile.
__global__ __launch_bounds__(256) void gateup_kernel(ExpertArgs a) {
    Group grp;
    if (!load_group(a, blockIdx.x / kGateTiles, grp)) return;
    const int tile = blockIdx.x % kGateTiles;
    const int wave = threadIdx.x >> 6;
    const int lane = threadIdx.x & 63;
    const int n = lane & 15;
    const int g = lane >> 4;
    const int row0 = tile * 16;
    const int k0 = wave * 512 + 8 * g;
    const uint16_t* gate_row = grp.gate + static_cast<size_t>(row0 + n) * kHidden + k0;
    const uint16_t* up_row = grp.up + static_cast<size_t>(row0 + n) * kHidden + k0;
    __shared__ f32x4 red[4][2][kWave];

    for (int nb = 0; nb < grp.count; nb += 16) {
        const int col = nb + n;
        const bool live = col < grp.count;
        const int token = live ? (grp.tokens ? grp.tokens[col] : col) : 0;
        const uint16_t* x_row = a.x + static_cast<size_t>(token) * kHidden + k0;
        f32x4 acc_g = {0.0f, 0.0f, 0.0f, 0.0f};
        f32x4 acc_u = {0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
        for (int half = 0; half < 2; ++half) {
            uint4 ag[8], au[8], bx[8];
#pragma unroll
            for (int s = 0; s < 8; ++s) {
                const int k = 32 * (8 * half + s);
                ag[s] = *reinterpret_cast<const uint4*>(gate_row + k);
                au[s] = *reinterpret_cast<const uint4*>(up_row + k);
                bx[s] = live ? *reinterpret_cast<const uint4*>(x_row + k) : zero4();
            }
#pragma unroll
            for (int s = 0; s < 8; ++s) {
                acc_g = mfma16x16x32(ag[s], bx[s], acc_g);
                acc_u = mfma16x16x32(au[s], bx[s], acc_u);
            }
        }
        red[wave][0][lane] = acc_g;
        red[wave][1][lane] = acc_u;
        __syncthreads();
        if (wave == 0) {
            const f32x4 sg = ((red[0][0][lane] + red[1][0][lane]) + red[2][0][lane]) + red[3][0][lane];
            const f32x4 su = ((red[0][1][lane] + red[1][1][lane]) + red[2][1][lane]) + red[3][1][lane];
            if (live) {
                uint32_t act[4];
#pragma unroll
                for (int i = 0; i < 4; ++i) act[i] = swiglu_bf16(rbf(sg[i]), rbf(su[i]));
                uint16_t* dst = a.ws.act + static_cast<size_t>(grp.pair0 + col) * kInner + row0 + 4 * g;
                *reinterpret_cast<uint2*>(dst) = make_uint2(act[0] | (act[1] << 16), act[2] | (act[3] << 16));
            }
        }
        __syncthreads();
    }
}

// Down projection: wave w owns 16 output rows of a 64-row tile, full k = 512.
__global__ __launch_bounds__(256) void down_kernel(ExpertArgs a) {
    Group grp;
    if (!load_group(a, blockIdx.x / kDownTiles, grp)) return;
    const int tile = blockIdx.x % kDownTiles;
    const int wave = threadIdx.x >> 6;
    const int lane = threadIdx.x & 63;
    const int n = lane & 15;
    const int g = lane >> 4;
    const int h0 = tile * kDownRowsPerWg + 16 * wave;
    const uint16_t* w_row = grp.down + static_cast<size_t>(h0 + n) * kInner + 8 * g;
    uint4 aw[16];
#pragma unroll
    for (int s = 0; s < 16; ++s) aw[s] = *reinterpret_cast<const uint4*>(w_row + 32 * s);
    for (int nb = 0; nb < grp.count; nb += 16) {
        const int col = nb + n;
        const bool live = col < grp.count;
        const uint16_t* act_row = a.ws.act + static_cast<size_t>(grp.pair0 + (live ? col : 0)) * kInner + 8 * g;
        uint4 bx[16];
#pragma unroll
        for (int s = 0; s < 16; ++s) bx[s] = live ? *reinterpret_cast<const uint4*>(act_row + 32 * s) : zero4();
        f32x4 acc = {0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
        for (int s = 0; s < 16; ++s) acc = mfma16x16x32(aw[s], bx[s], acc);
        if (live) {
            uint16_t* dst = a.ws.y + static_cast<size_t>(grp.pair0 + col) * kHidden + h0 + 4 * g;
            *reinterpret_cast<uint2*>(dst) = make_uint2(f2bf(acc[0]) | (f2bf(acc[1]) << 16),
                                                        f2bf(acc[2]) | (f2bf(acc[3]) << 16));
        }
    }
}

// Ordered combine: one workgroup per token, 8 columns per thread.
__global__ __launch_bounds__(256) void combine_kernel(ExpertArgs a) {
    const int t = blockIdx.x;
    const int c0 = threadIdx.x * 8;
    float acc[8] = {0.0f, 0.0f, 0.0f, 0.0f, 0.0f, 0.0f, 0.0f, 0.0f};
    const bool ok = *a.plan.status == 0;
    if (ok) {
        for (int r = 0; r < kTopK; ++r) {
            const int p = a.plan.route_pair[t * kTopK + r];
            const float scale = bf2f(a.weights[t * kTopK + a.plan.pair_slot[p]]);
            const uint4 v = *reinterpret_cast<const uint4*>(a.ws.y + static_cast<size_t>(p) * kHidden + c0);
            float f[8];
            unpack8(v, f);
#pragma unroll
            for (int j = 0; j < 8; ++j) acc[j] = rbf(acc[j] + rbf(f[j] * scale));
        }
        if (a.shared_down != nullptr) {
            const float gate = bf2f(a.sg[t]);
            const uint4 v = *reinterpret_cast<const uint4*>(
                a.ws.y + static_cast<size_t>(kTopK * a.tokens + t) * kHidden + c0);
            float f[8];
            unpack8(v, f);
#pragma unroll
            for (int j = 0; j < 8; ++j) acc[j] = rbf(acc[j] + rbf(gate * f[j]));
        }
    }
    if (a.residual != nullptr) {
        const uint4 v = *reinterpret_cast<const uint4*>(a.residual + static_cast<size_t>(t) * kHidden + c0);
        float f[8];
        unpack8(v, f);
#pragma unroll
        for (int j = 0; j < 8; ++j) acc[j] = rbf(f[j] + acc[j]);
    }
    uint32_t o[8];
#pragma unroll
    for (int j = 0; j < 8; ++j) o[j] = f2bf(acc[j]);
    *reinterpret_cast<uint4*>(a.out + static_cast<size_t>(t) * kHidden + c0) =
        make_uint4(o[0] | (o[1] << 16), o[2] | (o[3] << 16), o[4] | (o[5] << 16), o[6] | (o[7] << 16));
}

// ---- reference-shaped kernels (drop-in shims) -----------------------------

// fused_experts._matvec (fused_experts.py:8-24): result[e*N + r] =
// bf16(sum_k W_e[r, k] x_e[k]); W_e = table[stride*e + column] (skipped when
// zero and stride != 3); x_e = x (shared) or x + e*K.  One wave per row,
// lanes split k; K is a multiple of 512.
__global__ __launch_bounds__(256) void matvec_kernel(const int64_t* table, const uint16_t* x, uint16_t* result, int K,
                                                     int N, int column, int shared_x, int stride) {
    const int e = blockIdx.y;
    const int row = blockIdx.x * 4 + (threadIdx.x >> 6);
    const int lane = threadIdx.x & 63;
    const int64_t address = table[stride * e + column];
    if (row >= N || (stride != 3 && address == 0)) return;
    const uint16_t* w = reinterpret_cast<const uint16_t*>(address) + static_cast<size_t>(row) * K;
    const uint16_t* xe = shared_x ? x : x + static_cast<size_t>(e) * K;
    float acc = 0.0f;
    for (int k = 8 * lane; k < K; k += 8 * kWave) {
        float xf[8];
        unpack8(*reinterpret_cast<const uint4*>(xe + k), xf);
        acc = fma8(*reinterpret_cast<const uint4*>(w + k), xf, acc);
    }
    acc = wave_butterfly_sum(acc);
    if (lane == 0) result[static_cast<size_t>(e) * N + row] = static_cast<uint16_t>(f2bf(acc));
}

// fused_experts._ordered_sum (fused_experts.py:27-37) for stride 3 and
// packed_hybrid._combine (packed_hybrid.py:13-27) for stride 4 with a cold
// row in column 3 (>= 0 selects cold[row]).
__global__ __launch_bounds__(256) void ordered_sum_kernel(const int64_t* table, const uint16_t* hot, const uint16_t* cold,
                                                          const uint16_t* router, uint16_t* out, int stride) {
    const int h = blockIdx.x * blockDim.x + threadIdx.x;
    if (h >= kHidden) return;
    float acc = 0.0f;
    for (int r = 0; r < kTopK; ++r) {
        const int slot = static_cast<int>(table[stride * r + 2]);
        const int64_t cold_row = stride == 4 ? table[stride * r + 3] : -1;
        const float scale = bf2f(router[slot]);
        const float value = (cold != nullptr && cold_row >= 0) ? bf2f(cold[cold_row * kHidden + h])
                                                                : bf2f(hot[static_cast<size_t>(r) * kHidden + h]);
        acc = rbf(acc + rbf(value * scale));
    }
    out[h] = static_cast<uint16_t>(f2bf(acc));
}

// packed_ada.cu:13-40 (packed_gate_silu): active[e][r] = bf16(bf16(silu(g)) * u)
// for the 8 table rows whose gate pointer is non-zero.  One wave per row.
__global__ __launch_bounds__(256) void gate_silu_kernel(const int64_t* table, const uint16_t* hidden, uint16_t* active,
                                                        int stride) {
    const int e = blockIdx.y;
    const int row = blockIdx.x * 4 + (threadIdx.x >> 6);
    const int lane = threadIdx.x & 63;
    const int64_t address = table[stride * e];
    if (address == 0) return;
    const uint16_t* gate_row = reinterpret_cast<const uint16_t*>(address) + static_cast<size_t>(row) * kHidden;
    const uint16_t* up_row = gate_row + static_cast<size_t>(kInner) * kHidden;
    float gate = 0.0f, up = 0.0f;
    for (int k = 8 * lane; k < kHidden; k += 8 * kWave) {
        float xf[8];
        unpack8(*reinterpret_cast<const uint4*>(hidden + k), xf);
        gate = fma8(*reinterpret_cast<const uint4*>(gate_row + k), xf, gate);
        up = fma8(*reinterpret_cast<const uint4*>(up_row + k), xf, up);
    }
    gate = wave_butterfly_sum(gate);
    up = wave_butterfly_sum(up);
    if (lane == 0) active[e * kInner + row] = static_cast<uint16_t>(swiglu_bf16(rbf(gate), rbf(up)));
}

// block_experts._project (block_experts.py:12-28): per unique expert e and
// 16 route rows, Y[(e*16 + r)*OUT + c] = bf16(sum_k X[row][k] W[c][k]) with
// row = e*16 + r for the down projection, token routes[e*16 + r] otherwise;
// rows whose route is -1 read zeros.  W = pointers[2e + down].  A workgroup
// covers 64 output columns (4 waves x 16) of one expert.
__global__ __launch_bounds__(256) void project_kernel(const int64_t* pointers, const int32_t* routes, const uint16_t* X,
                                                      uint16_t* Y, int in, int out, int down) {
    const int e = blockIdx.x;
    const int wave = threadIdx.x >> 6;
    const int lane = threadIdx.x & 63;
    const int n = lane & 15;
    const int g = lane >> 4;
    const int c0 = blockIdx.y * 64 + 16 * wave;
    const uint16_t* w = reinterpret_cast<const uint16_t*>(pointers[2 * e + down]);
    const int token = routes[e * 16 + n];
    const bool live = token >= 0;
    const int input_row = down ? e * 16 + n : (live ? token : 0);
    const uint16_t* a_row = w + static_cast<size_t>(c0 + n) * in + 8 * g;
    const uint16_t* b_row = X + static_cast<size_t>(input_row) * in + 8 * g;
    f32x4 acc = {0.0f, 0.0f, 0.0f, 0.0f};
    for (int k = 0; k < in; k += 256) {
        uint4 av[8], bv[8];
#pragma unroll
        for (int s = 0; s < 8; ++s) {
            av[s] = *reinterpret_cast<const uint4*>(a_row + k + 32 * s);
            bv[s] = live ? *reinterpret_cast<const uint4*>(b_row + k + 32 * s) : zero4();
        }
#pragma unroll
        for (int s = 0; s < 8; ++s) acc = mfma16x16x32(av[s], bv[s], acc);
    }
    // D holds rows c0 + 4g + i (output columns) of route column n.
    uint16_t* dst = Y + static_cast<size_t>(e * 16 + n) * out + c0 + 4 * g;
    *reinterpret_cast<uint2*>(dst) = make_uint2(f2bf(acc[0]) | (f2bf(acc[1]) << 16), f2bf(acc[2]) | (f2bf(acc[3]) << 16));
}

// SwiGLU over [rows][1024] gate|up halves -> [rows][512] (the torch
// act_fn(gate) * up step between the two _project launches).
__global__ __launch_bounds__(256) void swiglu_rows_kernel(const uint16_t* gates, uint16_t* active, int rows) {
    const int i = blockIdx.x * blockDim.x + threadIdx.x;
    if (i >= rows * kInner) return;
    const int r = i / kInner;
    const int c = i % kInner;
    const float g = bf2f(gates[static_cast<size_t>(r) * 2 * kInner + c]);
    const float u = bf2f(gates[static_cast<size_t>(r) * 2 * kInner + kInner + c]);
    active[i] = static_cast<uint16_t>(swiglu_bf16(g, u));
}

// block_experts._combine (block_experts.py:31-49): inverse[t][r] =
// (expert, row, slot); X is [E][16][2048]; cold rows are used when hybrid and
// expert < 0.
__global__ __launch_bounds__(256) void block_combine_kernel(const int32_t* inverse, const uint16_t* X,
                                                            const uint16_t* cold, const uint16_t* router, uint16_t* out,
                                                            int hybrid) {
    const int t = blockIdx.x;
    const int h = blockIdx.y * blockDim.x + threadIdx.x;
    float acc = 0.0f;
    for (int r = 0; r < kTopK; ++r) {
        const int32_t* d = inverse + (t * kTopK + r) * 3;
        const int expert = d[0], row = d[1], slot = d[2];
        const float value = (hybrid && expert < 0) ? bf2f(cold[static_cast<size_t>(row) * kHidden + h])
                                                   : bf2f(X[(static_cast<size_t>(expert) * 16 + row) * kHidden + h]);
        const float scale = bf2f(router[t * kTopK + slot]);
        acc = rbf(acc + rbf(value * scale));
    }
    out[static_cast<size_t>(t) * kHidden + h] = static_cast<uint16_t>(f2bf(acc));
}

}  // namespace

hipError_t launch_experts(const ExpertArgs& a, hipStream_t stream) {
    if (a.tokens <= 0) return hipSuccess;
    const int max_unique = min(kTopK * a.tokens, kExperts);
    const int slots = max_unique + 1;
    const StageEvents gate_ev = timing_events(kStageGateUp);
    LRMOE_LAUNCH(gateup_kernel, dim3(slots * kGateTiles), dim3(256), 0, stream, gate_ev.start, gate_ev.stop, a);
    const StageEvents down_ev = timing_events(kStageDown);
    LRMOE_LAUNCH(down_kernel, dim3(slots * kDownTiles), dim3(256), 0, stream, down_ev.start, down_ev.stop, a);
    const StageEvents comb_ev = timing_events(kStageCombine);
    LRMOE_LAUNCH(combine_kernel, dim3(a.tokens), dim3(256), 0, stream, comb_ev.start, comb_ev.stop, a);
    return hipGetLastError();
}

hipError_t launch_matvec(const int64_t* table, const uint16_t* x, uint16_t* result, int K, int N, int column,
                         int shared_x, int stride, int experts, hipStream_t stream) {
    hipLaunchKernelGGL(matvec_kernel, dim3((N + 3) / 4, experts), dim3(256), 0, stream, table, x, result, K, N, column,
                       shared_x, stride);
    return hipGetLastError();
}

hipError_t launch_ordered_sum(const int64_t* table, const uint16_t* hot, const uint16_t* cold, const uint16_t* router,
                              uint16_t* out, int stride, hipStream_t stream) {
    hipLaunchKernelGGL(ordered_sum_kernel, dim3(kHidden / 256), dim3(256), 0, stream, table, hot, cold, router, out,
                       stride);
    return hipGetLastError();
}

hipError_t launch_gate_silu(const int64_t* table, const uint16_t* hidden, uint16_t* active, int stride, int experts,
                            hipStream_t stream) {
    hipLaunchKernelGGL(gate_silu_kernel, dim3(kInner / 4, experts), dim3(256), 0, stream, table, hidden, active, stride);
    return hipGetLastError();
}

hipError_t launch_project(const int64_t* pointers, const int32_t* routes, const uint16_t* X, uint16_t* Y, int in,
                          int out, int down, int experts, hipStream_t stream) {
    hipLaunchKernelGGL(project_kernel, dim3(experts, out / 64), dim3(256), 0, stream, pointers, routes, X, Y, in, out,
                       down);
    return hipGetLastError();
}

hipError_t launch_swiglu_rows(const uint16_t* gates, uint16_t* active, int rows, hipStream_t stream) {
    hipLaunchKernelGGL(swiglu_rows_kernel, dim3((rows * kInner + 255) / 256), dim3(256), 0, stream, gates, active, rows);
    return hipGetLastError();
}

hipError_t launch_block_combine(const int32_t* inverse, const uint16_t* X, const uint16_t* cold, const uint16_t* router,
                                uint16_t* out, int tokens, int hybrid, hipStream_t stream) {
    hipLaunchKernelGGL(block_combine_kernel, dim3(tokens, kHidden / 256), dim3(256), 0, stream, inverse, X, cold,
                       router, out, hybrid);
    return hipGetLastError();
}

}  // namespace lrmoe
