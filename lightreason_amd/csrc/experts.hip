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
// The grouped expert GEMMs of a prefill live in prefill.hip; this file holds
// the ordered combine that follows them and the reference-shaped kernels.
#include "lrmoe_device.h"
#include "lrmoe_internal.h"

namespace lrmoe {
namespace {

__device__ __forceinline__ uint4 zero4() { return make_uint4(0, 0, 0, 0); }

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
    *reinterpret_cast<uint2*>(dst) = make_uint2(pack_bf2(acc[0], acc[1]), pack_bf2(acc[2], acc[3]));
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
    const hipError_t err = launch_prefill_experts(a, stream);
    if (err != hipSuccess) return err;
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
