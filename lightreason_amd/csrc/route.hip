// Router (softmax/top-k/renormalise) and route bucketing kernels.
//
// Semantics follow the Transformers Qwen3_5MoeTopKRouter.forward that the
// reference patches around (modeling_qwen3_5_moe.py, called from
// SparseMoeBlock.forward; edge35b/expert_stream.py:383-454 receives its
// top_k_index / top_k_weights), and the reference's bucketing:
// edge35b/fused_experts.py:47-54 (routes sorted by expert),
// edge35b/block_experts.py:102-121 (experts ascending, tokens ascending,
// inverse map per token), edge35b/pipeline.py:59-76.
//
// Router logits use one fixed fp32 reduction order so that indices are
// reproducible bit-for-bit: lane l of a wave owns the 32 contiguous elements
// [32l, 32l+32) of the 2048-long dot product and accumulates them in order
// with fmaf from +0, then the 64 partials meet in an xor butterfly with
// offsets 1,2,4,...,32.  Top-k ranks by (bf16 logit desc, expert id asc).
#include "lrmoe_device.h"
#include "lrmoe_internal.h"

namespace lrmoe {
namespace {

constexpr int kTokTile = 16;     // tokens per router workgroup
constexpr int kXStride = kHidden + 8;  // LDS row stride in bf16 (16-byte pad)

// Stage up to 16 token rows of the router input into LDS, applying the
// RMSNorm (x * r) * (1 + w) with r = 1/sqrt(sum(x^2)/2048 + eps) when `norm`
// is given.  One wave per token; lane l owns elements [32l, 32l+32).
__device__ void stage_tokens(uint16_t* xs, const uint16_t* x, const uint16_t* norm, float eps, int t0, int count,
                             uint16_t* normed_out) {
    const int wave = threadIdx.x >> 6;
    const int lane = threadIdx.x & 63;
    for (int t = wave; t < count; t += 4) {
        const uint4* src = reinterpret_cast<const uint4*>(x + static_cast<size_t>(t0 + t) * kHidden + 32 * lane);
        uint4 v[4];
#pragma unroll
        for (int i = 0; i < 4; ++i) v[i] = src[i];
        if (norm != nullptr) {
            float f[32];
#pragma unroll
            for (int i = 0; i < 4; ++i) unpack8(v[i], f + 8 * i);
            float acc = 0.0f;
#pragma unroll
            for (int j = 0; j < 32; ++j) acc = __builtin_fmaf(f[j], f[j], acc);
            const float mean = wave_butterfly_sum(acc) / static_cast<float>(kHidden);
            const float r = 1.0f / __builtin_sqrtf(mean + eps);
            const uint4* wsrc = reinterpret_cast<const uint4*>(norm + 32 * lane);
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                const uint4 w = wsrc[i];
                float wf[8];
                unpack8(w, wf);
                uint32_t o[8];
#pragma unroll
                for (int j = 0; j < 8; ++j) o[j] = f2bf((f[8 * i + j] * r) * (1.0f + wf[j]));
                v[i] = make_uint4(o[0] | (o[1] << 16), o[2] | (o[3] << 16), o[4] | (o[5] << 16), o[6] | (o[7] << 16));
            }
            if (normed_out != nullptr) {
                uint4* dst = reinterpret_cast<uint4*>(normed_out + static_cast<size_t>(t0 + t) * kHidden + 32 * lane);
#pragma unroll
                for (int i = 0; i < 4; ++i) dst[i] = v[i];
            }
        }
        uint4* dst = reinterpret_cast<uint4*>(xs + t * kXStride + 32 * lane);
#pragma unroll
        for (int i = 0; i < 4; ++i) dst[i] = v[i];
    }
}

// Fixed-order dot of this lane's 32 weights with token row `t` in LDS.
__device__ __forceinline__ float lane_dot(const float* w, const uint16_t* xs, int t, int lane) {
    const uint4* row = reinterpret_cast<const uint4*>(xs + t * kXStride + 32 * lane);
    float acc = 0.0f;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        float xf[8];
        unpack8(row[i], xf);
#pragma unroll
        for (int j = 0; j < 8; ++j) acc = __builtin_fmaf(w[8 * i + j], xf[j], acc);
    }
    return acc;
}

// Exclusive scan of one value per thread over threads 0..255 of a workgroup
// of >= 256 threads (every thread must call it; values of threads >= 256 are
// ignored and get 0).  `total` receives the sum over threads 0..255.
__device__ uint32_t scan256(uint32_t value, uint32_t* scratch, uint32_t* total) {
    const int wave = threadIdx.x >> 6;
    const int lane = threadIdx.x & 63;
    if (threadIdx.x >= kExperts) value = 0;
    uint32_t inclusive = value;
#pragma unroll
    for (int offset = 1; offset < kWave; offset <<= 1) {
        const uint32_t up = static_cast<uint32_t>(__shfl_up(static_cast<int>(inclusive), offset, kWave));
        if (lane >= offset) inclusive += up;
    }
    if (lane == kWave - 1 && wave < 4) scratch[wave] = inclusive;
    __syncthreads();
    uint32_t before = 0;
    for (int w = 0; w < wave && w < 4; ++w) before += scratch[w];
    *total = scratch[0] + scratch[1] + scratch[2] + scratch[3];
    __syncthreads();
    return threadIdx.x < kExperts ? before + inclusive - value : 0u;
}

// Bucket <= 64 tokens held in LDS (ids[t*8 + r], already validated) with one
// 256-thread workgroup: a token bitmap per expert (one LDS atomic per route),
// a block scan for pair offsets and unique ranks, then every route places
// itself in O(1).
__device__ void build_plan_small(const int32_t* ids, int tokens, const Plan& plan) {
    __shared__ unsigned long long tokmask[kExperts];
    __shared__ uint32_t poff[kExperts];
    __shared__ uint32_t scan_scratch[4];
    const int e = threadIdx.x;
    if (e < kExperts) tokmask[e] = 0ull;
    __syncthreads();
    for (int i = threadIdx.x; i < tokens * kTopK; i += blockDim.x) atomicOr(&tokmask[ids[i]], 1ull << (i / kTopK));
    __syncthreads();
    const unsigned long long mask = e < kExperts ? tokmask[e] : 0ull;
    const uint32_t count = static_cast<uint32_t>(__popcll(mask));
    // One scan of (unique flag << 16 | count): counts are <= 64 and pairs <= 512.
    uint32_t packed_total = 0;
    const uint32_t packed = scan256((count ? (1u << 16) : 0u) | count, scan_scratch, &packed_total);
    const uint32_t pair_offset = packed & 0xffffu;
    const uint32_t rank = packed >> 16;
    const uint32_t pairs_total = packed_total & 0xffffu;
    const uint32_t unique_total = packed_total >> 16;
    if (e < kExperts) poff[e] = pair_offset;
    if (count) {
        plan.expert[rank] = e;
        plan.offset[rank] = static_cast<int32_t>(pair_offset);
        unsigned long long m = mask;
        for (int j = 0; m; ++j) {
            const int t = __ffsll(static_cast<long long>(m)) - 1;
            m &= m - 1ull;
            plan.pair_token[pair_offset + j] = t;
        }
    }
    if (e == 0) {
        plan.offset[unique_total] = static_cast<int32_t>(pairs_total);
        *plan.unique = static_cast<int32_t>(unique_total);
    }
    __syncthreads();
    for (int i = threadIdx.x; i < tokens * kTopK; i += blockDim.x) {
        const int t = i / kTopK;
        const int r = i % kTopK;
        const int ex = ids[i];
        const int p = static_cast<int>(poff[ex]) + __popcll(tokmask[ex] & ((1ull << t) - 1ull));
        plan.pair_slot[p] = r;
        int order = 0;
        for (int q = 0; q < kTopK; ++q) order += (ids[t * kTopK + q] < ex) ? 1 : 0;
        plan.route_pair[t * kTopK + order] = p;
    }
}

// Checks ids and returns the status bits for the whole set.
__device__ int32_t validate_ids(const int32_t* ids, int tokens) {
    __shared__ int32_t flags;
    if (threadIdx.x == 0) flags = 0;
    __syncthreads();
    int32_t mine = 0;
    for (int i = threadIdx.x; i < tokens * kTopK; i += blockDim.x) {
        const int e = ids[i];
        if (e < 0 || e >= kExperts) mine |= kStatusBadExpert;
        const int t = i / kTopK;
        for (int q = t * kTopK; q < i; ++q) mine |= (ids[q] == e) ? kStatusRepeatedExpert : 0;
    }
    if (mine) atomicOr(&flags, mine);
    __syncthreads();
    return flags;
}

// Router logits for a tile of <= 16 tokens: 4*RPW router rows per workgroup
// (RPW rows per wave).  With SHARED_ROW the last blockIdx.y instead computes
// the shared-expert gate for the tile (wave 0).  PREFILL also clears the
// bucketing histogram for the top-k kernel that follows on the stream.  No
// workgroup waits on another: the kernel boundary publishes the logits.
template <bool PREFILL, int RPW>
__global__ __launch_bounds__(256) void router_logits(RouteArgs a) {
    __shared__ __attribute__((aligned(16))) uint16_t xs[kTokTile * kXStride];
    const int wave = threadIdx.x >> 6;
    const int lane = threadIdx.x & 63;
    const int t0 = blockIdx.x * kTokTile;
    const int count = min(kTokTile, a.tokens - t0);
    constexpr int kRowGroups = kExperts / (4 * RPW);

    if (PREFILL && blockIdx.x == 0 && blockIdx.y == 0) {
        if (threadIdx.x == 0) *a.plan.status = 0;
    }

    // Issue this wave's weight loads before staging the tokens.
    const bool shared_row = blockIdx.y == kRowGroups;
    const bool router_rows = !shared_row && a.router != nullptr;
    const bool gate_row = shared_row && a.shared_gate != nullptr;
    uint4 wraw[RPW][4];
    if (router_rows) {
#pragma unroll
        for (int i = 0; i < RPW; ++i) {
            const int row = (blockIdx.y * 4 + wave) * RPW + i;
            const uint4* src = reinterpret_cast<const uint4*>(a.router + static_cast<size_t>(row) * kHidden + 32 * lane);
#pragma unroll
            for (int q = 0; q < 4; ++q) wraw[i][q] = src[q];
        }
    } else if (gate_row) {
        const uint4* src = reinterpret_cast<const uint4*>(a.shared_gate + 32 * lane);
#pragma unroll
        for (int q = 0; q < 4; ++q) wraw[0][q] = src[q];
    }

    if (router_rows || gate_row || (blockIdx.y == 0 && a.norm != nullptr)) {
        stage_tokens(xs, a.x, a.norm, a.eps, t0, count, blockIdx.y == 0 ? a.normed : nullptr);
    }
    __syncthreads();

    if (router_rows) {
#pragma unroll
        for (int i = 0; i < RPW; ++i) {
            const int row = (blockIdx.y * 4 + wave) * RPW + i;
            float w[32];
#pragma unroll
            for (int q = 0; q < 4; ++q) unpack8(wraw[i][q], w + 8 * q);
            for (int t = 0; t < count; ++t) {
                const float s = wave_butterfly_sum(lane_dot(w, xs, t, lane));
                if (lane == 0) a.logits[static_cast<size_t>(t0 + t) * kExperts + row] = static_cast<uint16_t>(f2bf(s));
            }
        }
    } else if (gate_row && wave == 0) {
        float w[32];
#pragma unroll
        for (int q = 0; q < 4; ++q) unpack8(wraw[0][q], w + 8 * q);
        for (int t = 0; t < count; ++t) {
            const float z = rbf(wave_butterfly_sum(lane_dot(w, xs, t, lane)));
            if (lane == 0) a.sg[t0 + t] = static_cast<uint16_t>(f2bf(1.0f / (1.0f + lr_exp(-z))));
        }
    }
}

// Top-8 of one token by ballot radix selection.  Lane l holds the logits of
// experts 4l..4l+3 as unique 24-bit keys; the 8th largest key is found bit by
// bit from the top with wave-wide counts.  The eight winners land in LDS with
// their exp() terms (already computed for the softmax denominator), lane k < 8
// ranks entry k, and probabilities and weights take one divide per lane.
// Indices, weights and the LDS expert row are written in rank order.
// Arithmetic and order match topk_token (and the oracle) exactly.
__device__ void topk_token_select(uint64_t packed, int64_t* indices_row, uint16_t* weights_row, int32_t* ids_row,
                                  uint32_t* keys8, float* vals8) {
    const int lane = threadIdx.x & 63;
    uint32_t bits[4], keys[4];
#pragma unroll
    for (int j = 0; j < 4; ++j) {
        bits[j] = static_cast<uint32_t>(packed >> (16 * j)) & 0xffffu;
        keys[j] = route_key(bits[j], 4 * lane + j);
    }
    uint32_t best = keys[0];
#pragma unroll
    for (int j = 1; j < 4; ++j) best = keys[j] > best ? keys[j] : best;
    best = wave_max_u32(best);
    uint32_t threshold = 0;
#pragma unroll 1
    for (int bit = 23; bit >= 0; --bit) {
        const uint32_t candidate = threshold | (1u << bit);
        int above = 0;
#pragma unroll
        for (int j = 0; j < 4; ++j) above += __popcll(__ballot(keys[j] >= candidate));
        if (above >= kTopK) threshold = candidate;
    }
    // Softmax terms of this lane's four experts, relative to the top logit.
    const float top = bf2f(key_bits(best));
    float ex[4];
#pragma unroll
    for (int j = 0; j < 4; ++j) ex[j] = lr_exp(bf2f(bits[j]) - top);
    float part = 0.0f;
#pragma unroll
    for (int j = 0; j < 4; ++j) part = part + ex[j];
    const float total = wave_butterfly_sum(part);
    // Exactly eight keys are >= threshold (keys are unique); compact them.
    int base = 0;
#pragma unroll
    for (int j = 0; j < 4; ++j) {
        const bool chosen = keys[j] >= threshold;
        const uint64_t mask = __ballot(chosen);
        if (chosen) {
            const int at = base + __popcll(mask & ((1ull << lane) - 1ull));
            keys8[at] = keys[j];
            vals8[at] = ex[j];
        }
        base += __popcll(mask);
    }
    // LDS accesses of one wave execute in order: the reads see the writes.
    __builtin_amdgcn_wave_barrier();
    const int k = lane & 7;
    const uint32_t my_key = keys8[k];
    int rank = 0;
#pragma unroll
    for (int i = 0; i < kTopK; ++i) rank += keys8[i] > my_key ? 1 : 0;
    const float prob = vals8[k] / total;
    __builtin_amdgcn_wave_barrier();
    if (lane < kTopK) vals8[rank] = prob;
    __builtin_amdgcn_wave_barrier();
    float sum = vals8[0];
#pragma unroll
    for (int i = 1; i < kTopK; ++i) sum = sum + vals8[i];
    const int expert = 255 - static_cast<int>(my_key & 255u);
    if (lane < kTopK) {
        indices_row[rank] = expert;
        weights_row[rank] = static_cast<uint16_t>(f2bf(prob / sum));
        ids_row[rank] = expert;
    }
}

// Decode routing tail in one workgroup of 16 waves (T <= 16): wave t runs
// the top-k of token t (from the router's logits or the caller's) and its
// shared-expert gate; then the workgroup builds the bucketing plan and the
// decode slot records.
__global__ __launch_bounds__(1024) void topk_bucket_small(RouteArgs a) {
    __shared__ int32_t ids[kTokTile * kTopK];
    __shared__ uint32_t keys8[kTokTile][kTopK];
    __shared__ float vals8[kTokTile][kTopK];
    const int t = threadIdx.x >> 6;
    const int lane = threadIdx.x & 63;
    const uint16_t* logits = a.logits_in != nullptr ? a.logits_in : a.logits;
    if (t < a.tokens) {
        // Issue every load of this wave first: its logits row, and the
        // shared-gate weights and token row.
        const uint64_t packed = reinterpret_cast<const uint64_t*>(logits + static_cast<size_t>(t) * kExperts)[lane];
        const bool gate = a.shared_gate != nullptr;
        uint4 wsg[4], xrow[4];
        if (gate) {
            const uint16_t* x = a.norm != nullptr ? a.normed : a.x;
            const uint4* src = reinterpret_cast<const uint4*>(a.shared_gate + 32 * lane);
            const uint4* row = reinterpret_cast<const uint4*>(x + static_cast<size_t>(t) * kHidden + 32 * lane);
#pragma unroll
            for (int q = 0; q < 4; ++q) {
                wsg[q] = src[q];
                xrow[q] = row[q];
            }
        }
        topk_token_select(packed, a.indices + t * kTopK, a.weights + t * kTopK, ids + t * kTopK, keys8[t], vals8[t]);
        if (gate) {
            float acc = 0.0f;
#pragma unroll
            for (int q = 0; q < 4; ++q) {
                float w[8], xf[8];
                unpack8(wsg[q], w);
                unpack8(xrow[q], xf);
#pragma unroll
                for (int j = 0; j < 8; ++j) acc = __builtin_fmaf(w[j], xf[j], acc);
            }
            const float z = rbf(wave_butterfly_sum(acc));
            if (lane == 0) a.sg[t] = static_cast<uint16_t>(f2bf(1.0f / (1.0f + lr_exp(-z))));
        }
    }
    __syncthreads();
    build_plan_small(ids, a.tokens, a.plan);
    if (threadIdx.x == 0) *a.plan.status = 0;
}

// Standalone bucketing of <= 64 caller-provided tokens in one workgroup.
__global__ __launch_bounds__(256) void bucket_small_kernel(const int64_t* indices, int tokens, Plan plan) {
    __shared__ int32_t ids[64 * kTopK];
    for (int i = threadIdx.x; i < tokens * kTopK; i += blockDim.x) {
        const int64_t e = indices[i];
        ids[i] = (e < 0 || e >= kExperts) ? -1 : static_cast<int32_t>(e);
    }
    __syncthreads();
    const int32_t status = validate_ids(ids, tokens);
    if (status) {
        if (threadIdx.x == 0) {
            *plan.status = status;
            *plan.unique = 0;
            plan.offset[0] = 0;
        }
        for (int i = threadIdx.x; i < tokens * kTopK; i += blockDim.x) plan.route_pair[i] = -1;
        return;
    }
    build_plan_small(ids, tokens, plan);
    if (threadIdx.x == 0) *plan.status = 0;
}

}  // namespace

hipError_t launch_route(const RouteArgs& a, hipStream_t stream) {
    if (a.tokens <= 0) return hipSuccess;
    const StageEvents ev = timing_events(kStageRoute);
    if (a.tokens <= kTokTile) {
        // Decode: router GEMV (one row per wave, 64 workgroups; skipped when
        // logits are given), then top-k + shared gate + bucketing in one
        // workgroup.
        hipEvent_t start = ev.start;
        if (a.router != nullptr || a.norm != nullptr) {
            LRMOE_LAUNCH((router_logits<false, 1>), dim3(1, kExperts / 4), dim3(256), 0, stream, start, nullptr, a);
            start = nullptr;
        }
        LRMOE_LAUNCH(topk_bucket_small, dim3(1), dim3(1024), 0, stream, start, ev.stop, a);
        return hipGetLastError();
    }
    const int tiles = (a.tokens + kTokTile - 1) / kTokTile;
    LRMOE_LAUNCH((router_logits<true, 4>), dim3(tiles, kExperts / 16 + 1), dim3(256), 0, stream, ev.start, nullptr, a);
    const hipError_t err = launch_prefill_plan(a.logits_in != nullptr ? a.logits_in : a.logits, nullptr, nullptr,
                                               a.indices, a.weights, a.tokens, a.shared_down != nullptr, a.ws, a.plan,
                                               stream);
    if (err != hipSuccess) return err;
    if (ev.stop != nullptr) return hipEventRecord(ev.stop, stream);
    return hipGetLastError();
}

hipError_t launch_bucket(const int64_t* indices, int tokens, const Workspace& ws, const Plan& plan, hipStream_t stream) {
    if (tokens <= 0) return hipSuccess;
    if (tokens <= 64) {
        hipLaunchKernelGGL(bucket_small_kernel, dim3(1), dim3(256), 0, stream, indices, tokens, plan);
        return hipGetLastError();
    }
    return launch_prefill_plan(nullptr, indices, nullptr, nullptr, nullptr, tokens, false, ws, plan, stream);
}

}  // namespace lrmoe
