// Decode / verify expert kernels (T <= 16 tokens, so at most 16 tokens per
// expert: one MFMA column block).
//
// gateup_decode: one wavefront per (expert, 16-row tile) streams the tile's
// 16 gate rows and 16 up rows over the full k = 2048 straight into MFMA A
// operands, eight k-steps of loads in flight ahead of the MFMAs; every token
// routed to the expert is a B column, so each weight byte is read once per
// call however many tokens share the expert.  The epilogue applies the
// cpu_experts.c:59-62 rounding points (bf16 gate/up, bf16 SiLU, bf16 product).
//
// down_combine_decode: one workgroup per 16 output rows owns those rows for
// every routed expert and the shared expert, so the ordered combine
// (fused_experts.py:27-37, block_experts.py:31-49: per token, ascending expert
// order, acc = bf16(acc + bf16(y * w)) from 0), the shared-expert add
// (bf16(sg * y_shared)) and the residual add finish inside the workgroup with
// no cross-workgroup synchronisation.
#include "lrmoe_device.h"
#include "lrmoe_internal.h"

namespace lrmoe {
namespace {

constexpr int kRowTiles = kInner / 16;   // 32 gate/up row tiles per expert
constexpr int kDepth = 8;                // k-steps of loads in flight per wave (of 16)
constexpr int kDownRows = 16;            // output rows per down workgroup
constexpr int kDownWaves = 8;            // 512 threads
constexpr int kActStride = kInner + 8;   // LDS act row stride (bf16), 16-byte pad
constexpr int kDecodeTokens = 16;
constexpr int kDecodeSlots = kTopK * kDecodeTokens + 1;  // unique routed experts + the shared expert
// Dynamic LDS of down_combine_decode at its largest (T = 16): 144 act rows.
constexpr int kMaxActLds = (kTopK + 1) * kDecodeTokens * kActStride * 2;

__device__ __forceinline__ uint4 zero4() { return make_uint4(0, 0, 0, 0); }

// Token of MFMA column n from a slot record's 16 packed token bytes.
__device__ __forceinline__ int column_token(const uint4 packed, int n) {
    const uint32_t word = n < 4 ? packed.x : n < 8 ? packed.y : n < 12 ? packed.z : packed.w;
    return static_cast<int>((word >> (8 * (n & 3))) & 0xffu);
}

// One workgroup per (slot, 16-row tile): wave w covers k in [512w, 512w+512)
// with kDepth k-steps of gate, up and x loads in flight; the four partial
// tiles meet in LDS in wave order.
__global__ __launch_bounds__(256) void gateup_decode(ExpertArgs a) {
    const int wave = threadIdx.x >> 6;
    const int lane = threadIdx.x & 63;
    const int slot = blockIdx.x / kRowTiles;
    const int row0 = (blockIdx.x % kRowTiles) * 16;
    // The record and the unique count are independent loads, issued together.
    const SlotDesc d = a.ws.slots[slot];
    const int unique = *a.plan.unique;
    if (slot > unique || !d.valid) return;
    __shared__ f32x4 red[4][2][kWave];
    const int n = lane & 15;
    const int g = lane >> 4;
    const bool live = n < d.count;
    // Columns past the slot's token count read token 0's row: an MFMA output
    // column depends only on its own B column, and those columns are dropped.
    const int token = column_token(*reinterpret_cast<const uint4*>(d.tokens), n);
    const int kb = wave * (kHidden / 4) + 8 * g;
    const uint16_t* gp = d.gate_up + static_cast<size_t>(row0 + n) * kHidden + kb;
    const uint16_t* up = d.up + static_cast<size_t>(row0 + n) * kHidden + kb;
    const uint16_t* xp = a.x + static_cast<size_t>(token) * kHidden + kb;

    constexpr int kSteps = kHidden / 32 / 4;
    uint4 ga[kDepth], ua[kDepth], xb[kDepth];
#pragma unroll
    for (int s = 0; s < kDepth; ++s) {
        ga[s] = ldg16(gp + 32 * s);
        ua[s] = ldg16(up + 32 * s);
        xb[s] = ldg16(xp + 32 * s);
    }
    // Keep the scheduler from sinking the prefetch next to its MFMAs.
    __builtin_amdgcn_sched_barrier(0);
    f32x4 acc_g = {0.0f, 0.0f, 0.0f, 0.0f};
    f32x4 acc_u = {0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
    for (int s0 = 0; s0 < kSteps; s0 += kDepth) {
#pragma unroll
        for (int j = 0; j < kDepth; ++j) {
            acc_g = mfma16x16x32(ga[j], xb[j], acc_g);
            acc_u = mfma16x16x32(ua[j], xb[j], acc_u);
            const int next = s0 + kDepth + j;
            if (next < kSteps) {
                ga[j] = ldg16(gp + 32 * next);
                ua[j] = ldg16(up + 32 * next);
                xb[j] = ldg16(xp + 32 * next);
            }
            __builtin_amdgcn_sched_barrier(0);
        }
    }
    red[wave][0][lane] = acc_g;
    red[wave][1][lane] = acc_u;
    __syncthreads();
    if (wave != 0 || !live) return;
    const f32x4 sg = ((red[0][0][lane] + red[1][0][lane]) + red[2][0][lane]) + red[3][0][lane];
    const f32x4 su = ((red[0][1][lane] + red[1][1][lane]) + red[2][1][lane]) + red[3][1][lane];
    uint32_t act[4];
#pragma unroll
    for (int i = 0; i < 4; ++i) act[i] = swiglu_bf16(rbf(sg[i]), rbf(su[i]));
    uint16_t* dst = a.ws.act + static_cast<size_t>(d.pair0 + n) * kInner + row0 + 4 * g;
    *reinterpret_cast<uint2*>(dst) = make_uint2(act[0] | (act[1] << 16), act[2] | (act[3] << 16));
}

// One workgroup per 16 output rows; wave w takes slots w, w+8, ...  The slot
// records and the act rows of every pair (the B operand) are staged into LDS
// once; each wave keeps the next slot's 16 down-weight loads in flight while
// the current slot's MFMAs run.
__global__ __launch_bounds__(kDownWaves * kWave) void down_combine_decode(ExpertArgs a) {
    extern __shared__ __attribute__((aligned(16))) uint16_t act_lds[];  // [9T][kActStride]
    __shared__ uint16_t ys[(kTopK + 1) * 16 * kDownRows];              // y bits of this tile
    __shared__ SlotDesc descs[kDecodeSlots];
    const int wave = threadIdx.x >> 6;
    const int lane = threadIdx.x & 63;
    const int n = lane & 15;
    const int g = lane >> 4;
    const int h0 = blockIdx.x * kDownRows;
    const int T = a.tokens;
    const int32_t status = *a.plan.status;
    const int unique = status ? 0 : *a.plan.unique;
    const int slots = unique + 1;

    for (int i = threadIdx.x; i < slots * 4; i += blockDim.x) {
        reinterpret_cast<uint4*>(descs)[i] = reinterpret_cast<const uint4*>(a.ws.slots)[i];
    }
    // All staging loads are issued before any LDS write, so their latencies
    // overlap (at T = 16: 18 loads per thread).
    const int chunks = (kTopK + 1) * T * (kInner / 8);
    constexpr int kStageIters = (kTopK + 1) * kDecodeTokens * (kInner / 8) / (kDownWaves * kWave);
    uint4 staged[kStageIters];
#pragma unroll
    for (int k = 0; k < kStageIters; ++k) {
        const int i = threadIdx.x + k * kDownWaves * kWave;
        if (i < chunks) staged[k] = ldg16(a.ws.act + static_cast<size_t>(i) * 8);
    }
#pragma unroll
    for (int k = 0; k < kStageIters; ++k) {
        const int i = threadIdx.x + k * kDownWaves * kWave;
        if (i < chunks) {
            const int r = i / (kInner / 8);
            const int c = (i % (kInner / 8)) * 8;
            *reinterpret_cast<uint4*>(act_lds + r * kActStride + c) = staged[k];
        }
    }
    __syncthreads();

    // Two register buffers alternate roles (no copies, so a prefetch is only
    // waited for when its expert is computed).
    auto next_valid = [&](int from) {
        while (from < slots && !descs[from].valid) from += kDownWaves;
        return from;
    };
    auto load = [&](int slot, uint4* buf) {
        const uint16_t* wp = descs[slot].down + static_cast<size_t>(h0 + n) * kInner + 8 * g;
#pragma unroll
        for (int s = 0; s < 16; ++s) buf[s] = ldg16(wp + 32 * s);
    };
    auto compute = [&](int slot, const uint4* buf) {
        const int pair0 = descs[slot].pair0;
        const bool live = n < descs[slot].count;
        // Dropped columns (n >= count) read the slot's first row instead.
        const uint16_t* bp = act_lds + (pair0 + (live ? n : 0)) * kActStride + 8 * g;
        f32x4 acc = {0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
        for (int s = 0; s < 16; ++s) acc = mfma16x16x32(buf[s], *reinterpret_cast<const uint4*>(bp + 32 * s), acc);
        if (live) {
            uint16_t* dst = ys + (pair0 + n) * kDownRows + 4 * g;
#pragma unroll
            for (int i = 0; i < 4; ++i) dst[i] = static_cast<uint16_t>(f2bf(acc[i]));
        }
    };
    // Prefetches are unconditional so the compiler can count outstanding
    // loads; past the wave's last slot they re-read the slot just computed,
    // which is still in L2.
    uint4 buf0[16], buf1[16];
    int s0 = next_valid(wave);
    if (s0 < slots) {
        load(s0, buf0);
        int s1 = next_valid(s0 + kDownWaves);
        while (true) {
            load(s1 < slots ? s1 : s0, buf1);
            compute(s0, buf0);
            if (s1 >= slots) break;
            s0 = next_valid(s1 + kDownWaves);
            load(s0 < slots ? s0 : s1, buf0);
            compute(s1, buf1);
            if (s0 >= slots) break;
            s1 = next_valid(s0 + kDownWaves);
        }
    }
    __syncthreads();

    if (static_cast<int>(threadIdx.x) >= T * kDownRows) return;
    const int t = threadIdx.x / kDownRows;
    const int r = threadIdx.x % kDownRows;
    float acc = 0.0f;
    if (status == 0) {
        for (int k = 0; k < kTopK; ++k) {
            const int p = a.plan.route_pair[t * kTopK + k];
            const float scale = bf2f(a.weights[t * kTopK + a.plan.pair_slot[p]]);
            acc = rbf(acc + rbf(bf2f(ys[p * kDownRows + r]) * scale));
        }
        if (a.shared_down != nullptr) {
            const float shared = bf2f(ys[(kTopK * T + t) * kDownRows + r]);
            acc = rbf(acc + rbf(bf2f(a.sg[t]) * shared));
        }
    }
    const size_t o = static_cast<size_t>(t) * kHidden + h0 + r;
    if (a.residual != nullptr) acc = rbf(bf2f(a.residual[o]) + acc);
    a.out[o] = static_cast<uint16_t>(f2bf(acc));
}

}  // namespace

hipError_t launch_experts_decode(const ExpertArgs& a, hipStream_t stream) {
    const int slots = min(kTopK * a.tokens, kExperts) + 1;
    const StageEvents gate_ev = timing_events(kStageGateUp);
    LRMOE_LAUNCH(gateup_decode, dim3(slots * kRowTiles), dim3(256), 0, stream, gate_ev.start, gate_ev.stop, a);
    const size_t act_bytes = static_cast<size_t>(kTopK + 1) * a.tokens * kActStride * sizeof(uint16_t);
    static bool lds_opt_in = false;
    if (!lds_opt_in) {
        const hipError_t err = hipFuncSetAttribute(reinterpret_cast<const void*>(down_combine_decode),
                                                   hipFuncAttributeMaxDynamicSharedMemorySize, kMaxActLds);
        if (err != hipSuccess) return err;
        lds_opt_in = true;
    }
    const StageEvents down_ev = timing_events(kStageDown);
    LRMOE_LAUNCH(down_combine_decode, dim3(kHidden / kDownRows), dim3(kDownWaves * kWave), act_bytes, stream,
                 down_ev.start, down_ev.stop, a);
    return hipGetLastError();
}

}  // namespace lrmoe
