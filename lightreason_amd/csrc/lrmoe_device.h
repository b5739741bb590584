// Device-side building blocks shared by the lrmoe kernels (gfx950 only).
//
// bf16 values travel as uint16 bit patterns.  Rounding to bf16 is
// round-to-nearest-even on the fp32 bits, the same rule as
// edge35b/cpu_experts.c:18-22 (to_bfloat), so every rounding point the
// reference applies can be reproduced exactly.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

namespace lrmoe {

constexpr int kHidden = 2048;      // model hidden size
constexpr int kInner = 512;        // expert intermediate size
constexpr int kExperts = 256;      // routed experts per layer
constexpr int kTopK = 8;           // routes per token
constexpr int kWave = 64;          // CDNA wavefront width

typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef unsigned int u32x4 __attribute__((ext_vector_type(4)));

__device__ __forceinline__ float bf2f(uint32_t bits16) { return __uint_as_float(bits16 << 16); }

// bf16 bits of a float rounded to nearest even (gfx950's v_cvt_pk_bf16_f32;
// for every non-NaN input the same bits as adding 0x7fff + the kept lsb and
// truncating).
__device__ __forceinline__ uint32_t f2bf(float value) {
    return __builtin_bit_cast(uint16_t, static_cast<__bf16>(value));
}

// Two floats as one word of bf16 bits, lo in the low half (one conversion).
__device__ __forceinline__ uint32_t pack_bf2(float lo, float hi) {
    typedef __bf16 bf16x2 __attribute__((ext_vector_type(2)));
    typedef float f32x2 __attribute__((ext_vector_type(2)));
    return __builtin_bit_cast(uint32_t, __builtin_convertvector((f32x2){lo, hi}, bf16x2));
}

__device__ __forceinline__ float rbf(float value) { return bf2f(f2bf(value)); }

// Low and high bf16 halves of a packed 32-bit word, as floats.
__device__ __forceinline__ float lo_bf(uint32_t word) { return __uint_as_float(word << 16); }
__device__ __forceinline__ float hi_bf(uint32_t word) { return __uint_as_float(word & 0xffff0000u); }

// exp(x): Cody-Waite reduction x = k ln2 + r, degree-7 Taylor polynomial for
// exp(r) on |r| <= ln2/2 in Horner form, then two exact power-of-two scalings.
// x < -87 gives 0 and x > 88.72283935546875 gives +inf, so every finite result
// is a normal float.  Only IEEE mul/fma/rint are used, so the host oracle
// reproduces it bit-for-bit.
__device__ __forceinline__ float pow2i(int k) { return __uint_as_float(static_cast<uint32_t>(k + 127) << 23); }

__device__ __forceinline__ float lr_exp(float x) {
    // Branch-free: the polynomial runs on x clamped into range and the
    // special cases are selected at the end (in-range results unchanged).
    const float xc = __builtin_fminf(__builtin_fmaxf(x, -87.0f), 88.72283935546875f);
    const float k = __builtin_rintf(xc * 0x1.715476p+0f);
    float r = __builtin_fmaf(-k, 0x1.62e400p-1f, xc);
    r = __builtin_fmaf(-k, 0x1.7f7d1cp-20f, r);
    float p = 0x1.a01a02p-13f;
    p = __builtin_fmaf(p, r, 0x1.6c16c2p-10f);
    p = __builtin_fmaf(p, r, 0x1.111112p-7f);
    p = __builtin_fmaf(p, r, 0x1.555556p-5f);
    p = __builtin_fmaf(p, r, 0x1.555556p-3f);
    p = __builtin_fmaf(p, r, 0.5f);
    p = __builtin_fmaf(p, r, 1.0f);
    p = __builtin_fmaf(p, r, 1.0f);
    const int ki = static_cast<int>(k);
    const int k1 = ki / 2;
    const float e = (p * pow2i(k1)) * pow2i(ki - k1);
    const float r2 = x > 88.72283935546875f ? __builtin_inff() : (x < -87.0f ? 0.0f : e);
    // NaN passes through; selected with bit operations so that no branch
    // splits the caller's code.
    const uint32_t nan_mask = 0u - static_cast<uint32_t>(x != x);
    return __uint_as_float((__float_as_uint(x) & nan_mask) | (__float_as_uint(r2) & ~nan_mask));
}

// The expert activation with cpu_experts.c:59-62 rounding points:
// a = bf16(bf16(g / (1 + exp(-g))) * u) with g, u already bf16 values.
__device__ __forceinline__ uint32_t swiglu_bf16(float gate, float up) {
    const float silu = rbf(gate / (1.0f + lr_exp(-gate)));
    return f2bf(silu * up);
}

// Value of lane (l ^ OFF) for a full wavefront: DPP quad permutes for 1 and
// 2, swizzles inside 32-lane halves for 4, 8 and 16, a permute for 32 (no
// bounds arithmetic, which __shfl_xor adds).
template <int OFF>
__device__ __forceinline__ int lane_xor(int x) {
    if constexpr (OFF == 1) {
        return __builtin_amdgcn_update_dpp(0, x, 0xB1, 0xf, 0xf, false);  // quad_perm [1,0,3,2]
    } else if constexpr (OFF == 2) {
        return __builtin_amdgcn_update_dpp(0, x, 0x4E, 0xf, 0xf, false);  // quad_perm [2,3,0,1]
    } else if constexpr (OFF == 32) {
        return __builtin_amdgcn_ds_bpermute(static_cast<int>((__lane_id() ^ 32u) << 2), x);
    } else {
        return __builtin_amdgcn_ds_swizzle(x, 0x1F | (OFF << 10));  // bitmask mode: lane ^ OFF
    }
}

// Steps 4 and 8 of an xor butterfly, on values already equal across each
// group of 4 (resp. 8) lanes: lane i and lane 7 - i (resp. 15 - i) then hold
// the same bits as lane i ^ 4 (resp. i ^ 8), so DPP row_half_mirror and
// row_mirror bring the partner's value without an LDS round trip.
__device__ __forceinline__ float butterfly_step4(float v) {
    return v + __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), 0x141, 0xf, 0xf, false));
}
__device__ __forceinline__ float butterfly_step8(float v) {
    return v + __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), 0x140, 0xf, 0xf, false));
}

// Steps 16 and 32 of an xor butterfly with gfx950's lane-half swaps (VALU,
// no LDS round trip): v_permlane16_swap on two copies of v leaves, in every
// lane, its own value in one output and the value of lane l ^ 16 in the
// other (v_permlane32_swap: lane l ^ 32); their sum is own + partner, or
// partner + own, the same bits.
__device__ __forceinline__ float butterfly_step16(float v) {
    const int x = __float_as_int(v);
    const auto r = __builtin_amdgcn_permlane16_swap(x, x, false, false);
    return __int_as_float(r[0]) + __int_as_float(r[1]);
}
__device__ __forceinline__ float butterfly_step32(float v) {
    const int x = __float_as_int(v);
    const auto r = __builtin_amdgcn_permlane32_swap(x, x, false, false);
    return __int_as_float(r[0]) + __int_as_float(r[1]);
}

// xor butterfly over the 64 lanes with offsets 1,2,4,...,32: the fixed
// reduction order shared with the oracle for router and norm sums (every lane
// ends with the same total; each partial sum is a+b on one lane and b+a on
// its partner, the same bits).
__device__ __forceinline__ float wave_butterfly_sum(float value) {
    value = value + __int_as_float(lane_xor<1>(__float_as_int(value)));
    value = value + __int_as_float(lane_xor<2>(__float_as_int(value)));
    value = butterfly_step4(value);
    value = butterfly_step8(value);
    value = butterfly_step16(value);
    value = butterfly_step32(value);
    return value;
}

// Maximum over the wavefront, returned to every lane (a wave-uniform value):
// running maxima inside 16-lane rows (row_shr 1,2,4,8), row broadcasts of
// lanes 15 and 31, then lane 63.  The order is irrelevant for a maximum.
__device__ __forceinline__ uint32_t wave_max_u32(uint32_t v) {
    v = max(v, static_cast<uint32_t>(__builtin_amdgcn_update_dpp(0, static_cast<int>(v), 0x111, 0xf, 0xf, false)));
    v = max(v, static_cast<uint32_t>(__builtin_amdgcn_update_dpp(0, static_cast<int>(v), 0x112, 0xf, 0xf, false)));
    v = max(v, static_cast<uint32_t>(__builtin_amdgcn_update_dpp(0, static_cast<int>(v), 0x114, 0xf, 0xf, false)));
    v = max(v, static_cast<uint32_t>(__builtin_amdgcn_update_dpp(0, static_cast<int>(v), 0x118, 0xf, 0xf, false)));
    v = max(v, static_cast<uint32_t>(__builtin_amdgcn_update_dpp(0, static_cast<int>(v), 0x142, 0xa, 0xf, false)));
    v = max(v, static_cast<uint32_t>(__builtin_amdgcn_update_dpp(0, static_cast<int>(v), 0x143, 0xc, 0xf, false)));
    return static_cast<uint32_t>(__builtin_amdgcn_readlane(static_cast<int>(v), 63));
}

// N independent wave maxima with their DPP steps interleaved, so that each
// chain's wait states are filled by the others.
template <int N>
__device__ __forceinline__ void wave_max_u32_n(uint32_t* v) {
#define LR_DPP_MAX_STEP(ctrl, row_mask)                                                                            \
    _Pragma("unroll") for (int n = 0; n < N; ++n) v[n] =                                                           \
        max(v[n], static_cast<uint32_t>(__builtin_amdgcn_update_dpp(0, static_cast<int>(v[n]), ctrl, row_mask, 0xf, false)));
    LR_DPP_MAX_STEP(0x111, 0xf)
    LR_DPP_MAX_STEP(0x112, 0xf)
    LR_DPP_MAX_STEP(0x114, 0xf)
    LR_DPP_MAX_STEP(0x118, 0xf)
    LR_DPP_MAX_STEP(0x142, 0xa)
    LR_DPP_MAX_STEP(0x143, 0xc)
#undef LR_DPP_MAX_STEP
#pragma unroll
    for (int n = 0; n < N; ++n) v[n] = static_cast<uint32_t>(__builtin_amdgcn_readlane(static_cast<int>(v[n]), 63));
}

// Dot product of 8 bf16 weights (one 16-byte load) with 8 floats, as an
// in-order fmaf chain onto acc.
__device__ __forceinline__ float fma8(uint4 w, const float* x, float acc) {
    acc = __builtin_fmaf(lo_bf(w.x), x[0], acc);
    acc = __builtin_fmaf(hi_bf(w.x), x[1], acc);
    acc = __builtin_fmaf(lo_bf(w.y), x[2], acc);
    acc = __builtin_fmaf(hi_bf(w.y), x[3], acc);
    acc = __builtin_fmaf(lo_bf(w.z), x[4], acc);
    acc = __builtin_fmaf(hi_bf(w.z), x[5], acc);
    acc = __builtin_fmaf(lo_bf(w.w), x[6], acc);
    acc = __builtin_fmaf(hi_bf(w.w), x[7], acc);
    return acc;
}

// 16-byte load through an explicitly global (address space 1) pointer.  Weight
// and activation addresses read from memory are generic pointers to the
// compiler, which would otherwise emit FLAT loads; those count against the
// LDS counter too, so every LDS access would wait for all weight loads.
typedef __attribute__((address_space(1))) const u32x4 global_u32x4;

// Eight values of a codec tile (format in codec.hip): the low bytes of
// values 0..3 in `low0` and of 4..7 in `low1`, the code of value j in nibble
// j / 4 of byte j % 4 of `codes`, base4 = base * 0x01010101.  Returns the
// eight bf16 values in order (value 2i in the low half of component i).  A
// high byte is (base + (code & 7)) | (sign << 7): four at a time, one per
// byte (a value's field base + (code & 7) <= 127, so no byte carries into the
// next), then v_perm_b32 interleaves them with the low bytes (byte i of the
// result is byte sel_i of {first operand : second operand}, the second
// operand holding bytes 0..3).
__device__ __forceinline__ uint4 codec_decode8(uint32_t low0, uint32_t low1, uint32_t codes, uint32_t base4) {
    const uint32_t h0 = ((codes & 0x07070707u) + base4) | ((codes << 4) & 0x80808080u);
    const uint32_t h1 = (((codes >> 4) & 0x07070707u) + base4) | (codes & 0x80808080u);
    return make_uint4(__builtin_amdgcn_perm(h0, low0, 0x05010400u), __builtin_amdgcn_perm(h0, low0, 0x07030602u),
                      __builtin_amdgcn_perm(h1, low1, 0x05010400u), __builtin_amdgcn_perm(h1, low1, 0x07030602u));
}

// 2-byte load through a global pointer (see ldg16), zero-extended.
__device__ __forceinline__ uint32_t ldg_u16(const void* p) {
    return *reinterpret_cast<__attribute__((address_space(1))) const uint16_t*>(reinterpret_cast<uintptr_t>(p));
}

__device__ __forceinline__ uint4 ldg16(const void* p) {
    const u32x4 v = *reinterpret_cast<global_u32x4*>(reinterpret_cast<uintptr_t>(p));
    return make_uint4(v.x, v.y, v.z, v.w);
}

// 16-byte non-temporal load (global_load_dwordx4 ... nt): for weight rows
// read once per call, streamed past the caches.
__device__ __forceinline__ uint4 ldg16_nt(const void* p) {
    const u32x4 v = __builtin_nontemporal_load(reinterpret_cast<global_u32x4*>(reinterpret_cast<uintptr_t>(p)));
    return make_uint4(v.x, v.y, v.z, v.w);
}

__device__ __forceinline__ void unpack8(uint4 w, float* out) {
    out[0] = lo_bf(w.x); out[1] = hi_bf(w.x);
    out[2] = lo_bf(w.y); out[3] = hi_bf(w.y);
    out[4] = lo_bf(w.z); out[5] = hi_bf(w.z);
    out[6] = lo_bf(w.w); out[7] = hi_bf(w.w);
}

// The decoder's input RMSNorm ([HF] Qwen3_5MoeRMSNorm 801-818) of one
// 2048-element bf16 row held by a wave, lane l holding elements
// 32 l .. 32 l + 31 in v: 1 / sqrt(mean(x^2) + eps), the sum in the
// canonical order of the router and norm sums (fmaf from +0 in element
// order, then the xor butterfly over offsets 1..32), so every caller gets the
// oracle's value bit for bit.
__device__ __forceinline__ float row_rms_scale(const uint4 (&v)[4], float eps) {
    float f[32];
#pragma unroll
    for (int i = 0; i < 4; ++i) unpack8(v[i], f + 8 * i);
    float acc = 0.0f;
#pragma unroll
    for (int j = 0; j < 32; ++j) acc = __builtin_fmaf(f[j], f[j], acc);
    const float mean = wave_butterfly_sum(acc) / static_cast<float>(kHidden);
    return 1.0f / __builtin_sqrtf(mean + eps);
}

// Eight normed elements: bf16((x * r) * (1 + w)) for bf16 x and weights w.
__device__ __forceinline__ uint4 rms_apply8(uint4 x, uint4 w, float r) {
    float xf[8], wf[8];
    unpack8(x, xf);
    unpack8(w, wf);
    uint32_t o[8];
#pragma unroll
    for (int j = 0; j < 8; ++j) o[j] = f2bf((xf[j] * r) * (1.0f + wf[j]));
    return make_uint4(o[0] | (o[1] << 16), o[2] | (o[3] << 16), o[4] | (o[5] << 16), o[6] | (o[7] << 16));
}

// v_mfma_f32_16x16x32_bf16.  A is 16x32 (lane l holds row l%16, k-group l/16),
// B is 32x16 (lane l holds column l%16, the same k-group), D is 16x16 with lane
// l holding rows 4*(l/16)+i, i=0..3, of column l%16.  The k order inside a
// group is irrelevant to the result as long as A and B use the same one.
__device__ __forceinline__ f32x4 mfma16x16x32(uint4 a, uint4 b, f32x4 c) {
    return __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(bf16x8, a), __builtin_bit_cast(bf16x8, b),
                                                   c, 0, 0, 0);
}

// Orderable key for top-k: bf16 logit (with -0 folded onto +0) in the high
// 16 bits, 255 - expert id in the low 8 bits, so the maximum key is the
// largest logit and, among equal logits, the lowest expert id.
__device__ __forceinline__ uint32_t route_key(uint32_t bits, int expert) {
    if (bits == 0x8000u) bits = 0;
    const uint32_t ordered = (bits & 0x8000u) ? (~bits & 0xffffu) : (bits | 0x8000u);
    return (ordered << 8) | static_cast<uint32_t>(255 - expert);
}

__device__ __forceinline__ uint32_t key_bits(uint32_t key) {
    const uint32_t ordered = key >> 8;
    return (ordered & 0x8000u) ? (ordered & 0x7fffu) : (~ordered & 0xffffu);
}

// Top-8 of one token by one wave: lane l holds experts 4l..4l+3 as unique
// keys (bf16 logit order, then lower expert id); eight wave-wide maximum
// extractions give the winners in rank order.  Softmax over all 256 in fp32
// relative to the top logit (the per-lane sums meet in the fixed butterfly),
// then the eight probabilities are renormalised by their sum in rank order
// and rounded to bf16.  Lane k < 8 receives the expert and weight bits of
// rank k.  Same arithmetic and order as the oracle.  topk8_waves does this
// for N tokens at once, their steps interleaved.  `lane` is the caller's lane
// index (threadIdx.x % 64).
template <int N>
__device__ __forceinline__ void topk8_waves(const uint64_t* packed, int* expert, uint32_t* weight_bits, int lane) {
    uint32_t bits[N][4], k[N][4];
#pragma unroll
    for (int n = 0; n < N; ++n) {
#pragma unroll
        for (int j = 0; j < 4; ++j) {
            bits[n][j] = static_cast<uint32_t>(packed[n] >> (16 * j)) & 0xffffu;
            k[n][j] = route_key(bits[n][j], 4 * lane + j) + 1u;  // 0 marks an empty place
        }
    }
    // Each lane's keys in descending order (keys are unique): an extraction
    // then looks at one head key and shifts the lane's list when it wins.
    auto order2 = [](uint32_t& hi, uint32_t& lo) {
        const uint32_t a = max(hi, lo), b = min(hi, lo);
        hi = a;
        lo = b;
    };
#pragma unroll
    for (int n = 0; n < N; ++n) {
        order2(k[n][0], k[n][1]);
        order2(k[n][2], k[n][3]);
        order2(k[n][0], k[n][2]);
        order2(k[n][1], k[n][3]);
        order2(k[n][1], k[n][2]);
    }
    uint32_t chosen[N][kTopK];
    float part[N];
#pragma unroll
    for (int r = 0; r < kTopK; ++r) {
        uint32_t head[N];
#pragma unroll
        for (int n = 0; n < N; ++n) head[n] = k[n][0];
        wave_max_u32_n<N>(head);
#pragma unroll
        for (int n = 0; n < N; ++n) {
            chosen[n][r] = head[n];
            if (r == 0) {
                // Softmax terms relative to the top logit, computed here so
                // that they fill the extraction chains that follow.
                const float top = bf2f(key_bits(head[n] - 1u));
                part[n] = 0.0f;
#pragma unroll
                for (int j = 0; j < 4; ++j) part[n] = part[n] + lr_exp(bf2f(bits[n][j]) - top);
            }
            const bool won = k[n][0] == head[n];
            k[n][0] = won ? k[n][1] : k[n][0];
            k[n][1] = won ? k[n][2] : k[n][1];
            k[n][2] = won ? k[n][3] : k[n][2];
            k[n][3] = won ? 0u : k[n][3];
        }
    }
#pragma unroll
    for (int n = 0; n < N; ++n) {
        const float top = bf2f(key_bits(chosen[n][0] - 1u));
        const float total = wave_butterfly_sum(part[n]);
        uint32_t my = chosen[n][0];
#pragma unroll
        for (int r = 1; r < kTopK; ++r) my = lane == r ? chosen[n][r] : my;
        const float prob = lr_exp(bf2f(key_bits(my - 1u)) - top) / total;
        float sum = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(prob), 0));
#pragma unroll
        for (int r = 1; r < kTopK; ++r) sum = sum + __int_as_float(__builtin_amdgcn_readlane(__float_as_int(prob), r));
        expert[n] = 255 - static_cast<int>((my - 1u) & 255u);
        weight_bits[n] = f2bf(prob / sum);
    }
}

__device__ __forceinline__ void topk8_wave(uint64_t packed, int& expert, uint32_t& weight_bits, int lane) {
    topk8_waves<1>(&packed, &expert, &weight_bits, lane);
}

// Exclusive scan over threads 0..255 (all threads call, tid = threadIdx.x;
// others contribute 0).
__device__ __forceinline__ uint32_t block_scan256(uint32_t value, uint32_t* scratch, uint32_t* total, int tid) {
    const int wave = tid >> 6;
    const int lane = tid & 63;
    if (tid >= kExperts) value = 0;
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
    return tid < kExperts ? before + inclusive - value : 0u;
}

// ---- agent-scope memory operations (coherent across the XCDs' L2s) -----------
//
// Rows that one workgroup writes and a workgroup of the same launch on
// another XCD reads go through these: agent-scope (sc1) stores and loads.

typedef __attribute__((address_space(1))) uint64_t g_u64;
typedef __attribute__((address_space(1))) uint32_t g_u32;

__device__ __forceinline__ g_u64* as_g64(const void* p) {
    return reinterpret_cast<g_u64*>(reinterpret_cast<uintptr_t>(p));
}
__device__ __forceinline__ g_u32* as_g32(const void* p) {
    return reinterpret_cast<g_u32*>(reinterpret_cast<uintptr_t>(p));
}
__device__ __forceinline__ void st_agent64(void* p, uint64_t v) {
    __hip_atomic_store(as_g64(p), v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ uint64_t ld_agent64(const void* p) {
    return __hip_atomic_load(as_g64(p), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ void st_agent32(void* p, uint32_t v) {
    __hip_atomic_store(as_g32(p), v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ uint32_t ld_agent32(const void* p) {
    return __hip_atomic_load(as_g32(p), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

// 16 bytes at base + byte_offset with an agent-scope (sc1) buffer load from a
// raw buffer of `bytes` bytes at base: a load at or past the end reads zeros
// and touches no memory (the buffer's range check), so callers need no
// branch around it.
__device__ __forceinline__ uint4 ld_agent16(const void* base, uint32_t byte_offset, uint32_t bytes = 0x7fffffffu) {
    // dword 3 = gfx9 untyped 32-bit data format
    const __amdgpu_buffer_rsrc_t rsrc =
        __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(base), 0, static_cast<int>(bytes), 0x00020000);
    constexpr int kSc1 = 16;  // cache policy: sc1 (agent scope)
    const u32x4 v = __builtin_amdgcn_raw_buffer_load_b128(rsrc, static_cast<int>(byte_offset), 0, kSc1);
    return make_uint4(v.x, v.y, v.z, v.w);
}

// A wave-uniform copy of a 64-bit value (each half through readfirstlane,
// whose int result is taken as unsigned before widening).
__device__ __forceinline__ uint64_t uniform64(uint64_t v) {
    const uint32_t lo = static_cast<uint32_t>(__builtin_amdgcn_readfirstlane(static_cast<int>(static_cast<uint32_t>(v))));
    const uint32_t hi = static_cast<uint32_t>(__builtin_amdgcn_readfirstlane(static_cast<int>(static_cast<uint32_t>(v >> 32))));
    return static_cast<uint64_t>(lo) | (static_cast<uint64_t>(hi) << 32);
}

}  // namespace lrmoe
