// The decoder layer's glue around its mixer (the Gated DeltaNet mixer or
// the full attention) for T <= 16 tokens: the input RMSNorm before the mixer
// ([HF] Qwen3_5MoeDecoderLayer: input_layernorm, Qwen3_5MoeRMSNorm 801-818)
// and the residual add after it ([HF] 866: hidden = residual + mixer_out).
// One wave per token row: lane l holds elements 32 l .. 32 l + 31, the
// canonical order of the router and norm sums (fmaf from +0 in element
// order, then the xor butterfly over offsets 1..32), so the normalised rows
// are the oracle's bit for bit.
#include "lrmoe_device.h"
#include "lrmoe_internal.h"

namespace lrmoe {
namespace {

__global__ __launch_bounds__(kWave) void add_rmsnorm_kernel(const uint16_t* x, const uint16_t* add,
                                                             const uint16_t* norm, float eps, uint16_t* sum_out,
                                                             uint16_t* norm_out) {
    const int t = blockIdx.x;
    const int lane = threadIdx.x;
    const size_t at = static_cast<size_t>(t) * kHidden + 32 * lane;
    // every load at once: the row, the addend and the norm weights (one
    // round trip; dummy addresses where a pointer is null)
    uint4 v[4], bv[4], w[4];
    const uint16_t* add_row = add != nullptr ? add + at : x + at;
    const uint16_t* w_row = (norm != nullptr ? norm : x) + 32 * lane;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        v[i] = ldg16(x + at + 8 * i);
        bv[i] = ldg16(add_row + 8 * i);
        w[i] = ldg16(w_row + 8 * i);
    }
    if (add != nullptr) {
        // bf16(x + add) elementwise, the bf16 tensor add of the residual
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            const uint4 b = bv[i];
            float xf[8], bf[8];
            unpack8(v[i], xf);
            unpack8(b, bf);
            uint32_t o[8];
#pragma unroll
            for (int j = 0; j < 8; ++j) o[j] = f2bf(xf[j] + bf[j]);
            v[i] = make_uint4(o[0] | (o[1] << 16), o[2] | (o[3] << 16), o[4] | (o[5] << 16), o[6] | (o[7] << 16));
        }
    }
    if (sum_out != nullptr) {
#pragma unroll
        for (int i = 0; i < 4; ++i) *reinterpret_cast<uint4*>(sum_out + at + 8 * i) = v[i];
    }
    if (norm == nullptr) return;
    const float r = row_rms_scale(v, eps);
#pragma unroll
    for (int i = 0; i < 4; ++i) *reinterpret_cast<uint4*>(norm_out + at + 8 * i) = rms_apply8(v[i], w[i], r);
}

}  // namespace

hipError_t launch_add_rmsnorm(const uint16_t* x, const uint16_t* add, int tokens, const uint16_t* norm, float eps,
                              uint16_t* sum_out, uint16_t* norm_out, hipStream_t stream) {
    hipLaunchKernelGGL(add_rmsnorm_kernel, dim3(tokens), dim3(kWave), 0, stream, x, add, norm, eps, sum_out, norm_out);
    return hipGetLastError();
}

}  // namespace lrmoe
