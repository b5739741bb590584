/*
 * lro.c -- CPU oracle for the MoE expert-layer hot path.
 *
 * TEST INFRASTRUCTURE ONLY.  Nothing in the product (lightreason_amd/) links,
 * loads or calls this file; only tests/, __graft_entry__.smoke() and the
 * cpu_baseline leg of bench.py use it, and only as the checker.
 *
 * It restates, in plain C with explicit fmaf() and no FP contraction, the
 * arithmetic the reference performs on this path:
 *
 *   - expert SwiGLU arithmetic and its bf16 rounding points:
 *       edge35b/cpu_experts.c:11-22 (from_bfloat / to_bfloat),
 *       :29-41 (dot: two 8-lane FMA accumulators, then add + hadd tree),
 *       :43-71 (expert_rows), :74-105 (expert_block_rows);
 *   - the ordered bf16 combine: edge35b/fused_experts.py:27-37 (_ordered_sum),
 *       edge35b/block_experts.py:31-49 (_combine), edge35b/cpu_route.py:66-68;
 *   - route bucketing: edge35b/fused_experts.py:47-54 (T=1 schedule),
 *       edge35b/block_experts.py:102-121 (experts ascending, tokens ascending,
 *       inverse map per token in ascending-expert order);
 *   - the router, shared expert, shared gate and RMSNorm of the third-party
 *       Transformers Qwen3_5Moe classes the reference patches
 *       (modeling_qwen3_5_moe.py: TopKRouter.forward, MLP.forward,
 *       SparseMoeBlock.forward, RMSNorm.forward), called from
 *       edge35b/expert_stream.py:383-454;
 *   - the Gated DeltaNet decode step (edge35b/delta_decode.py and the
 *       Transformers Qwen3_5MoeGatedDeltaNet it patches) and the
 *       full-attention decode step (Transformers Qwen3_5MoeAttention with
 *       eager_attention_forward, which the reference runs stock).
 *
 * The router GEMV, the softmax denominator and the RMSNorm sum of squares use
 * one fixed fp32 reduction order (64 lane partials over contiguous chunks,
 * then an xor butterfly with offsets 1,2,4,8,16,32) so that routing indices
 * can be reproduced bit-exactly by the HIP kernels.  Top-k ties break toward
 * the lower expert id.  exp() for softmax/sigmoid is lro_exp (Cody-Waite
 * reduction plus a degree-7 Taylor polynomial), reproducible bit-for-bit on the
 * device; the expert SiLU keeps libm expf, exactly as cpu_experts.c does.
 *
 * Build: oracle/Makefile (gcc -O3 -mavx2 -mfma -ffp-contract=off).
 */
#include <math.h>
#include <stdint.h>
#include <stdlib.h>
#include <string.h>

#define LRO_HIDDEN 2048
#define LRO_INNER 512
#define LRO_EXPERTS 256
#define LRO_TOPK 8

/* ---- bf16 helpers: cpu_experts.c:11-22 ---------------------------------- */

float lro_bf16_value(uint16_t value) {
    uint32_t bits = (uint32_t)value << 16;
    float result;
    memcpy(&result, &bits, sizeof(result));
    return result;
}

uint16_t lro_bf16_round(float value) {
    uint32_t bits;
    memcpy(&bits, &value, sizeof(bits));
    return (uint16_t)((bits + 0x7fffu + ((bits >> 16) & 1u)) >> 16);
}

static inline float rbf(float value) { return lro_bf16_value(lro_bf16_round(value)); }

/* ---- exp(): Cody-Waite reduction + degree-7 Taylor polynomial ------------ */
/* x = k ln2 + r with k = rint(x log2 e); exp(r) by Horner on |r| <= ln2/2;
 * result = p * 2^k applied as two exact power-of-two scalings.  Inputs below
 * -87 return 0 and above 88.72283935546875 return +inf so every finite result
 * is a normal float and no step depends on denormal handling. */
static const float LRO_LOG2E = 0x1.715476p+0f;
static const float LRO_LN2_HI = 0x1.62e400p-1f;
static const float LRO_LN2_LO = 0x1.7f7d1cp-20f;
static const float LRO_C7 = 0x1.a01a02p-13f; /* 1/5040 */
static const float LRO_C6 = 0x1.6c16c2p-10f; /* 1/720 */
static const float LRO_C5 = 0x1.111112p-7f;  /* 1/120 */
static const float LRO_C4 = 0x1.555556p-5f;  /* 1/24 */
static const float LRO_C3 = 0x1.555556p-3f;  /* 1/6 */

static inline float pow2i(int k) {
    uint32_t bits = (uint32_t)(k + 127) << 23;
    float result;
    memcpy(&result, &bits, sizeof(result));
    return result;
}

float lro_exp(float x) {
    if (x != x) return x;
    if (x > 88.72283935546875f) return INFINITY;
    if (x < -87.0f) return 0.0f;
    float k = rintf(x * LRO_LOG2E);
    float r = fmaf(-k, LRO_LN2_HI, x);
    r = fmaf(-k, LRO_LN2_LO, r);
    float p = LRO_C7;
    p = fmaf(p, r, LRO_C6);
    p = fmaf(p, r, LRO_C5);
    p = fmaf(p, r, LRO_C4);
    p = fmaf(p, r, LRO_C3);
    p = fmaf(p, r, 0.5f);
    p = fmaf(p, r, 1.0f);
    p = fmaf(p, r, 1.0f);
    int ki = (int)k;
    int k1 = ki / 2;
    int k2 = ki - k1;
    return (p * pow2i(k1)) * pow2i(k2);
}

/* ---- synthetic generator ------------------------------------------------ */
/* Counter-based: h = splitmix64(key + index), key = splitmix64(seed * phi +
 * stream).  Irwin-Hall sum of the four 16-bit fields of h, centred and scaled
 * to unit variance in double, times sigma, rounded to float then bf16 (RNE). */
static inline uint64_t splitmix64(uint64_t z) {
    z += 0x9E3779B97F4A7C15ull;
    z = (z ^ (z >> 30)) * 0xBF58476D1CE4E5B9ull;
    z = (z ^ (z >> 27)) * 0x94D049BB133111EBull;
    return z ^ (z >> 31);
}

void lro_fill_normal_bf16(uint16_t *out, int64_t count, uint64_t seed, uint64_t stream,
                          double sigma, int64_t first) {
    const uint64_t key = splitmix64(seed * 0x9E3779B97F4A7C15ull + stream);
    const double inv_std = 1.0 / sqrt(1431655765.0);
    for (int64_t i = 0; i < count; ++i) {
        uint64_t h = splitmix64(key + (uint64_t)(first + i));
        int64_t s = (int64_t)(h & 0xffff) + (int64_t)((h >> 16) & 0xffff) +
                    (int64_t)((h >> 32) & 0xffff) + (int64_t)(h >> 48);
        double z = ((double)s - 131070.0) * inv_std;
        out[i] = lro_bf16_round((float)(z * sigma));
    }
}

/* ---- expert arithmetic: cpu_experts.c:29-105 ---------------------------- */

/* cpu_experts.c:29-41: low/high 8-lane FMA accumulators over 16-element
 * steps, lanes = low + high, (lanes[0:4] + lanes[4:8]), then two hadds. */
float lro_expert_dot(const uint16_t *weights, const float *input, int width) {
    float low[8] = {0}, high[8] = {0};
    for (int i = 0; i < width; i += 16) {
        for (int j = 0; j < 8; ++j) {
            low[j] = fmaf(lro_bf16_value(weights[i + j]), input[i + j], low[j]);
            high[j] = fmaf(lro_bf16_value(weights[i + 8 + j]), input[i + 8 + j], high[j]);
        }
    }
    float lanes[8];
    for (int j = 0; j < 8; ++j) lanes[j] = low[j] + high[j];
    float s[4];
    for (int j = 0; j < 4; ++j) s[j] = lanes[j] + lanes[j + 4];
    return (s[0] + s[1]) + (s[2] + s[3]);
}

/* One (expert, token) pair: cpu_experts.c:54-69 for a single expert.  gate and
 * up are the two [512, 2048] halves (for routed experts up = gate + 512*2048),
 * down is [2048, 512]; x is the token as floats; y receives 2048 bf16. */
void lro_expert_pair(const uint16_t *gate, const uint16_t *up, const uint16_t *down,
                     const float *x, uint16_t *y) {
    float active[LRO_INNER];
    for (int row = 0; row < LRO_INNER; ++row) {
        float g = rbf(lro_expert_dot(gate + (size_t)row * LRO_HIDDEN, x, LRO_HIDDEN));
        float u = rbf(lro_expert_dot(up + (size_t)row * LRO_HIDDEN, x, LRO_HIDDEN));
        float silu = rbf(g / (1.0f + expf(-g)));
        active[row] = rbf(silu * u);
    }
    for (int row = 0; row < LRO_HIDDEN; ++row) {
        y[row] = lro_bf16_round(lro_expert_dot(down + (size_t)row * LRO_INNER, active, LRO_INNER));
    }
}

static void to_floats(const uint16_t *x, float *out, int n) {
    for (int i = 0; i < n; ++i) out[i] = lro_bf16_value(x[i]);
}

/* cpu_experts.c:43-71 (single-threaded restatement). */
void lro_expert_rows(const uint16_t *const *gate_up, const uint16_t *const *down,
                     const uint16_t *input, uint16_t *output, int experts) {
    float hidden[LRO_HIDDEN];
    to_floats(input, hidden, LRO_HIDDEN);
    for (int e = 0; e < experts; ++e) {
        lro_expert_pair(gate_up[e], gate_up[e] + (size_t)LRO_INNER * LRO_HIDDEN, down[e], hidden,
                        output + (size_t)e * LRO_HIDDEN);
    }
}

/* cpu_experts.c:74-105: row i uses input token token_ids[i]. */
void lro_expert_block_rows(const uint16_t *const *gate_up, const uint16_t *const *down,
                           const uint16_t *input, const int32_t *token_ids, uint16_t *output,
                           int tokens, int experts) {
    float *hidden = (float *)malloc(sizeof(float) * (size_t)tokens * LRO_HIDDEN);
    for (int t = 0; t < tokens; ++t) to_floats(input + (size_t)t * LRO_HIDDEN, hidden + (size_t)t * LRO_HIDDEN, LRO_HIDDEN);
    for (int e = 0; e < experts; ++e) {
        lro_expert_pair(gate_up[e], gate_up[e] + (size_t)LRO_INNER * LRO_HIDDEN, down[e],
                        hidden + (size_t)token_ids[e] * LRO_HIDDEN, output + (size_t)e * LRO_HIDDEN);
    }
    free(hidden);
}

/* ---- fixed-order reductions (router, shared gate, RMSNorm) -------------- */

static float butterfly64(float *p) {
    for (int offset = 1; offset < 64; offset <<= 1) {
        float q[64];
        for (int l = 0; l < 64; ++l) q[l] = p[l] + p[l ^ offset];
        memcpy(p, q, sizeof(q));
    }
    return p[0];
}

/* Lane l of 64 owns elements [l*K/64, (l+1)*K/64) and accumulates them in
 * ascending order with fmaf from +0; lane partials meet in butterfly64. */
float lro_canon_dot(const uint16_t *weights, const float *x, int width) {
    float p[64];
    const int chunk = width / 64;
    for (int l = 0; l < 64; ++l) {
        float acc = 0.0f;
        for (int j = 0; j < chunk; ++j) acc = fmaf(lro_bf16_value(weights[l * chunk + j]), x[l * chunk + j], acc);
        p[l] = acc;
    }
    return butterfly64(p);
}

/* Orderable 24-bit key: bf16 value (with -0 folded onto +0), then lower id. */
static uint32_t route_key(uint16_t bits, int expert) {
    if (bits == 0x8000) bits = 0;
    uint32_t ordered = (bits & 0x8000) ? (uint32_t)(~bits & 0xffff) : (uint32_t)(bits | 0x8000);
    return (ordered << 8) | (uint32_t)(255 - expert);
}

/* Top-8 of one token's bf16 router logits, [HF] Qwen3_5MoeTopKRouter.forward
 * 768-777 after the GEMV: softmax in fp32 over 256 experts, top-8 by (logit
 * desc, id asc), renormalised over the 8 in fp32 (sequential sum in rank
 * order), weights rounded to bf16.  Indices are written in rank order, like
 * torch.topk(sorted=True).  softmax is monotonic, so ranking the logits ranks
 * the probabilities; its sum runs over 64 partials of 4 terms, then a
 * butterfly (the device order). */
static void topk_token(const uint16_t *logits, int64_t *indices, uint16_t *weights) {
    float value[LRO_EXPERTS];
    for (int e = 0; e < LRO_EXPERTS; ++e) value[e] = lro_bf16_value(logits[e]);
    int chosen[LRO_TOPK];
    uint8_t taken[LRO_EXPERTS] = {0};
    for (int k = 0; k < LRO_TOPK; ++k) {
        uint32_t best = 0;
        int best_e = -1;
        for (int e = 0; e < LRO_EXPERTS; ++e) {
            if (taken[e]) continue;
            uint32_t key = route_key(logits[e], e);
            if (best_e < 0 || key > best) {
                best = key;
                best_e = e;
            }
        }
        taken[best_e] = 1;
        chosen[k] = best_e;
    }
    const float top = value[chosen[0]];
    float expo[LRO_EXPERTS];
    for (int e = 0; e < LRO_EXPERTS; ++e) expo[e] = lro_exp(value[e] - top);
    float p[64];
    for (int l = 0; l < 64; ++l) {
        float acc = 0.0f;
        for (int j = 0; j < 4; ++j) acc = acc + expo[4 * l + j];
        p[l] = acc;
    }
    const float total = butterfly64(p);
    float prob[LRO_TOPK];
    for (int k = 0; k < LRO_TOPK; ++k) prob[k] = expo[chosen[k]] / total;
    float sum = prob[0];
    for (int k = 1; k < LRO_TOPK; ++k) sum = sum + prob[k];
    for (int k = 0; k < LRO_TOPK; ++k) {
        indices[k] = chosen[k];
        weights[k] = lro_bf16_round(prob[k] / sum);
    }
}

/* Router for one token: logits = bf16(x . Wr^T) (fixed order), then
 * topk_token. */
static void route_token(const float *x, const uint16_t *router, uint16_t *logits,
                        int64_t *indices, uint16_t *weights) {
    for (int e = 0; e < LRO_EXPERTS; ++e) {
        logits[e] = lro_bf16_round(lro_canon_dot(router + (size_t)e * LRO_HIDDEN, x, LRO_HIDDEN));
    }
    topk_token(logits, indices, weights);
}

/* Top-8 on caller logits [tokens, 256] (the decode kernel's logits_in path). */
void lro_route_logits(const uint16_t *logits, int tokens, int64_t *indices, uint16_t *weights) {
    for (int t = 0; t < tokens; ++t) {
        topk_token(logits + (size_t)t * LRO_EXPERTS, indices + (size_t)t * LRO_TOPK, weights + (size_t)t * LRO_TOPK);
    }
}

void lro_route(const uint16_t *x, const uint16_t *router, int tokens, uint16_t *logits,
               int64_t *indices, uint16_t *weights) {
    float hidden[LRO_HIDDEN];
    for (int t = 0; t < tokens; ++t) {
        to_floats(x + (size_t)t * LRO_HIDDEN, hidden, LRO_HIDDEN);
        route_token(hidden, router, logits + (size_t)t * LRO_EXPERTS, indices + (size_t)t * LRO_TOPK,
                    weights + (size_t)t * LRO_TOPK);
    }
}

/* Shared-expert gate: sg = bf16(sigmoid(bf16(x . w_sg))) with the fixed
 * reduction order and lro_exp. */
void lro_shared_gate(const uint16_t *x, const uint16_t *gate_weight, int tokens, uint16_t *out) {
    float hidden[LRO_HIDDEN];
    for (int t = 0; t < tokens; ++t) {
        to_floats(x + (size_t)t * LRO_HIDDEN, hidden, LRO_HIDDEN);
        float z = rbf(lro_canon_dot(gate_weight, hidden, LRO_HIDDEN));
        out[t] = lro_bf16_round(1.0f / (1.0f + lro_exp(-z)));
    }
}

/* RMSNorm with the (1 + w) scale: n = bf16((x * r) * (1 + w)),
 * r = 1 / sqrt(sum(x^2)/H + eps), sum(x^2) in the fixed order. */
void lro_rmsnorm(const uint16_t *x, const uint16_t *weight, int tokens, float eps, uint16_t *out) {
    float hidden[LRO_HIDDEN];
    for (int t = 0; t < tokens; ++t) {
        to_floats(x + (size_t)t * LRO_HIDDEN, hidden, LRO_HIDDEN);
        float p[64];
        for (int l = 0; l < 64; ++l) {
            float acc = 0.0f;
            for (int j = 0; j < LRO_HIDDEN / 64; ++j) {
                float v = hidden[l * (LRO_HIDDEN / 64) + j];
                acc = fmaf(v, v, acc);
            }
            p[l] = acc;
        }
        float mean = butterfly64(p) / (float)LRO_HIDDEN;
        float r = 1.0f / sqrtf(mean + eps);
        for (int i = 0; i < LRO_HIDDEN; ++i) {
            out[(size_t)t * LRO_HIDDEN + i] =
                lro_bf16_round((hidden[i] * r) * (1.0f + lro_bf16_value(weight[i])));
        }
    }
}

/* ---- bucketing ---------------------------------------------------------- */
/* Unique experts ascending; per expert its (token, slot) pairs in ascending
 * token order; route_pair[t*8 + r] = pair index of token t's r-th route in
 * ascending-expert order.  Returns the unique count, or -1 for an
 * out-of-range id, -2 for a token that repeats an expert. */
int lro_bucket(const int64_t *indices, int tokens, int32_t *expert, int32_t *offset,
               int32_t *pair_token, int32_t *pair_slot, int32_t *route_pair) {
    int32_t count[LRO_EXPERTS] = {0};
    for (int t = 0; t < tokens; ++t) {
        for (int r = 0; r < LRO_TOPK; ++r) {
            int64_t e = indices[t * LRO_TOPK + r];
            if (e < 0 || e >= LRO_EXPERTS) return -1;
            for (int q = 0; q < r; ++q) {
                if (indices[t * LRO_TOPK + q] == e) return -2;
            }
            count[e] += 1;
        }
    }
    int32_t start[LRO_EXPERTS];
    int unique = 0, pairs = 0;
    for (int e = 0; e < LRO_EXPERTS; ++e) {
        start[e] = pairs;
        if (count[e]) {
            expert[unique] = e;
            offset[unique] = pairs;
            ++unique;
        }
        pairs += count[e];
    }
    offset[unique] = pairs;
    int32_t fill[LRO_EXPERTS];
    memcpy(fill, start, sizeof(fill));
    for (int t = 0; t < tokens; ++t) {
        int32_t order[LRO_TOPK];
        for (int r = 0; r < LRO_TOPK; ++r) order[r] = r;
        for (int i = 1; i < LRO_TOPK; ++i) {
            for (int j = i; j > 0 && indices[t * LRO_TOPK + order[j - 1]] > indices[t * LRO_TOPK + order[j]]; --j) {
                int32_t tmp = order[j];
                order[j] = order[j - 1];
                order[j - 1] = tmp;
            }
        }
        for (int r = 0; r < LRO_TOPK; ++r) {
            int slot = order[r];
            int e = (int)indices[t * LRO_TOPK + slot];
            int p = fill[e]++;
            pair_token[p] = t;
            pair_slot[p] = slot;
            route_pair[t * LRO_TOPK + r] = p;
        }
    }
    return unique;
}

/* ---- combine: fused_experts.py:27-37, block_experts.py:31-49 ------------ */
/* out[t] = bf16 sum over token t's routes in ascending expert order of
 * bf16(y[pair] * w[t, slot]), starting from 0, rounding after each multiply
 * and add; then out = bf16(out + bf16(sg[t] * y_shared[t])) when y_shared is
 * given (SparseMoeBlock.forward), then out = bf16(residual[t] + out) when a
 * residual is given (decoder-layer residual add). */
void lro_combine(const uint16_t *y, const int32_t *route_pair, const int32_t *pair_slot,
                 const uint16_t *weights, const uint16_t *y_shared, const uint16_t *shared_gate,
                 const uint16_t *residual, int tokens, uint16_t *out) {
    for (int t = 0; t < tokens; ++t) {
        for (int h = 0; h < LRO_HIDDEN; ++h) {
            float acc = 0.0f;
            for (int r = 0; r < LRO_TOPK; ++r) {
                int p = route_pair[t * LRO_TOPK + r];
                float scale = lro_bf16_value(weights[t * LRO_TOPK + pair_slot[p]]);
                float value = lro_bf16_value(y[(size_t)p * LRO_HIDDEN + h]);
                acc = rbf(acc + rbf(value * scale));
            }
            if (y_shared) {
                float s = rbf(lro_bf16_value(shared_gate[t]) * lro_bf16_value(y_shared[(size_t)t * LRO_HIDDEN + h]));
                acc = rbf(acc + s);
            }
            if (residual) acc = rbf(lro_bf16_value(residual[(size_t)t * LRO_HIDDEN + h]) + acc);
            out[(size_t)t * LRO_HIDDEN + h] = lro_bf16_round(acc);
        }
    }
}

/* ---- a whole MoE layer for a set of tokens ------------------------------ */
/* x: [tokens, 2048] (the layer input h when norm_weight is given, else the
 * MoE input).  gate_up/down: 256 per-expert pointers.  The shared expert is
 * (shared_gate_proj, shared_up_proj [512,2048], shared_down [2048,512],
 * shared_expert_gate [2048]); pass shared_down == NULL for a routed-only
 * layer.  With norm_weight: n = RMSNorm(h), out = bf16(h + MoE(n)). */
void lro_moe_layer(const uint16_t *x, int tokens, const uint16_t *router,
                   const uint16_t *const *gate_up, const uint16_t *const *down,
                   const uint16_t *shared_gate_proj, const uint16_t *shared_up_proj,
                   const uint16_t *shared_down, const uint16_t *shared_expert_gate,
                   const uint16_t *norm_weight, float eps, uint16_t *out, int64_t *indices_out,
                   uint16_t *weights_out) {
    const size_t H = LRO_HIDDEN;
    uint16_t *normed = NULL;
    const uint16_t *input = x;
    if (norm_weight) {
        normed = (uint16_t *)malloc(sizeof(uint16_t) * tokens * H);
        lro_rmsnorm(x, norm_weight, tokens, eps, normed);
        input = normed;
    }
    uint16_t *logits = (uint16_t *)malloc(sizeof(uint16_t) * tokens * LRO_EXPERTS);
    lro_route(input, router, tokens, logits, indices_out, weights_out);
    int32_t expert[LRO_EXPERTS], offset[LRO_EXPERTS + 1];
    int32_t *pair_token = (int32_t *)malloc(sizeof(int32_t) * tokens * LRO_TOPK);
    int32_t *pair_slot = (int32_t *)malloc(sizeof(int32_t) * tokens * LRO_TOPK);
    int32_t *route_pair = (int32_t *)malloc(sizeof(int32_t) * tokens * LRO_TOPK);
    int unique = lro_bucket(indices_out, tokens, expert, offset, pair_token, pair_slot, route_pair);
    uint16_t *y = (uint16_t *)malloc(sizeof(uint16_t) * tokens * LRO_TOPK * H);
    float *hidden = (float *)malloc(sizeof(float) * tokens * H);
    for (int t = 0; t < tokens; ++t) to_floats(input + t * H, hidden + t * H, (int)H);
    for (int u = 0; u < unique; ++u) {
        const uint16_t *gu = gate_up[expert[u]];
        for (int p = offset[u]; p < offset[u + 1]; ++p) {
            lro_expert_pair(gu, gu + (size_t)LRO_INNER * H, down[expert[u]], hidden + pair_token[p] * H, y + p * H);
        }
    }
    uint16_t *y_shared = NULL, *sg = NULL;
    if (shared_down) {
        y_shared = (uint16_t *)malloc(sizeof(uint16_t) * tokens * H);
        sg = (uint16_t *)malloc(sizeof(uint16_t) * tokens);
        for (int t = 0; t < tokens; ++t) {
            lro_expert_pair(shared_gate_proj, shared_up_proj, shared_down, hidden + t * H, y_shared + t * H);
        }
        lro_shared_gate(input, shared_expert_gate, tokens, sg);
    }
    lro_combine(y, route_pair, pair_slot, weights_out, y_shared, sg, norm_weight ? x : NULL, tokens, out);
    free(y_shared);
    free(sg);
    free(hidden);
    free(y);
    free(route_pair);
    free(pair_slot);
    free(pair_token);
    free(logits);
    free(normed);
}

/* ---- lossless BF16 tile codec, in the decode kernel's layout ----------------
 *
 * Format of edge35b/cpu_bf16_reads.h:16-52 (pack_cpu_read_tiles) and
 * bf16_gather_ada.cu:117-123 (unpack_cpu_tile_pair): a row is cut into tiles
 * of 256 values.  base = the smallest 7-bit field (bits 14..8) of the tile's
 * values; a tile whose fields span more than 8 values does not fit (base 255,
 * the reference's raw marker).  Each value keeps its low byte (bits 7..0) and
 * the 4-bit code (field - base) | (sign << 3).
 *
 * Byte order (the decode kernel's MFMA lane mapping; the reference stores
 * values in index order): value k = 8g + 32s + j of a tile (g 0..3, s 0..7,
 * j 0..7) has its low byte at LRO_CODEC_LOW(g, s, j) = 64(s/2) + 16g +
 * 8(s%2) + j and its code in the nibble j/4 (low nibble first) of byte
 * LRO_CODEC_CODE(g, s, j) = 256 + 64(s/4) + 16g + 4(s%4) + j%4.  The six
 * 16-byte blocks of a k-group g then sit at 16g + 64i (i = 0..5), and those of
 * the next tile continue at 16g + 64i for i = 6..11.  A tile is 384 bytes; the
 * base of tile t of row r is bases[r * (cols / 256) + t].
 */
#define LRO_CODEC_LOW(g, s, j) (64 * ((s) >> 1) + 16 * (g) + 8 * ((s) & 1) + (j))
#define LRO_CODEC_CODE(g, s, j) (256 + 64 * ((s) >> 2) + 16 * (g) + 4 * ((s) & 3) + ((j) & 3))
#define LRO_CODEC_TILE 256
#define LRO_CODEC_TILE_BYTES 384

int64_t lro_codec_pack(const uint16_t *w, int64_t rows, int cols, uint8_t *packed, uint8_t *bases) {
    const int tiles = cols / LRO_CODEC_TILE;
    int64_t misfit = 0;
    for (int64_t r = 0; r < rows; ++r) {
        for (int t = 0; t < tiles; ++t) {
            const uint16_t *v = w + r * cols + (int64_t)t * LRO_CODEC_TILE;
            uint8_t *out = packed + (r * tiles + t) * LRO_CODEC_TILE_BYTES;
            int low = 127, high = 0;
            for (int k = 0; k < LRO_CODEC_TILE; ++k) {
                const int field = (v[k] >> 8) & 127;
                if (field < low) low = field;
                if (field > high) high = field;
            }
            memset(out, 0, LRO_CODEC_TILE_BYTES);
            if (high - low > 7) {
                bases[r * tiles + t] = 255;
                ++misfit;
                continue;
            }
            bases[r * tiles + t] = (uint8_t)low;
            for (int k = 0; k < LRO_CODEC_TILE; ++k) {
                const int g = (k >> 3) & 3, s = k >> 5, j = k & 7;
                const int code = (((v[k] >> 8) & 127) - low) | ((v[k] >> 15) << 3);
                out[LRO_CODEC_LOW(g, s, j)] = (uint8_t)(v[k] & 255);
                out[LRO_CODEC_CODE(g, s, j)] |= (uint8_t)(code << (4 * (j >> 2)));
            }
        }
    }
    return misfit;
}

/* Inverse of lro_codec_pack for tiles that fit; a tile with base 255 decodes
 * to 0xffff in every position. */
void lro_codec_unpack(const uint8_t *packed, const uint8_t *bases, int64_t rows, int cols, uint16_t *w) {
    const int tiles = cols / LRO_CODEC_TILE;
    for (int64_t r = 0; r < rows; ++r) {
        for (int t = 0; t < tiles; ++t) {
            const uint8_t *in = packed + (r * tiles + t) * LRO_CODEC_TILE_BYTES;
            const int base = bases[r * tiles + t];
            uint16_t *v = w + r * cols + (int64_t)t * LRO_CODEC_TILE;
            for (int k = 0; k < LRO_CODEC_TILE; ++k) {
                if (base == 255) {
                    v[k] = 0xffff;
                    continue;
                }
                const int g = (k >> 3) & 3, s = k >> 5, j = k & 7;
                const int code = (in[LRO_CODEC_CODE(g, s, j)] >> (4 * (j >> 2))) & 15;
                const int high = (base + (code & 7)) | ((code & 8) << 4);
                v[k] = (uint16_t)((high << 8) | in[LRO_CODEC_LOW(g, s, j)]);
            }
        }
    }
}

/* ---- Gated DeltaNet decode ---------------------------------------------------
 *
 * The single-step linear-attention mixer of the 35B runner's Gated DeltaNet
 * layers ([HF] Qwen3_5MoeGatedDeltaNet.forward 430-543 with a cached state)
 * with the recurrence of edge35b/delta_decode.py:11-36 (_delta: one token at
 * a time, the state rounded to the cache dtype after every token).  Floating
 * point throughout: sums run in ascending index order in fp32. */

/* [HF] l2norm 243-247 on a bf16 vector: every op rounds to bf16 (x*x, the
 * sum, + eps, rsqrt, x * inv). */
static void l2norm_bf16(const uint16_t *x, int n, float *out) {
    float sum = 0.0f;
    for (int i = 0; i < n; ++i) {
        float v = lro_bf16_value(x[i]);
        sum += rbf(v * v);
    }
    float s = rbf(rbf(sum) + 1e-6f);
    float inv = rbf(1.0f / sqrtf(s));
    for (int i = 0; i < n; ++i) out[i] = rbf(lro_bf16_value(x[i]) * inv);
}

static float state_get(const void *s, int bf16, size_t i) {
    return bf16 ? lro_bf16_value(((const uint16_t *)s)[i]) : ((const float *)s)[i];
}

static void state_put(void *s, int bf16, size_t i, float v) {
    if (bf16) ((uint16_t *)s)[i] = lro_bf16_round(v);
    else ((float *)s)[i] = v;
}

/* The gated delta rule over T tokens and H heads (edge35b/delta_decode.py:
 * 11-36 _delta, 38-55 _run): q, k [T][H][D] bf16; v [T][H][E] bf16;
 * G [T][H] fp32 (= exp(g)); beta [T][H] bf16; state_in [H][D][E] (fp32, or
 * bf16 when state_bf16).  normalize: q and k through l2norm first.  Per
 * token and head: state *= G; mem[e] = sum_d state[d][e] k[d]; delta[e] =
 * (v[e] - mem[e]) beta; state[d][e] += k[d] delta[e]; out[e] = sum_d
 * state[d][e] (q[d] D^-1/2), stored as bf16; then the state is rounded to
 * its dtype.  states_out [T][H][D][E] with record, else [H][D][E] (the
 * final state), in the state dtype. */
void lro_delta_rule(const uint16_t *q, const uint16_t *k, const uint16_t *v, const float *G, const uint16_t *beta,
                    const void *state_in, int state_bf16, int T, int H, int D, int E, int normalize, int record,
                    uint16_t *out, void *states_out) {
    float *state = (float *)malloc(sizeof(float) * (size_t)D * E);
    float *qf = (float *)malloc(sizeof(float) * D);
    float *kf = (float *)malloc(sizeof(float) * D);
    float *mem = (float *)malloc(sizeof(float) * E);
    const float scale = 1.0f / sqrtf((float)D);
    for (int h = 0; h < H; ++h) {
        for (size_t i = 0; i < (size_t)D * E; ++i) state[i] = state_get(state_in, state_bf16, (size_t)h * D * E + i);
        for (int t = 0; t < T; ++t) {
            const uint16_t *qt = q + ((size_t)t * H + h) * D;
            const uint16_t *kt = k + ((size_t)t * H + h) * D;
            const uint16_t *vt = v + ((size_t)t * H + h) * E;
            if (normalize) {
                l2norm_bf16(qt, D, qf);
                l2norm_bf16(kt, D, kf);
            } else {
                for (int d = 0; d < D; ++d) qf[d] = lro_bf16_value(qt[d]), kf[d] = lro_bf16_value(kt[d]);
            }
            for (int d = 0; d < D; ++d) qf[d] = qf[d] * scale;
            const float g = G[(size_t)t * H + h];
            const float b = lro_bf16_value(beta[(size_t)t * H + h]);
            for (size_t i = 0; i < (size_t)D * E; ++i) state[i] = state[i] * g;
            for (int e = 0; e < E; ++e) {
                float m = 0.0f;
                for (int d = 0; d < D; ++d) m += state[(size_t)d * E + e] * kf[d];
                mem[e] = (lro_bf16_value(vt[e]) - m) * b;
            }
            for (int d = 0; d < D; ++d)
                for (int e = 0; e < E; ++e) state[(size_t)d * E + e] = state[(size_t)d * E + e] + kf[d] * mem[e];
            for (int e = 0; e < E; ++e) {
                float o = 0.0f;
                for (int d = 0; d < D; ++d) o += state[(size_t)d * E + e] * qf[d];
                out[((size_t)t * H + h) * E + e] = lro_bf16_round(o);
            }
            if (state_bf16)
                for (size_t i = 0; i < (size_t)D * E; ++i) state[i] = rbf(state[i]);
            if (record)
                for (size_t i = 0; i < (size_t)D * E; ++i)
                    state_put(states_out, state_bf16, (((size_t)t * H + h) * D) * E + i, state[i]);
        }
        if (!record)
            for (size_t i = 0; i < (size_t)D * E; ++i) state_put(states_out, state_bf16, (size_t)h * D * E + i, state[i]);
    }
    free(state);
    free(qf);
    free(kf);
    free(mem);
}

#define LRO_DN_KH 16      /* key heads */
#define LRO_DN_VH 32      /* value heads */
#define LRO_DN_D 128      /* key / value head width */
#define LRO_DN_KEY (LRO_DN_KH * LRO_DN_D)     /* 2048 */
#define LRO_DN_VAL (LRO_DN_VH * LRO_DN_D)     /* 4096 */
#define LRO_DN_CONV (2 * LRO_DN_KEY + LRO_DN_VAL)  /* 8192 */
#define LRO_DN_K 4        /* conv kernel */

static inline float silu_f(float x) { return x / (1.0f + lro_exp(-x)); }
static inline float softplus_f(float x) { return x > 20.0f ? x : log1pf(lro_exp(x)); }

/* The Gated DeltaNet mixer for T tokens with a cached state ([HF]
 * Qwen3_5MoeGatedDeltaNet.forward 430-543; dims of the 35B model: 16 key
 * heads, 32 value heads, width 128, conv kernel 4):
 *   mixed = bf16(x W_qkv^T), z = bf16(x W_z^T), b = bf16(x W_b^T),
 *   a = bf16(x W_a^T) (fixed fp32 order, lro_canon_dot);
 *   per channel c the sequence [conv_state[c][0..3], mixed[0..T-1][c]],
 *   token t: bf16(silu(bf16(sum_j w[c][j] seq[t + 1 + j]))) (causal_conv1d
 *   201-218 / 221-240 with the cached left context), conv_state <- the last
 *   4 of the sequence;
 *   q = channels 0..2047 (16 heads), k = 2048..4095, v = 4096..8191 (32
 *   heads); value head h reads key head h / 2 (repeat_interleave);
 *   beta = bf16(sigmoid(b)); g = -exp(A_log) softplus(a + dt_bias) in fp32,
 *   G = exp(g);
 *   lro_delta_rule(normalize = 1) on the cached state (fp32 or bf16);
 *   per token and value head the gated RMSNorm (Qwen3_5MoeRMSNormGated
 *   169-185): n = bf16(o rsqrt(mean(o^2) + eps)), bf16(bf16(w n) silu(z));
 *   out = bf16(normed W_out^T) (fixed fp32 order over 4096).
 * conv_state [8192][4] and state [32][128][128] are updated in place;
 * states_record ([T][32][128][128], state dtype) may be NULL. */
void lro_delta_mixer(const uint16_t *x, int T, const uint16_t *w_qkv, const uint16_t *w_z, const uint16_t *w_b,
                     const uint16_t *w_a, const uint16_t *conv_w, const uint16_t *A_log, const uint16_t *dt_bias,
                     const uint16_t *norm_w, float eps, const uint16_t *w_out, uint16_t *conv_state, void *state,
                     int state_bf16, void *states_record, uint16_t *out) {
    const size_t H = LRO_HIDDEN;
    uint16_t *mixed = (uint16_t *)malloc(sizeof(uint16_t) * T * LRO_DN_CONV);
    uint16_t *z = (uint16_t *)malloc(sizeof(uint16_t) * T * LRO_DN_VAL);
    uint16_t *bb = (uint16_t *)malloc(sizeof(uint16_t) * T * LRO_DN_VH);
    uint16_t *aa = (uint16_t *)malloc(sizeof(uint16_t) * T * LRO_DN_VH);
    float *xf = (float *)malloc(sizeof(float) * LRO_DN_VAL);
    for (int t = 0; t < T; ++t) {
        to_floats(x + t * H, xf, (int)H);
        for (int r = 0; r < LRO_DN_CONV; ++r) mixed[(size_t)t * LRO_DN_CONV + r] = lro_bf16_round(lro_canon_dot(w_qkv + r * H, xf, (int)H));
        for (int r = 0; r < LRO_DN_VAL; ++r) z[(size_t)t * LRO_DN_VAL + r] = lro_bf16_round(lro_canon_dot(w_z + r * H, xf, (int)H));
        for (int r = 0; r < LRO_DN_VH; ++r) bb[t * LRO_DN_VH + r] = lro_bf16_round(lro_canon_dot(w_b + r * H, xf, (int)H));
        for (int r = 0; r < LRO_DN_VH; ++r) aa[t * LRO_DN_VH + r] = lro_bf16_round(lro_canon_dot(w_a + r * H, xf, (int)H));
    }
    /* causal conv with the cached context, SiLU */
    uint16_t *act = (uint16_t *)malloc(sizeof(uint16_t) * T * LRO_DN_CONV);
    float *seq = (float *)malloc(sizeof(float) * (LRO_DN_K + T));
    uint16_t *seqb = (uint16_t *)malloc(sizeof(uint16_t) * (LRO_DN_K + T));
    for (int c = 0; c < LRO_DN_CONV; ++c) {
        for (int j = 0; j < LRO_DN_K; ++j) seqb[j] = conv_state[c * LRO_DN_K + j];
        for (int t = 0; t < T; ++t) seqb[LRO_DN_K + t] = mixed[(size_t)t * LRO_DN_CONV + c];
        for (int i = 0; i < LRO_DN_K + T; ++i) seq[i] = lro_bf16_value(seqb[i]);
        for (int t = 0; t < T; ++t) {
            float acc = 0.0f;
            for (int j = 0; j < LRO_DN_K; ++j) acc = fmaf(lro_bf16_value(conv_w[c * LRO_DN_K + j]), seq[t + 1 + j], acc);
            act[(size_t)t * LRO_DN_CONV + c] = lro_bf16_round(silu_f(rbf(acc)));
        }
        for (int j = 0; j < LRO_DN_K; ++j) conv_state[c * LRO_DN_K + j] = seqb[T + j];
    }
    /* q, k (value heads' copies), v, beta, G */
    uint16_t *q = (uint16_t *)malloc(sizeof(uint16_t) * T * LRO_DN_VAL);
    uint16_t *k = (uint16_t *)malloc(sizeof(uint16_t) * T * LRO_DN_VAL);
    uint16_t *v = (uint16_t *)malloc(sizeof(uint16_t) * T * LRO_DN_VAL);
    uint16_t *beta = (uint16_t *)malloc(sizeof(uint16_t) * T * LRO_DN_VH);
    float *G = (float *)malloc(sizeof(float) * T * LRO_DN_VH);
    for (int t = 0; t < T; ++t) {
        const uint16_t *row = act + (size_t)t * LRO_DN_CONV;
        for (int h = 0; h < LRO_DN_VH; ++h) {
            for (int d = 0; d < LRO_DN_D; ++d) {
                q[((size_t)t * LRO_DN_VH + h) * LRO_DN_D + d] = row[(h / 2) * LRO_DN_D + d];
                k[((size_t)t * LRO_DN_VH + h) * LRO_DN_D + d] = row[LRO_DN_KEY + (h / 2) * LRO_DN_D + d];
                v[((size_t)t * LRO_DN_VH + h) * LRO_DN_D + d] = row[2 * LRO_DN_KEY + h * LRO_DN_D + d];
            }
            const float bv = lro_bf16_value(bb[t * LRO_DN_VH + h]);
            beta[t * LRO_DN_VH + h] = lro_bf16_round(1.0f / (1.0f + lro_exp(-bv)));
            const float gv = -lro_exp(lro_bf16_value(A_log[h])) *
                             softplus_f(lro_bf16_value(aa[t * LRO_DN_VH + h]) + lro_bf16_value(dt_bias[h]));
            G[t * LRO_DN_VH + h] = lro_exp(gv);
        }
    }
    uint16_t *core = (uint16_t *)malloc(sizeof(uint16_t) * T * LRO_DN_VAL);
    const size_t state_elems = (size_t)LRO_DN_VH * LRO_DN_D * LRO_DN_D;
    const size_t esz = state_bf16 ? 2 : 4;
    void *rec = states_record ? states_record : malloc(esz * state_elems * T);
    lro_delta_rule(q, k, v, G, beta, state, state_bf16, T, LRO_DN_VH, LRO_DN_D, LRO_DN_D, 1, 1, core, rec);
    memcpy(state, (const char *)rec + esz * state_elems * (T - 1), esz * state_elems);
    if (!states_record) free(rec);
    /* gated RMSNorm per token and value head */
    uint16_t *normed = (uint16_t *)malloc(sizeof(uint16_t) * T * LRO_DN_VAL);
    for (int t = 0; t < T; ++t) {
        for (int h = 0; h < LRO_DN_VH; ++h) {
            const uint16_t *o = core + ((size_t)t * LRO_DN_VH + h) * LRO_DN_D;
            float var = 0.0f;
            for (int e = 0; e < LRO_DN_D; ++e) var += lro_bf16_value(o[e]) * lro_bf16_value(o[e]);
            var = var / (float)LRO_DN_D;
            const float r = 1.0f / sqrtf(var + eps);
            for (int e = 0; e < LRO_DN_D; ++e) {
                const float n = rbf(lro_bf16_value(o[e]) * r);
                const float wn = rbf(lro_bf16_value(norm_w[e]) * n);
                const float zz = lro_bf16_value(z[(size_t)t * LRO_DN_VAL + h * LRO_DN_D + e]);
                normed[(size_t)t * LRO_DN_VAL + h * LRO_DN_D + e] = lro_bf16_round(wn * silu_f(zz));
            }
        }
    }
    for (int t = 0; t < T; ++t) {
        to_floats(normed + (size_t)t * LRO_DN_VAL, xf, LRO_DN_VAL);
        for (size_t r = 0; r < H; ++r) out[t * H + r] = lro_bf16_round(lro_canon_dot(w_out + r * LRO_DN_VAL, xf, LRO_DN_VAL));
    }
    free(normed);
    free(core);
    free(G);
    free(beta);
    free(v);
    free(k);
    free(q);
    free(seqb);
    free(seq);
    free(act);
    free(xf);
    free(aa);
    free(bb);
    free(z);
    free(mixed);
}

/* ---- full-attention decode step ([HF] Qwen3_5MoeAttention) -------------- */

#define LRO_AT_HEADS 16   /* query heads */
#define LRO_AT_KV 2       /* key/value heads */
#define LRO_AT_D 256      /* head width */
#define LRO_AT_ROT 64     /* rotary width (partial_rotary_factor 0.25) */
#define LRO_AT_QG (LRO_AT_HEADS * 2 * LRO_AT_D)   /* 8192 q_proj rows: per head 256 query, 256 gate */
#define LRO_AT_O (LRO_AT_HEADS * LRO_AT_D)        /* 4096 o_proj inputs */

/* Qwen3_5MoeRMSNorm over one head (fp32: x rsqrt(mean x^2 + eps), times
 * (1 + w), then bf16), then the rotary embedding of dims 0..63
 * (apply_rotary_pos_emb with cos, sin bf16 as given: every product and the
 * sum rounded to bf16, rotate_half = [-x[32..63], x[0..31]]). */
static void attn_norm_rope(const uint16_t *raw, const uint16_t *w, float eps, const uint16_t *cos_r,
                           const uint16_t *sin_r, uint16_t *out) {
    float var = 0.0f;
    for (int d = 0; d < LRO_AT_D; ++d) var += lro_bf16_value(raw[d]) * lro_bf16_value(raw[d]);
    var = var / (float)LRO_AT_D;
    const float r = 1.0f / sqrtf(var + eps);
    float n[LRO_AT_D];
    for (int d = 0; d < LRO_AT_D; ++d) n[d] = rbf((lro_bf16_value(raw[d]) * r) * (1.0f + lro_bf16_value(w[d])));
    for (int d = 0; d < LRO_AT_D; ++d) {
        if (d < LRO_AT_ROT) {
            const float rot = d < LRO_AT_ROT / 2 ? -n[d + LRO_AT_ROT / 2] : n[d - LRO_AT_ROT / 2];
            const float a = rbf(n[d] * lro_bf16_value(cos_r[d]));
            const float b = rbf(rot * lro_bf16_value(sin_r[d]));
            out[d] = lro_bf16_round(a + b);
        } else {
            out[d] = lro_bf16_round(n[d]);
        }
    }
}

/* One cached full-attention forward of T tokens after `length` cached
 * positions ([HF] Qwen3_5MoeAttention.forward with eager_attention_forward;
 * 35B dims: hidden 2048, 16 query heads over 2 key/value heads, width 256,
 * rotary width 64):
 *   qg = bf16(x Wq^T) viewed [T][16][512]: query = [..., :256], gate = [..., 256:];
 *   k = bf16(x Wk^T), v = bf16(x Wv^T) viewed [T][2][256];
 *   query and k: per-head RMSNorm with (1 + w), then the rotary embedding
 *   (attn_norm_rope) with cos, sin [T][64];
 *   k_cache, v_cache [2][capacity][256] receive positions length .. length + T - 1;
 *   head h reads key/value head h / 8 (repeat_kv); for token t the scores
 *   over positions p <= length + t (the causal mask) are
 *   s = bf16(q . k_p) / 16 (exact), p = bf16(softmax_fp32(s)),
 *   o = bf16(sum_p p v_p) (fp32, positions ascending);
 *   a = bf16(o bf16(sigmoid(gate))); out = bf16(a Wo^T) [T][2048].
 * Projections and q.k use lro_canon_dot's fixed fp32 order. */
void lro_attn_decode(const uint16_t *x, int T, const uint16_t *w_q, const uint16_t *w_k, const uint16_t *w_v,
                     const uint16_t *w_o, const uint16_t *q_norm, const uint16_t *k_norm, float eps,
                     const uint16_t *cos_t, const uint16_t *sin_t, uint16_t *k_cache, uint16_t *v_cache,
                     int capacity, int length, uint16_t *out) {
    const size_t H = LRO_HIDDEN;
    const size_t KVW = (size_t)LRO_AT_KV * LRO_AT_D;
    uint16_t *qg = (uint16_t *)malloc(sizeof(uint16_t) * T * LRO_AT_QG);
    uint16_t *kr = (uint16_t *)malloc(sizeof(uint16_t) * T * KVW);
    uint16_t *vr = (uint16_t *)malloc(sizeof(uint16_t) * T * KVW);
    uint16_t *q = (uint16_t *)malloc(sizeof(uint16_t) * T * LRO_AT_O);
    uint16_t *att = (uint16_t *)malloc(sizeof(uint16_t) * T * LRO_AT_O);
    float *xf = (float *)malloc(sizeof(float) * LRO_AT_O);
    const int total = length + T;
    float *s = (float *)malloc(sizeof(float) * total);
    for (int t = 0; t < T; ++t) {
        to_floats(x + t * H, xf, (int)H);
        for (int r = 0; r < LRO_AT_QG; ++r) qg[(size_t)t * LRO_AT_QG + r] = lro_bf16_round(lro_canon_dot(w_q + r * H, xf, (int)H));
        for (size_t r = 0; r < KVW; ++r) kr[t * KVW + r] = lro_bf16_round(lro_canon_dot(w_k + r * H, xf, (int)H));
        for (size_t r = 0; r < KVW; ++r) vr[t * KVW + r] = lro_bf16_round(lro_canon_dot(w_v + r * H, xf, (int)H));
    }
    for (int t = 0; t < T; ++t) {
        const uint16_t *cr = cos_t + t * LRO_AT_ROT;
        const uint16_t *sr = sin_t + t * LRO_AT_ROT;
        for (int h = 0; h < LRO_AT_HEADS; ++h)
            attn_norm_rope(qg + (size_t)t * LRO_AT_QG + h * 2 * LRO_AT_D, q_norm, eps, cr, sr,
                           q + (size_t)t * LRO_AT_O + h * LRO_AT_D);
        for (int g = 0; g < LRO_AT_KV; ++g) {
            const size_t at = ((size_t)g * capacity + length + t) * LRO_AT_D;
            attn_norm_rope(kr + t * KVW + g * LRO_AT_D, k_norm, eps, cr, sr, k_cache + at);
            memcpy(v_cache + at, vr + t * KVW + g * LRO_AT_D, sizeof(uint16_t) * LRO_AT_D);
        }
    }
    float qf[LRO_AT_D];
    float o[LRO_AT_D];
    for (int t = 0; t < T; ++t) {
        const int seen = length + t + 1;
        for (int h = 0; h < LRO_AT_HEADS; ++h) {
            const int g = h / (LRO_AT_HEADS / LRO_AT_KV);
            const uint16_t *kc = k_cache + (size_t)g * capacity * LRO_AT_D;
            const uint16_t *vc = v_cache + (size_t)g * capacity * LRO_AT_D;
            to_floats(q + (size_t)t * LRO_AT_O + h * LRO_AT_D, qf, LRO_AT_D);
            float m = -INFINITY;
            for (int p = 0; p < seen; ++p) {
                s[p] = rbf(lro_canon_dot(kc + (size_t)p * LRO_AT_D, qf, LRO_AT_D)) * 0.0625f;
                if (s[p] > m) m = s[p];
            }
            float sum = 0.0f;
            for (int p = 0; p < seen; ++p) {
                s[p] = lro_exp(s[p] - m);
                sum += s[p];
            }
            for (int d = 0; d < LRO_AT_D; ++d) o[d] = 0.0f;
            for (int p = 0; p < seen; ++p) {
                const float pr = rbf(s[p] / sum);
                for (int d = 0; d < LRO_AT_D; ++d) o[d] = fmaf(pr, lro_bf16_value(vc[(size_t)p * LRO_AT_D + d]), o[d]);
            }
            const uint16_t *gate = qg + (size_t)t * LRO_AT_QG + h * 2 * LRO_AT_D + LRO_AT_D;
            for (int d = 0; d < LRO_AT_D; ++d) {
                const float sg = rbf(1.0f / (1.0f + lro_exp(-lro_bf16_value(gate[d]))));
                att[(size_t)t * LRO_AT_O + h * LRO_AT_D + d] = lro_bf16_round(rbf(o[d]) * sg);
            }
        }
    }
    for (int t = 0; t < T; ++t) {
        to_floats(att + (size_t)t * LRO_AT_O, xf, LRO_AT_O);
        for (size_t r = 0; r < H; ++r) out[t * H + r] = lro_bf16_round(lro_canon_dot(w_o + r * LRO_AT_O, xf, LRO_AT_O));
    }
    free(s);
    free(xf);
    free(att);
    free(q);
    free(vr);
    free(kr);
    free(qg);
}
