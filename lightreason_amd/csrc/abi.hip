// extern "C" entry points of liblrmoe.so (declared in include/lrmoe.h).
// Host-side argument checks happen here; nothing is launched when they fail.
#include <string.h>

#include <mutex>

#include "lrmoe_internal.h"

namespace {

using lrmoe::Plan;
using lrmoe::Workspace;

constexpr int kMaxTokens = 1 << 16;

hipStream_t as_stream(void* stream) { return reinterpret_cast<hipStream_t>(stream); }

int status_of(hipError_t err) { return err == hipSuccess ? LRMOE_OK : static_cast<int>(err); }

// gfx950 check of the current device, cached per device ordinal.
int check_device() {
    static int device_state[64] = {0};  // 0 unknown, 1 ok, 2 wrong device
    int device = 0;
    hipError_t err = hipGetDevice(&device);
    if (err != hipSuccess) return static_cast<int>(err);
    if (device >= 0 && device < 64 && device_state[device] != 0) return device_state[device] == 1 ? LRMOE_OK : LRMOE_E_DEVICE;
    hipDeviceProp_t prop;
    err = hipGetDeviceProperties(&prop, device);
    if (err != hipSuccess) return static_cast<int>(err);
    const bool ok = strncmp(prop.gcnArchName, "gfx950", 6) == 0;
    if (device >= 0 && device < 64) device_state[device] = ok ? 1 : 2;
    return ok ? LRMOE_OK : LRMOE_E_DEVICE;
}

bool bad_tokens(int tokens) { return tokens < 0 || tokens > kMaxTokens; }

// A non-null pointer that is not a multiple of `bytes`.
bool misaligned(const void* p, size_t bytes) { return (reinterpret_cast<uintptr_t>(p) % bytes) != 0; }

// ---- the no-allocation decode layer (lrmoe_moe_layer_static) ----------------
//
// Its scratch is this file-scope device array: one copy per GPU, held until the
// process ends, shared by every call on that GPU (it keeps the last call's
// counters and tagged rows).  Host code never uses the array's name as an
// address: the per-device address comes from hipGetSymbolAddress once per
// device (static_scratch()), and only that address is handed to kernels.
constexpr size_t kStaticScratchBytes = 3u << 20;  // >= lrmoe::workspace_bytes(16)
__device__ __align__(256) uint8_t scratch[kStaticScratchBytes];

// Zeroes the scratch on its first uncaptured use on a device.  The array has
// static storage and no initialiser, so the code-object loader hands it out
// zero-filled; the clear only restates that for a first call made outside a
// graph capture.  A first call made under capture does not record it (a
// recorded clear would rerun on every replay and reset the counters and
// tagged rows that later calls rely on).
__global__ __launch_bounds__(256) void clear_scratch(uint4* p, size_t n16) {
    for (size_t i = static_cast<size_t>(blockIdx.x) * 256 + threadIdx.x; i < n16; i += static_cast<size_t>(gridDim.x) * 256)
        p[i] = make_uint4(0u, 0u, 0u, 0u);
}

struct StaticScratch {
    std::mutex lock;
    void* ptr[64] = {};     // device address of `scratch`, per device
    bool cleared[64] = {};  // clear_scratch enqueued on that device
};

StaticScratch& static_state() {
    static StaticScratch s;
    return s;
}

// The scratch address on the current device, looked up (and the scratch
// zeroed on `stream`) on the device's first call.
int static_scratch(void** out, hipStream_t stream) {
    int device = 0;
    hipError_t err = hipGetDevice(&device);
    if (err != hipSuccess) return static_cast<int>(err);
    if (device < 0 || device >= 64) return static_cast<int>(hipErrorInvalidDevice);
    StaticScratch& s = static_state();
    std::lock_guard<std::mutex> guard(s.lock);
    if (!s.ptr[device]) {
        void* p = nullptr;
        err = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
        if (err != hipSuccess) return static_cast<int>(err);
        if (!p) return static_cast<int>(hipErrorInvalidSymbol);
        s.ptr[device] = p;
    }
    if (!s.cleared[device]) {
        hipStreamCaptureStatus capture = hipStreamCaptureStatusNone;
        err = hipStreamIsCapturing(stream, &capture);
        if (err != hipSuccess) return static_cast<int>(err);
        if (capture == hipStreamCaptureStatusNone) {
            hipLaunchKernelGGL(clear_scratch, dim3(256), dim3(256), 0, stream, static_cast<uint4*>(s.ptr[device]),
                               kStaticScratchBytes / 16);
            err = hipGetLastError();
            if (err != hipSuccess) return static_cast<int>(err);
        }
        s.cleared[device] = true;
    }
    *out = s.ptr[device];
    return LRMOE_OK;
}

}  // namespace

extern "C" {

const char* lrmoe_version(void) { return "lrmoe 0.1 gfx950"; }

const char* lrmoe_error_string(int code) {
    switch (code) {
        case LRMOE_OK: return "ok";
        case LRMOE_E_ARG: return "lrmoe: invalid argument (null pointer, size or shape)";
        case LRMOE_E_WORKSPACE: return "lrmoe: workspace smaller than lrmoe_workspace_bytes(tokens)";
        case LRMOE_E_DEVICE: return "lrmoe: the current HIP device is not gfx950 (MI355X)";
        default: return code > 0 ? hipGetErrorString(static_cast<hipError_t>(code)) : "lrmoe: unknown error";
    }
}

int lrmoe_device_check(void) { return check_device(); }

size_t lrmoe_workspace_bytes(int tokens) { return lrmoe::workspace_bytes(tokens); }

int lrmoe_route_topk(const uint16_t* hidden, int tokens, const uint16_t* router_weight, const uint16_t* logits_in,
                     const uint16_t* norm_weight, float eps, const uint16_t* shared_expert_gate, uint16_t* logits_out,
                     int64_t* indices_out, uint16_t* weights_out, uint16_t* shared_gate_out, uint16_t* normed_out,
                     void* workspace, size_t workspace_bytes, void* stream) {
    if (bad_tokens(tokens)) return LRMOE_E_ARG;
    if (tokens > 0 && (!hidden || !indices_out || !weights_out || !workspace || (!router_weight == !logits_in)))
        return LRMOE_E_ARG;
    if (tokens == 0) return LRMOE_OK;
    if (workspace_bytes < lrmoe::workspace_bytes(tokens)) return LRMOE_E_WORKSPACE;
    if (int d = check_device()) return d;
    const Workspace ws = lrmoe::carve(workspace, tokens);
    lrmoe::RouteArgs a{};
    a.x = hidden;
    a.norm = norm_weight;
    a.eps = eps;
    a.router = router_weight;
    a.logits_in = logits_in;
    a.shared_gate = shared_expert_gate;
    a.tokens = tokens;
    a.normed = normed_out ? normed_out : ws.normed;
    a.logits = logits_out ? logits_out : ws.logits;
    a.indices = indices_out;
    a.weights = weights_out;
    a.sg = shared_gate_out ? shared_gate_out : ws.sg;
    a.plan = ws.plan;
    a.ws = ws;
    return status_of(lrmoe::launch_route(a, as_stream(stream)));
}

int lrmoe_bucket(const int64_t* indices, int tokens, int32_t* expert, int32_t* offset, int32_t* pair_token,
                 int32_t* pair_slot, int32_t* route_pair, int32_t* unique, int32_t* status, void* workspace,
                 size_t workspace_bytes, void* stream) {
    if (bad_tokens(tokens)) return LRMOE_E_ARG;
    if (tokens == 0) return LRMOE_OK;
    if (!indices || !expert || !offset || !pair_token || !pair_slot || !route_pair || !unique || !status)
        return LRMOE_E_ARG;
    if (tokens > 64 && (!workspace || workspace_bytes < lrmoe::workspace_bytes(tokens))) return LRMOE_E_WORKSPACE;
    if (int d = check_device()) return d;
    const Workspace ws = lrmoe::carve(workspace, tokens);
    Plan plan{expert, offset, pair_token, pair_slot, route_pair, unique, status};
    return status_of(lrmoe::launch_bucket(indices, tokens, ws, plan, as_stream(stream)));
}

int lrmoe_moe_experts(const uint16_t* hidden, int tokens, const int64_t* indices, const uint16_t* weights,
                      const int64_t* expert_ptrs, uint16_t* out, void* workspace, size_t workspace_bytes,
                      void* stream) {
    if (bad_tokens(tokens)) return LRMOE_E_ARG;
    if (tokens == 0) return LRMOE_OK;
    if (!hidden || !indices || !weights || !expert_ptrs || !out || !workspace) return LRMOE_E_ARG;
    if (workspace_bytes < lrmoe::workspace_bytes(tokens)) return LRMOE_E_WORKSPACE;
    if (int d = check_device()) return d;
    const Workspace ws = lrmoe::carve(workspace, tokens);
    hipStream_t s = as_stream(stream);
    if (tokens <= lrmoe::kDecodeMaxTokens) {
        lrmoe::DecodeArgs d{};
        d.x = hidden;
        d.indices_in = indices;
        d.weights_in = weights;
        d.expert_ptrs = expert_ptrs;
        d.out = out;
        d.logits = ws.dlogits;
        d.act = ws.dact;
        d.y = ws.dy;
        d.sync = ws.sync;
        d.status = ws.plan.status;
        d.tokens = tokens;
        return status_of(lrmoe::launch_moe_decode(d, s));
    }
    hipError_t err = lrmoe::launch_prefill_plan(nullptr, indices, weights, nullptr, nullptr, tokens, 0, ws, ws.plan, s);
    if (err != hipSuccess) return status_of(err);
    lrmoe::ExpertArgs a{};
    a.x = hidden;
    a.expert_ptrs = expert_ptrs;
    a.weights = weights;
    a.out = out;
    a.tokens = tokens;
    a.plan = ws.plan;
    a.ws = ws;
    return status_of(lrmoe::launch_experts(a, s));
}

int lrmoe_moe_layer(const uint16_t* hidden, int tokens, const uint16_t* router_weight, const uint16_t* logits_in,
                    const int64_t* expert_ptrs, const int64_t* expert_codec,
                    const uint16_t* shared_gate_proj, const uint16_t* shared_up_proj,
                    const uint16_t* shared_down_proj, const uint16_t* shared_expert_gate,
                    const uint16_t* norm_weight, float eps, uint16_t* out, int64_t* indices_out,
                    uint16_t* weights_out, void* workspace, size_t workspace_bytes, void* stream) {
    if (bad_tokens(tokens)) return LRMOE_E_ARG;
    if (tokens == 0) return LRMOE_OK;
    if (!hidden || !expert_ptrs || !out || !workspace || (!router_weight == !logits_in)) return LRMOE_E_ARG;
    const bool any_shared = shared_gate_proj || shared_up_proj || shared_down_proj || shared_expert_gate;
    const bool all_shared = shared_gate_proj && shared_up_proj && shared_down_proj && shared_expert_gate;
    if (any_shared && !all_shared) return LRMOE_E_ARG;
    if (workspace_bytes < lrmoe::workspace_bytes(tokens)) return LRMOE_E_WORKSPACE;
    if (int d = check_device()) return d;
    const Workspace ws = lrmoe::carve(workspace, tokens);
    hipStream_t s = as_stream(stream);
    if (tokens <= lrmoe::kDecodeMaxTokens) {
        lrmoe::DecodeArgs d{};
        d.x = hidden;
        d.norm = norm_weight;
        d.eps = eps;
        d.router = logits_in ? nullptr : router_weight;
        d.logits_in = logits_in;
        d.shared_expert_gate = shared_expert_gate;
        d.sh_gate = shared_gate_proj;
        d.sh_up = shared_up_proj;
        d.sh_down = shared_down_proj;
        d.expert_ptrs = expert_ptrs;
        d.codec = expert_codec;
        d.out = out;
        d.indices_out = indices_out;
        d.weights_out = weights_out;
        d.logits = ws.dlogits;
        d.act = ws.dact;
        d.y = ws.dy;
        d.sync = ws.sync;
        d.status = ws.plan.status;
        d.tokens = tokens;
        d.residual = norm_weight != nullptr;
        return status_of(lrmoe::launch_moe_decode(d, s));
    }
    lrmoe::RouteArgs r{};
    r.x = hidden;
    r.norm = norm_weight;
    r.eps = eps;
    r.router = router_weight;
    r.logits_in = logits_in;
    r.shared_gate = shared_expert_gate;
    r.tokens = tokens;
    r.normed = ws.normed;
    r.logits = ws.logits;
    r.indices = indices_out ? indices_out : ws.indices;
    r.weights = weights_out ? weights_out : ws.weights;
    r.sg = ws.sg;
    r.shared_down = shared_down_proj;
    r.plan = ws.plan;
    r.ws = ws;
    hipError_t err = lrmoe::launch_route(r, s);
    if (err != hipSuccess) return status_of(err);
    lrmoe::ExpertArgs a{};
    a.x = norm_weight ? ws.normed : hidden;
    a.expert_ptrs = expert_ptrs;
    a.shared_gate_proj = shared_gate_proj;
    a.shared_up_proj = shared_up_proj;
    a.shared_down = shared_down_proj;
    a.weights = r.weights;
    a.sg = ws.sg;
    a.residual = norm_weight ? hidden : nullptr;
    a.out = out;
    a.tokens = tokens;
    a.plan = ws.plan;
    a.ws = ws;
    return status_of(lrmoe::launch_experts(a, s));
}

int lrmoe_moe_layer_static(const uint16_t* hidden, int tokens, const uint16_t* router_weight,
                           const uint16_t* logits_in, const int64_t* expert_ptrs, const int64_t* expert_codec,
                           const uint16_t* shared_gate_proj, const uint16_t* shared_up_proj,
                           const uint16_t* shared_down_proj, const uint16_t* shared_expert_gate,
                           const uint16_t* norm_weight, float eps, uint16_t* out, int64_t* indices_out,
                           uint16_t* weights_out, int32_t* status_out, void* stream) {
    if (tokens < 0 || tokens > LRMOE_STATIC_MAX_TOKENS) return LRMOE_E_ARG;
    if (tokens == 0) return LRMOE_OK;
    if (!hidden || !expert_ptrs || !out || (!router_weight == !logits_in)) return LRMOE_E_ARG;
    const bool any_shared = shared_gate_proj || shared_up_proj || shared_down_proj || shared_expert_gate;
    const bool all_shared = shared_gate_proj && shared_up_proj && shared_down_proj && shared_expert_gate;
    if (any_shared && !all_shared) return LRMOE_E_ARG;
    if (lrmoe::workspace_bytes(LRMOE_STATIC_MAX_TOKENS) > kStaticScratchBytes) return LRMOE_E_WORKSPACE;
    if (int d = check_device()) return d;
    hipStream_t s = as_stream(stream);
    void* base = nullptr;
    if (int e = static_scratch(&base, s)) return e;
    // The decode layer's scratch (counters, tagged rows) sits at fixed
    // offsets of a 16-token workspace, whatever the call's token count.
    const Workspace ws = lrmoe::carve(base, LRMOE_STATIC_MAX_TOKENS);
    lrmoe::DecodeArgs d{};
    d.x = hidden;
    d.norm = norm_weight;
    d.eps = eps;
    d.router = logits_in ? nullptr : router_weight;
    d.logits_in = logits_in;
    d.shared_expert_gate = shared_expert_gate;
    d.sh_gate = shared_gate_proj;
    d.sh_up = shared_up_proj;
    d.sh_down = shared_down_proj;
    d.expert_ptrs = expert_ptrs;
    d.codec = expert_codec;
    d.out = out;
    d.indices_out = indices_out;
    d.weights_out = weights_out;
    d.logits = ws.dlogits;
    d.act = ws.dact;
    d.y = ws.dy;
    d.sync = ws.sync;
    d.status = status_out ? status_out : ws.plan.status;
    d.tokens = tokens;
    d.residual = norm_weight != nullptr;
    return status_of(lrmoe::launch_moe_decode(d, s));
}

int lrmoe_moe_chain(const uint16_t* hidden, int tokens, int layers, const int64_t* layer_table, float eps,
                    uint16_t* out, int64_t* indices_out, uint16_t* weights_out, void* workspace,
                    size_t workspace_bytes, void* stream) {
    static_assert(lrmoe::kChainMaxLayers == LRMOE_CHAIN_MAX_LAYERS, "chain layer limit");
    if (tokens < 0 || tokens > lrmoe::kDecodeMaxTokens || layers < 0 || layers > LRMOE_CHAIN_MAX_LAYERS)
        return LRMOE_E_ARG;
    if (tokens == 0 || layers == 0) return LRMOE_OK;
    if (!hidden || !layer_table || !out || !workspace) return LRMOE_E_ARG;
    if (workspace_bytes < lrmoe::workspace_bytes(tokens)) return LRMOE_E_WORKSPACE;
    lrmoe::ChainArgs c{};
    for (int l = 0; l < layers; ++l) {
        const int64_t* row = layer_table + static_cast<size_t>(l) * LRMOE_CHAIN_PTRS;
        auto at = [&](int i) { return reinterpret_cast<const uint16_t*>(static_cast<uintptr_t>(row[i])); };
        lrmoe::ChainLayer& w = c.layer[l];
        w.router = at(LRMOE_CHAIN_ROUTER);
        w.expert_ptrs = reinterpret_cast<const int64_t*>(at(LRMOE_CHAIN_EXPERTS));
        w.sh_gate = at(LRMOE_CHAIN_SHARED_GATE_PROJ);
        w.sh_up = at(LRMOE_CHAIN_SHARED_UP_PROJ);
        w.sh_down = at(LRMOE_CHAIN_SHARED_DOWN_PROJ);
        w.shared_expert_gate = at(LRMOE_CHAIN_SHARED_EXPERT_GATE);
        w.norm = at(LRMOE_CHAIN_NORM);
        w.codec = reinterpret_cast<const int64_t*>(at(LRMOE_CHAIN_CODEC));
        if (!w.router || !w.expert_ptrs) return LRMOE_E_ARG;
        const bool any_shared = w.sh_gate || w.sh_up || w.sh_down || w.shared_expert_gate;
        const bool all_shared = w.sh_gate && w.sh_up && w.sh_down && w.shared_expert_gate;
        if (any_shared && !all_shared) return LRMOE_E_ARG;
    }
    if (int d = check_device()) return d;
    const Workspace ws = lrmoe::carve(workspace, tokens);
    c.base.eps = eps;
    c.base.indices_out = indices_out;
    c.base.weights_out = weights_out;
    c.base.logits = ws.dlogits;
    c.base.act = ws.dact;
    c.base.y = ws.dy;
    c.base.sync = ws.sync;
    c.base.status = ws.plan.status;
    c.base.tokens = tokens;
    c.hidden = hidden;
    c.out = out;
    c.inner = ws.chain;
    c.layers = layers;
    return status_of(lrmoe::launch_moe_chain(c, as_stream(stream)));
}

int lrmoe_codec_pack(const uint16_t* w, int64_t rows, int cols, uint8_t* packed, uint8_t* bases,
                     unsigned long long* misfit, void* stream) {
    if (rows < 0 || cols < 0 || cols % lrmoe::kCodecTile != 0) return LRMOE_E_ARG;
    if (rows == 0 || cols == 0) return LRMOE_OK;
    if (!w || !packed || !bases) return LRMOE_E_ARG;
    if (int d = check_device()) return d;
    return status_of(lrmoe::launch_codec_pack(w, rows, cols, packed, bases, misfit, as_stream(stream)));
}

int lrmoe_codec_unpack(const uint8_t* packed, const uint8_t* bases, int64_t rows, int cols, uint16_t* w,
                       void* stream) {
    if (rows < 0 || cols < 0 || cols % lrmoe::kCodecTile != 0) return LRMOE_E_ARG;
    if (rows == 0 || cols == 0) return LRMOE_OK;
    if (!w || !packed || !bases) return LRMOE_E_ARG;
    if (int d = check_device()) return d;
    return status_of(lrmoe::launch_codec_unpack(packed, bases, rows, cols, w, as_stream(stream)));
}

int lrmoe_gather(const int64_t* descriptors, const int64_t* destinations, const int64_t* sizes,
                 const int32_t* src_ids, const int32_t* dst_ids, const int64_t* count, int experts, int banks,
                 int max_copies, int stripes, int threads, int keep_in_l2, int32_t* status, void* stream) {
    if (!descriptors || !destinations || !sizes || !src_ids || !dst_ids || !count) return LRMOE_E_ARG;
    if (experts <= 0 || banks <= 0 || banks > 65535 || max_copies < 0 || max_copies > 65535 || stripes <= 0 ||
        stripes > 65535 || threads < 64 || threads > 256 || threads % 64 != 0)
        return LRMOE_E_ARG;
    if (max_copies == 0) return LRMOE_OK;
    if (int d = check_device()) return d;
    return status_of(lrmoe::launch_gather(descriptors, destinations, sizes, src_ids, dst_ids, count, experts, banks,
                                          max_copies, stripes, threads, keep_in_l2, status, as_stream(stream)));
}

int lrmoe_gather_tiles(const int64_t* descriptors, const int64_t* destinations, const int64_t* sizes,
                       const int32_t* src_ids, const int32_t* dst_ids, const int64_t* count, int experts, int banks,
                       int max_copies, int stripes, int threads, int compact, void* stream) {
    if (!descriptors || !destinations || !sizes || !src_ids || !dst_ids || !count) return LRMOE_E_ARG;
    if (experts <= 0 || banks <= 0 || banks > 65535 || max_copies < 0 || max_copies > 65535 || stripes <= 0 ||
        stripes > 65535 || threads < 64 || threads > 256 || threads % 64 != 0)
        return LRMOE_E_ARG;
    if (max_copies == 0) return LRMOE_OK;
    if (int d = check_device()) return d;
    return status_of(lrmoe::launch_gather_tiles(descriptors, destinations, sizes, src_ids, dst_ids, count, experts,
                                                banks, max_copies, stripes, threads, compact, as_stream(stream)));
}

int lrmoe_matvec(const int64_t* table, const uint16_t* x, uint16_t* result, int K, int N, int column, int shared_x,
                 int stride, int experts, void* stream) {
    if (!table || !x || !result || K <= 0 || K % 512 != 0 || N <= 0 || experts <= 0 || experts > 65535 ||
        stride < 2 || column < 0 || column >= stride)
        return LRMOE_E_ARG;
    if (int d = check_device()) return d;
    return status_of(lrmoe::launch_matvec(table, x, result, K, N, column, shared_x, stride, experts, as_stream(stream)));
}

int lrmoe_ordered_sum(const int64_t* table, const uint16_t* hot, const uint16_t* cold, const uint16_t* router,
                      uint16_t* out, int stride, void* stream) {
    if (!table || !hot || !router || !out || (stride != 3 && stride != 4)) return LRMOE_E_ARG;
    if (int d = check_device()) return d;
    return status_of(lrmoe::launch_ordered_sum(table, hot, cold, router, out, stride, as_stream(stream)));
}

int lrmoe_gate_silu(const int64_t* table, const uint16_t* hidden, uint16_t* active, int stride, int experts,
                    void* stream) {
    if (!table || !hidden || !active || stride < 1 || experts <= 0 || experts > 65535) return LRMOE_E_ARG;
    if (int d = check_device()) return d;
    return status_of(lrmoe::launch_gate_silu(table, hidden, active, stride, experts, as_stream(stream)));
}

int lrmoe_project(const int64_t* pointers, const int32_t* routes, const uint16_t* X, uint16_t* Y, int in, int out,
                  int down, int experts, void* stream) {
    if (!pointers || !routes || !X || !Y || in <= 0 || in % 256 != 0 || out <= 0 || out % 64 != 0 || experts < 0 ||
        experts > 65535)
        return LRMOE_E_ARG;
    if (experts == 0) return LRMOE_OK;
    if (int d = check_device()) return d;
    return status_of(lrmoe::launch_project(pointers, routes, X, Y, in, out, down ? 1 : 0, experts, as_stream(stream)));
}

int lrmoe_swiglu_rows(const uint16_t* gates, uint16_t* active, int rows, void* stream) {
    if (!gates || !active || rows < 0) return LRMOE_E_ARG;
    if (rows == 0) return LRMOE_OK;
    if (int d = check_device()) return d;
    return status_of(lrmoe::launch_swiglu_rows(gates, active, rows, as_stream(stream)));
}

int lrmoe_add_rmsnorm(const uint16_t* x, const uint16_t* add, int tokens, const uint16_t* norm_weight, float eps,
                      uint16_t* sum_out, uint16_t* norm_out, void* stream) {
    if (bad_tokens(tokens)) return LRMOE_E_ARG;
    if (tokens > 0 && (!x || (!sum_out && !norm_out) || (norm_weight && !norm_out) || (!norm_weight && norm_out) ||
                       (sum_out && !add)))
        return LRMOE_E_ARG;
    if (misaligned(x, 16) || misaligned(add, 16) || misaligned(norm_weight, 16) || misaligned(sum_out, 16) ||
        misaligned(norm_out, 16))
        return LRMOE_E_ARG;
    if (tokens == 0) return LRMOE_OK;
    if (int d = check_device()) return d;
    return status_of(lrmoe::launch_add_rmsnorm(x, add, tokens, norm_weight, eps, sum_out, norm_out, as_stream(stream)));
}

int lrmoe_block_combine(const int32_t* inverse, const uint16_t* X, const uint16_t* cold, const uint16_t* router,
                        uint16_t* out, int tokens, int hybrid, void* stream) {
    if (!inverse || !X || !router || !out || bad_tokens(tokens) || (hybrid && !cold)) return LRMOE_E_ARG;
    if (tokens == 0) return LRMOE_OK;
    if (int d = check_device()) return d;
    return status_of(lrmoe::launch_block_combine(inverse, X, cold, router, out, tokens, hybrid ? 1 : 0,
                                                 as_stream(stream)));
}

int lrmoe_fill_normal_bf16(uint16_t* out, int64_t count, uint64_t seed, uint64_t stream_id, double sigma,
                           int64_t first, void* stream) {
    if (!out || count < 0) return LRMOE_E_ARG;
    if (count == 0) return LRMOE_OK;
    if (int d = check_device()) return d;
    return status_of(lrmoe::launch_fill_normal(out, count, seed, stream_id, sigma, first, as_stream(stream)));
}

// ---- Gated DeltaNet decode ----

size_t lrmoe_delta_workspace_bytes(int tokens) {
    if (tokens < 1 || tokens > lrmoe::kDeltaMaxTokens) return 0;
    return lrmoe::delta_workspace_bytes(tokens);
}

int lrmoe_delta_rule(const uint16_t* q, const uint16_t* k, const uint16_t* v, const float* G, const uint16_t* beta,
                     const void* initial, int state_bf16, int tokens, int heads, int key_width, int value_width,
                     int normalize, int record, uint16_t* out, void* states, void* stream) {
    if (bad_tokens(tokens) || heads <= 0 || heads > 65535 ||
        (key_width != 64 && key_width != 128 && key_width != 256) || value_width <= 0 || value_width % 16 != 0 ||
        value_width / 4 > 65535 || !initial || !states)
        return LRMOE_E_ARG;
    if (tokens > 0 && (!q || !k || !v || !G || !beta || !out)) return LRMOE_E_ARG;
    const size_t qk_align = key_width == 64 ? 8 : 16;
    if ((tokens > 0 && (misaligned(q, qk_align) || misaligned(k, qk_align) || misaligned(v, 8) || misaligned(out, 8))) ||
        misaligned(initial, 16) || misaligned(states, 16))
        return LRMOE_E_ARG;
    if (tokens == 0 && record) return LRMOE_OK;
    if (int d = check_device()) return d;
    lrmoe::DnRuleArgs a{};
    a.q = q;
    a.k = k;
    a.v = v;
    a.qk_stride = static_cast<int64_t>(heads) * key_width;
    a.v_stride = static_cast<int64_t>(heads) * value_width;
    a.kv_shift = 0;
    a.G = G;
    a.beta = beta;
    a.initial = initial;
    a.final_state = record ? nullptr : states;
    a.record = record ? states : nullptr;
    a.out = out;
    a.tokens = tokens;
    a.heads = heads;
    a.width = value_width;
    a.normalize = normalize ? 1 : 0;
    return status_of(lrmoe::launch_delta_rule(a, key_width, state_bf16 != 0, as_stream(stream)));
}

// Both mixer entry points; `glue` (the decoder layer's input norm and
// residual add) is all null for lrmoe_delta_mixer.
static int delta_mixer(const uint16_t* hidden, int tokens, const uint16_t* in_proj_qkv, const uint16_t* in_proj_z,
                       const uint16_t* in_proj_b, const uint16_t* in_proj_a, const uint16_t* conv_weight,
                       const uint16_t* A_log, const uint16_t* dt_bias, const uint16_t* norm_weight, float eps,
                       const uint16_t* out_proj, uint16_t* conv_state, void* state, int state_bf16,
                       uint16_t* conv_record, void* state_record, uint16_t* out, const lrmoe::AttnGlue& glue,
                       void* workspace, size_t workspace_bytes, void* stream) {
    if (tokens < 0 || tokens > lrmoe::kDeltaMaxTokens) return LRMOE_E_ARG;
    if (tokens == 0) return LRMOE_OK;
    if (!hidden || !in_proj_qkv || !in_proj_z || !in_proj_b || !in_proj_a || !conv_weight || !A_log || !dt_bias ||
        !norm_weight || !out_proj || !conv_state || !state || !out || !workspace)
        return LRMOE_E_ARG;
    if (misaligned(hidden, 16) || misaligned(in_proj_qkv, 16) || misaligned(in_proj_z, 16) ||
        misaligned(in_proj_b, 16) || misaligned(in_proj_a, 16) || misaligned(out_proj, 16) ||
        misaligned(norm_weight, 16) || misaligned(state, 16) || misaligned(state_record, 16) ||
        misaligned(conv_weight, 8) || misaligned(conv_state, 8) || misaligned(conv_record, 8) ||
        misaligned(workspace, 256))
        return LRMOE_E_ARG;
    if (workspace_bytes < lrmoe::delta_workspace_bytes(tokens)) return LRMOE_E_WORKSPACE;
    if (int d = check_device()) return d;
    lrmoe::DnProjectArgs p{};
    p.x = hidden;
    p.w_qkv = in_proj_qkv;
    p.w_z = in_proj_z;
    p.w_b = in_proj_b;
    p.w_a = in_proj_a;
    p.conv_w = conv_weight;
    p.A_log = A_log;
    p.dt_bias = dt_bias;
    p.norm_w = norm_weight;
    p.w_out = out_proj;
    p.eps = eps;
    p.conv_state = conv_state;
    p.conv_record = conv_record;
    p.out = out;
    p.tokens = tokens;
    p.in_norm = glue.in_norm;
    p.in_eps = glue.in_eps;
    p.norm_out = glue.norm_out;
    p.sum_out = glue.sum_out;
    const lrmoe::DeltaWorkspace w = lrmoe::carve_delta(workspace, tokens);
    return status_of(lrmoe::launch_delta_mixer(p, state, state_bf16 != 0, state_record, w, as_stream(stream)));
}

int lrmoe_delta_mixer(const uint16_t* hidden, int tokens, const uint16_t* in_proj_qkv, const uint16_t* in_proj_z,
                      const uint16_t* in_proj_b, const uint16_t* in_proj_a, const uint16_t* conv_weight,
                      const uint16_t* A_log, const uint16_t* dt_bias, const uint16_t* norm_weight, float eps,
                      const uint16_t* out_proj, uint16_t* conv_state, void* state, int state_bf16,
                      uint16_t* conv_record, void* state_record, uint16_t* out, void* workspace,
                      size_t workspace_bytes, void* stream) {
    return delta_mixer(hidden, tokens, in_proj_qkv, in_proj_z, in_proj_b, in_proj_a, conv_weight, A_log, dt_bias,
                       norm_weight, eps, out_proj, conv_state, state, state_bf16, conv_record, state_record, out,
                       lrmoe::AttnGlue{}, workspace, workspace_bytes, stream);
}

int lrmoe_delta_mixer_step(const uint16_t* residual, int tokens, const uint16_t* input_norm, float input_eps,
                           const uint16_t* in_proj_qkv, const uint16_t* in_proj_z, const uint16_t* in_proj_b,
                           const uint16_t* in_proj_a, const uint16_t* conv_weight, const uint16_t* A_log,
                           const uint16_t* dt_bias, const uint16_t* norm_weight, float eps, const uint16_t* out_proj,
                           uint16_t* conv_state, void* state, int state_bf16, uint16_t* conv_record,
                           void* state_record, uint16_t* out, uint16_t* sum_out, uint16_t* norm_out,
                           void* workspace, size_t workspace_bytes, void* stream) {
    if (tokens > 0 && (!input_norm || !sum_out)) return LRMOE_E_ARG;
    if (misaligned(input_norm, 16) || misaligned(sum_out, 2) || misaligned(norm_out, 16)) return LRMOE_E_ARG;
    return delta_mixer(residual, tokens, in_proj_qkv, in_proj_z, in_proj_b, in_proj_a, conv_weight, A_log, dt_bias,
                       norm_weight, eps, out_proj, conv_state, state, state_bf16, conv_record, state_record, out,
                       lrmoe::AttnGlue{input_norm, input_eps, norm_out, sum_out}, workspace, workspace_bytes,
                       stream);
}

size_t lrmoe_attn_workspace_bytes(int tokens) {
    if (tokens < 1 || tokens > lrmoe::kAttnMaxTokens) return 0;
    return lrmoe::attn_workspace_bytes(tokens);
}

// Both attention entry points: `length_dev` null runs the call at `length`
// (checked here); otherwise the kernels read the length from length_dev and
// the chunks cover `capacity`.
static int attn_decode(const uint16_t* hidden, int tokens, const uint16_t* q_proj, const uint16_t* k_proj,
                const uint16_t* v_proj, const uint16_t* o_proj, const uint16_t* q_norm, const uint16_t* k_norm,
                float eps, const uint16_t* cos, const uint16_t* sin, uint16_t* k_cache, uint16_t* v_cache,
                int capacity, int length, const int32_t* length_dev, uint16_t* out,
                const lrmoe::AttnGlue& glue, void* workspace, size_t workspace_bytes, void* stream) {
    if (tokens < 0 || tokens > lrmoe::kAttnMaxTokens || length < 0 || capacity < 1 || capacity > (1 << 22) ||
        length > capacity - tokens)
        return LRMOE_E_ARG;
    if (tokens == 0) return LRMOE_OK;
    if (length_dev != nullptr && misaligned(length_dev, 4)) return LRMOE_E_ARG;
    if (!hidden || !q_proj || !k_proj || !v_proj || !o_proj || !q_norm || !k_norm || !cos || !sin || !k_cache ||
        !v_cache || !out || !workspace)
        return LRMOE_E_ARG;
    if (misaligned(hidden, 16) || misaligned(q_proj, 16) || misaligned(k_proj, 16) || misaligned(v_proj, 16) ||
        misaligned(o_proj, 16) || misaligned(q_norm, 8) || misaligned(k_norm, 8) || misaligned(cos, 8) ||
        misaligned(sin, 8) || misaligned(k_cache, 16) || misaligned(v_cache, 16) || misaligned(out, 2) ||
        misaligned(workspace, 256))
        return LRMOE_E_ARG;
    if (workspace_bytes < lrmoe::attn_workspace_bytes(tokens)) return LRMOE_E_WORKSPACE;
    if (int d = check_device()) return d;
    const lrmoe::AttnWorkspace w = lrmoe::carve_attn(workspace, tokens);
    lrmoe::AttnArgs a{};
    a.proj = w.proj;
    a.q_norm = q_norm;
    a.k_norm = k_norm;
    a.eps = eps;
    a.cos = cos;
    a.sin = sin;
    a.k_cache = k_cache;
    a.v_cache = v_cache;
    a.capacity = capacity;
    a.length = length;
    a.length_dev = length_dev;
    a.tokens = tokens;
    const int span = length_dev != nullptr ? capacity : length + tokens;  // positions the chunks cover
    lrmoe::attn_geometry(a, tokens, span);
    a.part_o = w.part_o;
    a.part_ml = w.part_ml;
    a.att = w.att;
    return status_of(
        lrmoe::launch_attn_decode(a, hidden, q_proj, k_proj, v_proj, o_proj, out, glue, as_stream(stream)));
}

int lrmoe_attn_decode(const uint16_t* hidden, int tokens, const uint16_t* q_proj, const uint16_t* k_proj,
                      const uint16_t* v_proj, const uint16_t* o_proj, const uint16_t* q_norm, const uint16_t* k_norm,
                      float eps, const uint16_t* cos, const uint16_t* sin, uint16_t* k_cache, uint16_t* v_cache,
                      int capacity, int length, uint16_t* out, void* workspace, size_t workspace_bytes,
                      void* stream) {
    return attn_decode(hidden, tokens, q_proj, k_proj, v_proj, o_proj, q_norm, k_norm, eps, cos, sin, k_cache,
                       v_cache, capacity, length, nullptr, out, lrmoe::AttnGlue{}, workspace, workspace_bytes, stream);
}

int lrmoe_attn_decode_at(const uint16_t* hidden, int tokens, const uint16_t* q_proj, const uint16_t* k_proj,
                         const uint16_t* v_proj, const uint16_t* o_proj, const uint16_t* q_norm,
                         const uint16_t* k_norm, float eps, const uint16_t* cos, const uint16_t* sin,
                         uint16_t* k_cache, uint16_t* v_cache, int capacity, const int32_t* length, uint16_t* out,
                         void* workspace, size_t workspace_bytes, void* stream) {
    if (length == nullptr) return LRMOE_E_ARG;
    return attn_decode(hidden, tokens, q_proj, k_proj, v_proj, o_proj, q_norm, k_norm, eps, cos, sin, k_cache,
                       v_cache, capacity, 0, length, out, lrmoe::AttnGlue{}, workspace, workspace_bytes, stream);
}

int lrmoe_attn_decode_step(const uint16_t* residual, int tokens, const uint16_t* input_norm, float input_eps,
                           const uint16_t* q_proj, const uint16_t* k_proj, const uint16_t* v_proj,
                           const uint16_t* o_proj, const uint16_t* q_norm, const uint16_t* k_norm, float eps,
                           const uint16_t* cos, const uint16_t* sin, uint16_t* k_cache, uint16_t* v_cache,
                           int capacity, int length, const int32_t* length_dev, uint16_t* out, uint16_t* sum_out,
                           uint16_t* norm_out, void* workspace, size_t workspace_bytes, void* stream) {
    if (tokens > 0 && (!input_norm || !sum_out)) return LRMOE_E_ARG;
    if (misaligned(input_norm, 16) || misaligned(sum_out, 2) || misaligned(norm_out, 16)) return LRMOE_E_ARG;
    return attn_decode(residual, tokens, q_proj, k_proj, v_proj, o_proj, q_norm, k_norm, eps, cos, sin, k_cache,
                       v_cache, capacity, length_dev != nullptr ? 0 : length, length_dev, out,
                       lrmoe::AttnGlue{input_norm, input_eps, norm_out, sum_out}, workspace, workspace_bytes, stream);
}

}  // extern "C"
