// HBM-resident expert gather (raw BF16 rows) and the synthetic generator.
//
// Gather semantics: edge35b/bf16_gather_ada.cu:36-112 as launched by
// edge35b/native_bf16_gather.py:71-77: for every copy row below the
// device-resident *count, for every bank b, fill sizes[b] bytes at
// destinations[b] + dst_ids[row]*sizes[b] from the descriptor
// descriptors[(b*experts + src_ids[row])*3] = (address, base, escapes): a raw
// row (base < 0) is copied; an escape-codec row (edge35b/bf16_expert_codec.py
// pack_row) is decoded.  The count stays on the device, so a captured graph
// replays with new counts and descriptors.
//
// On MI355X every expert row is resident in HBM, so the copy is HBM->HBM.
// Each workgroup owns one contiguous stripe of one row of one bank and moves
// it with 16-byte loads, several in flight per lane, and 16-byte stores.
#include "lrmoe_device.h"
#include "lrmoe_internal.h"

namespace lrmoe {
namespace {

constexpr int kGatherUnroll = 8;

// kStream = true: nontemporal loads and stores (the rows stream past the
// caches, the "default" policy); false: ordinary cached accesses that leave
// the rows in L2 ("l2").
// Two values of an escape-codec row: their sign|fraction bytes in bits 0..7
// and 8..15 of sf, their exponent deltas in nibbles 0 and 1 of nib, base_pair
// = base * 0x10001.  A value is sign << 15 | (base + delta) << 7 | fraction;
// base + delta <= 255, so the two halves never carry into each other.
__device__ __forceinline__ uint32_t escape_pair(uint32_t sf, uint32_t nib, uint32_t base_pair) {
    const uint32_t bytes = (sf & 0xffu) | ((sf & 0xff00u) << 8);
    const uint32_t delta = (nib & 0x0fu) | ((nib & 0xf0u) << 12);
    return ((bytes & 0x00800080u) << 8) | (bytes & 0x007f007fu) | ((base_pair + delta) << 7);
}

// First index in the sorted escape list not below value.
__device__ __forceinline__ int escape_lower_bound(const int32_t* indices, int count, int64_t value) {
    int lo = 0, hi = count;
    while (lo < hi) {
        const int mid = lo + (hi - lo) / 2;
        if (indices[mid] < value) {
            lo = mid + 1;
        } else {
            hi = mid;
        }
    }
    return lo;
}

// Escape-codec row of n = row_bytes / 2 values (bf16_expert_codec.py:37-60):
// bytes [0, n) sign|fraction, [n, 3n/2) exponent deltas from base (value 2i
// in the low nibble of byte i), then `escapes` sorted int32 indices and their
// raw 16-bit values.  The workgroup decodes its units [begin, end) (8 values
// each), waits for those stores, then writes the escapes inside its units.
template <bool kStream>
__device__ __forceinline__ void gather_escape_row(const uint8_t* src, int base, int escapes, int64_t row_bytes,
                                                  u32x4* dst, int64_t begin, int64_t end) {
    const int64_t n = row_bytes / 2;
    typedef unsigned int u32x2 __attribute__((ext_vector_type(2)));
    const u32x2* sf = reinterpret_cast<const u32x2*>(src);
    const uint32_t* deltas = reinterpret_cast<const uint32_t*>(src + n);
    const uint32_t base_pair = static_cast<uint32_t>(base) * 0x10001u;
    auto decode = [&](const u32x2& s, uint32_t d) {
        u32x4 v;
        v.x = escape_pair(s.x, d, base_pair);
        v.y = escape_pair(s.x >> 16, d >> 8, base_pair);
        v.z = escape_pair(s.y, d >> 16, base_pair);
        v.w = escape_pair(s.y >> 16, d >> 24, base_pair);
        return v;
    };
    // Four units' loads in flight per lane, then the rest one at a time.
    constexpr int kUnits = 4;
    int64_t i = begin + threadIdx.x;
    for (; i + (kUnits - 1) * blockDim.x < end; i += kUnits * blockDim.x) {
        u32x2 s[kUnits];
        uint32_t d[kUnits];
#pragma unroll
        for (int u = 0; u < kUnits; ++u) {
            s[u] = kStream ? __builtin_nontemporal_load(sf + i + u * blockDim.x) : sf[i + u * blockDim.x];
            d[u] = kStream ? __builtin_nontemporal_load(deltas + i + u * blockDim.x) : deltas[i + u * blockDim.x];
        }
#pragma unroll
        for (int u = 0; u < kUnits; ++u) dst[i + u * blockDim.x] = decode(s[u], d[u]);
    }
    for (; i < end; i += blockDim.x) {
        const u32x2 s = kStream ? __builtin_nontemporal_load(sf + i) : sf[i];
        const uint32_t d = kStream ? __builtin_nontemporal_load(deltas + i) : deltas[i];
        dst[i] = decode(s, d);
    }
    if (escapes <= 0) return;
    const int32_t* indices = reinterpret_cast<const int32_t*>(src + n + n / 2);
    const uint16_t* values = reinterpret_cast<const uint16_t*>(indices + escapes);
    __shared__ int range[2];
    if (threadIdx.x == 0) {
        range[0] = escape_lower_bound(indices, escapes, begin * 8);
        range[1] = escape_lower_bound(indices, escapes, end * 8);
    }
    __syncthreads();  // also orders this workgroup's decoded stores before the escapes
    uint16_t* out = reinterpret_cast<uint16_t*>(dst);
    for (int j = range[0] + static_cast<int>(threadIdx.x); j < range[1]; j += blockDim.x) out[indices[j]] = values[j];
}

template <bool kStream>
__global__ __launch_bounds__(256) void gather_kernel(const int64_t* descriptors, const int64_t* destinations,
                                                     const int64_t* sizes, const int32_t* src_ids,
                                                     const int32_t* dst_ids, const int64_t* count, int experts,
                                                     int32_t* status) {
    const int stripe = blockIdx.x;
    const int bank = blockIdx.y;
    const int row = blockIdx.z;
    if (row >= *count) return;
    const int64_t* desc = descriptors + (static_cast<int64_t>(bank) * experts + src_ids[row]) * 3;
    const u32x4* src = reinterpret_cast<const u32x4*>(desc[0]);
    const int64_t row_bytes = sizes[bank];
    u32x4* dst = reinterpret_cast<u32x4*>(destinations[bank] + static_cast<int64_t>(dst_ids[row]) * row_bytes);
    const int64_t units = row_bytes >> 4;
    const int64_t per = (units + gridDim.x - 1) / gridDim.x;
    const int64_t begin = stripe * per;
    const int64_t end = begin + per < units ? begin + per : units;
    if (desc[1] >= 0) {
        if (threadIdx.x == 0 && stripe == 0 && status != nullptr) atomicOr(status, kStatusCodecRow);
        gather_escape_row<kStream>(reinterpret_cast<const uint8_t*>(desc[0]), static_cast<int>(desc[1]),
                                   static_cast<int>(desc[2]), row_bytes, dst, begin, end);
        return;
    }
    const int64_t step = static_cast<int64_t>(blockDim.x) * kGatherUnroll;
    int64_t i = begin + threadIdx.x;
    for (; i + (kGatherUnroll - 1) * blockDim.x < end; i += step) {
        u32x4 v[kGatherUnroll];
#pragma unroll
        for (int u = 0; u < kGatherUnroll; ++u) {
            v[u] = kStream ? __builtin_nontemporal_load(src + i + u * blockDim.x) : src[i + u * blockDim.x];
        }
#pragma unroll
        for (int u = 0; u < kGatherUnroll; ++u) {
            if (kStream) {
                __builtin_nontemporal_store(v[u], dst + i + u * blockDim.x);
            } else {
                dst[i + u * blockDim.x] = v[u];
            }
        }
    }
    for (; i < end; i += blockDim.x) dst[i] = src[i];
}

// Eight values of a codec tile in the reference's byte order
// (cpu_bf16_reads.h:16-52): the low bytes of values 0..3 in low0 and of 4..7
// in low1, the codes of values 2i and 2i+1 in the low and high nibble of byte
// i of `codes`, base4 = base * 0x01010101.  The high bytes of the even and
// of the odd values come four at a time (no byte carries: a field is at most
// 127), v_perm_b32 puts them in value order and then beside the low bytes.
__device__ __forceinline__ u32x4 ref_tile_decode8(uint32_t low0, uint32_t low1, uint32_t codes, uint32_t base4) {
    const uint32_t even = ((codes & 0x07070707u) + base4) | ((codes << 4) & 0x80808080u);
    const uint32_t odd = (((codes >> 4) & 0x07070707u) + base4) | (codes & 0x80808080u);
    const uint32_t h03 = __builtin_amdgcn_perm(odd, even, 0x05010400u);
    const uint32_t h47 = __builtin_amdgcn_perm(odd, even, 0x07030602u);
    u32x4 v;
    v.x = __builtin_amdgcn_perm(h03, low0, 0x05010400u);
    v.y = __builtin_amdgcn_perm(h03, low0, 0x07030602u);
    v.z = __builtin_amdgcn_perm(h47, low1, 0x05010400u);
    v.w = __builtin_amdgcn_perm(h47, low1, 0x07030602u);
    return v;
}

// Rows in the tile codec (edge35b/bf16_gather_ada.cu:127-180,
// gather_cpu_tiles), with the launch protocol of gather_kernel.  Descriptor
// (packed, bases, raw): bases 0 copies the raw row; otherwise tile t of the
// row (512 bytes) has base bases[t] (one byte) and 384 packed bytes at
// packed + 384t, or is copied from raw + 512t when its base is 255.  With
// kCompact and raw == -1 (the reference's "resident" rows): bases holds a
// 32-bit header per tile, (tiles read raw before it) << 8 | base, the tile's
// bytes start at packed + 384t + 128 * (tiles read raw before it), and a raw
// tile's 512 bytes are stored there.  Half a wave per tile, 16 bytes per
// lane; every tile of the row is covered (stripes of ceil(tiles / stripes)).
template <bool kCompact>
__global__ __launch_bounds__(256) void gather_tiles_kernel(const int64_t* descriptors, const int64_t* destinations,
                                                           const int64_t* sizes, const int32_t* src_ids,
                                                           const int32_t* dst_ids, const int64_t* count,
                                                           int experts) {
    const int stripe = blockIdx.x;
    const int bank = blockIdx.y;
    const int row = blockIdx.z;
    if (row >= *count) return;
    const int64_t* desc = descriptors + (static_cast<int64_t>(bank) * experts + src_ids[row]) * 3;
    const uint8_t* packed = reinterpret_cast<const uint8_t*>(desc[0]);
    const uint8_t* bases = reinterpret_cast<const uint8_t*>(desc[1]);
    const int64_t raw_at = desc[2];
    const int64_t row_bytes = sizes[bank];
    u32x4* dst = reinterpret_cast<u32x4*>(destinations[bank] + static_cast<int64_t>(dst_ids[row]) * row_bytes);
    const int64_t tiles = row_bytes / 512;
    const int64_t per = (tiles + gridDim.x - 1) / gridDim.x;
    const int64_t begin = stripe * per;
    const int64_t end = begin + per < tiles ? begin + per : tiles;
    if (bases == nullptr) {
        const u32x4* raw = reinterpret_cast<const u32x4*>(raw_at);
        for (int64_t i = begin * 32 + threadIdx.x; i < end * 32; i += blockDim.x) dst[i] = raw[i];
        return;
    }
    const bool compact = kCompact && raw_at == -1;
    const u32x4* raw = reinterpret_cast<const u32x4*>(raw_at);
    const int lane = threadIdx.x & 31;
    const int64_t step = blockDim.x >> 5;
    int64_t tile = begin + (threadIdx.x >> 5);
    if (!compact) {
        // Every tile has its 384 bytes at packed + 384t, so a tile's loads do
        // not wait for its base: four tiles' loads in flight per lane.
        constexpr int kTiles = 4;
        for (; tile + (kTiles - 1) * step < end; tile += kTiles * step) {
            uint32_t base[kTiles], codes[kTiles];
            uint2 low[kTiles];
#pragma unroll
            for (int u = 0; u < kTiles; ++u) {
                const int64_t t = tile + u * step;
                base[u] = bases[t];
                low[u] = *reinterpret_cast<const uint2*>(packed + t * 384 + 8 * lane);
                codes[u] = *reinterpret_cast<const uint32_t*>(packed + t * 384 + 256 + 4 * lane);
            }
#pragma unroll
            for (int u = 0; u < kTiles; ++u) {
                const int64_t i = (tile + u * step) * 32 + lane;
                dst[i] = base[u] == 255u ? raw[i]
                                         : ref_tile_decode8(low[u].x, low[u].y, codes[u], base[u] * 0x01010101u);
            }
        }
    }
    for (; tile < end; tile += step) {
        const uint32_t header = compact ? reinterpret_cast<const uint32_t*>(bases)[tile] : bases[tile];
        const uint32_t base = compact ? header & 255u : header;
        const uint8_t* data = packed + tile * 384 + (compact ? static_cast<int64_t>(header >> 8) * 128 : 0);
        const int64_t i = tile * 32 + lane;
        if (base == 255u) {
            dst[i] = compact ? reinterpret_cast<const u32x4*>(data)[lane] : raw[i];
            continue;
        }
        const uint2 low = *reinterpret_cast<const uint2*>(data + 8 * lane);
        const uint32_t codes = *reinterpret_cast<const uint32_t*>(data + 256 + 4 * lane);
        dst[i] = ref_tile_decode8(low.x, low.y, codes, base * 0x01010101u);
    }
}

// Counter-based synthetic bf16 ~N(0, sigma): h = splitmix64(key + index),
// key = splitmix64(seed * 0x9E3779B97F4A7C15 + stream); Irwin-Hall sum of the
// four 16-bit fields of h, centred and scaled to unit variance in double,
// times sigma, rounded to float and then to bf16.  Integer and IEEE double
// operations only, so any host can regenerate a tensor bit-for-bit.
__device__ __forceinline__ uint64_t splitmix64(uint64_t z) {
    z += 0x9E3779B97F4A7C15ull;
    z = (z ^ (z >> 30)) * 0xBF58476D1CE4E5B9ull;
    z = (z ^ (z >> 27)) * 0x94D049BB133111EBull;
    return z ^ (z >> 31);
}

__global__ __launch_bounds__(256) void fill_normal_kernel(uint16_t* out, int64_t count, uint64_t key, double inv_std,
                                                          double sigma, int64_t first) {
    const int64_t stride = static_cast<int64_t>(gridDim.x) * blockDim.x;
    for (int64_t i = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x; i < count; i += stride) {
        const uint64_t h = splitmix64(key + static_cast<uint64_t>(first + i));
        const int64_t s = static_cast<int64_t>(h & 0xffff) + static_cast<int64_t>((h >> 16) & 0xffff) +
                          static_cast<int64_t>((h >> 32) & 0xffff) + static_cast<int64_t>(h >> 48);
        const double z = (static_cast<double>(s) - 131070.0) * inv_std;
        out[i] = static_cast<uint16_t>(f2bf(static_cast<float>(z * sigma)));
    }
}

uint64_t host_splitmix64(uint64_t z) {
    z += 0x9E3779B97F4A7C15ull;
    z = (z ^ (z >> 30)) * 0xBF58476D1CE4E5B9ull;
    z = (z ^ (z >> 27)) * 0x94D049BB133111EBull;
    return z ^ (z >> 31);
}

}  // namespace

hipError_t launch_gather(const int64_t* descriptors, const int64_t* destinations, const int64_t* sizes,
                         const int32_t* src_ids, const int32_t* dst_ids, const int64_t* count, int experts, int banks,
                         int max_copies, int stripes, int threads, int keep_in_l2, int32_t* status,
                         hipStream_t stream) {
    if (max_copies <= 0 || banks <= 0) return hipSuccess;
    const StageEvents ev = timing_events(kStageGather);
    const dim3 grid(stripes, banks, max_copies);
    if (keep_in_l2) {
        LRMOE_LAUNCH(gather_kernel<false>, grid, dim3(threads), 0, stream, ev.start, ev.stop, descriptors,
                     destinations, sizes, src_ids, dst_ids, count, experts, status);
    } else {
        LRMOE_LAUNCH(gather_kernel<true>, grid, dim3(threads), 0, stream, ev.start, ev.stop, descriptors,
                     destinations, sizes, src_ids, dst_ids, count, experts, status);
    }
    return hipGetLastError();
}

hipError_t launch_gather_tiles(const int64_t* descriptors, const int64_t* destinations, const int64_t* sizes,
                               const int32_t* src_ids, const int32_t* dst_ids, const int64_t* count, int experts,
                               int banks, int max_copies, int stripes, int threads, int compact, hipStream_t stream) {
    if (max_copies <= 0 || banks <= 0) return hipSuccess;
    const StageEvents ev = timing_events(kStageGather);
    const dim3 grid(stripes, banks, max_copies);
    if (compact) {
        LRMOE_LAUNCH(gather_tiles_kernel<true>, grid, dim3(threads), 0, stream, ev.start, ev.stop, descriptors,
                     destinations, sizes, src_ids, dst_ids, count, experts);
    } else {
        LRMOE_LAUNCH(gather_tiles_kernel<false>, grid, dim3(threads), 0, stream, ev.start, ev.stop, descriptors,
                     destinations, sizes, src_ids, dst_ids, count, experts);
    }
    return hipGetLastError();
}

hipError_t launch_fill_normal(uint16_t* out, int64_t count, uint64_t seed, uint64_t stream_id, double sigma,
                              int64_t first, hipStream_t stream) {
    if (count <= 0) return hipSuccess;
    const uint64_t key = host_splitmix64(seed * 0x9E3779B97F4A7C15ull + stream_id);
    const double inv_std = 1.0 / __builtin_sqrt(1431655765.0);
    int64_t blocks = (count + 255) / 256;
    if (blocks > 65536) blocks = 65536;
    hipLaunchKernelGGL(fill_normal_kernel, dim3(static_cast<unsigned>(blocks)), dim3(256), 0, stream, out, count, key,
                       inv_std, sigma, first);
    return hipGetLastError();
}

}  // namespace lrmoe
