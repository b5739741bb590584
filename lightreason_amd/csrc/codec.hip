// Lossless BF16 tile codec in the decode kernel's layout.
//
// Format of the reference's tile packer (edge35b/cpu_bf16_reads.h:16-52,
// pack_cpu_read_tiles; decoded by bf16_gather_ada.cu:117-123): a row is cut
// into tiles of 256 values; base = the smallest 7-bit field (bits 14..8) of a
// tile's values, and a tile whose fields span more than 8 values does not fit
// (base 255, the reference's raw marker).  Each value keeps its low byte and
// the 4-bit code (field - base) | (sign << 3): 384 bytes per 512-byte tile.
//
// Byte order (not the reference's index order): value k = 8g + 32s + j of a
// tile (g 0..3, s 0..7, j 0..7) has its low byte at 64(s/2) + 16g + 8(s%2) + j
// and its code in nibble j/4 (low nibble first) of byte 256 + 64(s/4) + 16g +
// 4(s%4) + j%4 (so that one shift separates the codes of values 0..3 from
// those of 4..7).  An MFMA lane of k-group g then reads its 8 k-steps of a tile
// as six 16-byte blocks at 16g + 64i (i = 0..5), in the same k order as a raw
// row, and those of the row's next tile at 16g + 64i for i = 6..11: the same
// offsets as its raw loads (moe_decode's items).
#include "lrmoe_device.h"
#include "lrmoe_internal.h"

namespace lrmoe {
namespace {

constexpr int kPackThreads = 256;
constexpr int kTilesPerWave = 2;  // 32 lanes per tile
constexpr int kTilesPerBlock = kPackThreads / kWave * kTilesPerWave;

// Lane (half h, g, s) of a wave handles values 8g + 32s .. +7 of tile
// 2 * wave_index + h.
struct TileLane {
    int64_t tile;
    int g;
    int s;
    bool valid;
};

__device__ __forceinline__ TileLane tile_lane(int64_t total_tiles) {
    const int lane = threadIdx.x & 63;
    const int64_t wave = static_cast<int64_t>(blockIdx.x) * (kPackThreads / kWave) + (threadIdx.x >> 6);
    TileLane t;
    t.tile = kTilesPerWave * wave + (lane >> 5);
    t.g = (lane >> 3) & 3;
    t.s = lane & 7;
    t.valid = t.tile < total_tiles;
    return t;
}

// Bytes of a lane's 8 low bytes and 4 code bytes within its tile.
__device__ __forceinline__ int low_offset(const TileLane& t) { return 64 * (t.s >> 1) + 16 * t.g + 8 * (t.s & 1); }
__device__ __forceinline__ int code_offset(const TileLane& t) { return 256 + 64 * (t.s >> 2) + 16 * t.g + 4 * (t.s & 3); }

// Minimum and maximum over the 32 lanes of a half wave.
__device__ __forceinline__ void half_min_max(int& lo, int& hi) {
#pragma unroll
    for (int o = 1; o < 32; o <<= 1) {
        lo = min(lo, __shfl_xor(lo, o, kWave));
        hi = max(hi, __shfl_xor(hi, o, kWave));
    }
}

__global__ __launch_bounds__(kPackThreads) void codec_pack(const uint16_t* w, int64_t total_tiles, int tiles_per_row,
                                                           int cols, uint8_t* packed, uint8_t* bases,
                                                           unsigned long long* misfit) {
    const TileLane t = tile_lane(total_tiles);
    const int64_t row = t.valid ? t.tile / tiles_per_row : 0;
    const int64_t col = t.valid ? (t.tile % tiles_per_row) * kCodecTile : 0;
    const int k0 = 8 * t.g + 32 * t.s;
    uint4 v = make_uint4(0u, 0u, 0u, 0u);
    if (t.valid) v = ldg16(w + row * cols + col + k0);
    const uint32_t word[4] = {v.x, v.y, v.z, v.w};
    int lo = 127, hi = 0;
#pragma unroll
    for (int i = 0; i < 8; ++i) {
        const int field = static_cast<int>((word[i >> 1] >> (16 * (i & 1) + 8)) & 127u);
        lo = min(lo, field);
        hi = max(hi, field);
    }
    half_min_max(lo, hi);
    if (!t.valid) return;
    uint8_t* out = packed + t.tile * kCodecTileBytes;
    const bool fits = hi - lo <= 7;
    uint32_t low[2] = {0u, 0u};
    uint32_t codes = 0u;
    if (fits) {
#pragma unroll
        for (int i = 0; i < 8; ++i) {
            const uint32_t bits = (word[i >> 1] >> (16 * (i & 1))) & 0xffffu;
            low[i >> 2] |= (bits & 0xffu) << (8 * (i & 3));
            const uint32_t code = (((bits >> 8) & 127u) - static_cast<uint32_t>(lo)) | ((bits >> 15) << 3);
            codes |= code << (8 * (i & 3) + 4 * (i >> 2));
        }
    }
    *reinterpret_cast<uint2*>(out + low_offset(t)) = make_uint2(low[0], low[1]);
    *reinterpret_cast<uint32_t*>(out + code_offset(t)) = codes;
    if ((threadIdx.x & 31) == 0) {
        bases[t.tile] = fits ? static_cast<uint8_t>(lo) : static_cast<uint8_t>(kCodecMisfit);
        if (!fits && misfit != nullptr) atomicAdd(misfit, 1ull);
    }
}

__global__ __launch_bounds__(kPackThreads) void codec_unpack(const uint8_t* packed, const uint8_t* bases,
                                                             int64_t total_tiles, int tiles_per_row, int cols,
                                                             uint16_t* w) {
    const TileLane t = tile_lane(total_tiles);
    if (!t.valid) return;
    const int64_t row = t.tile / tiles_per_row;
    const int64_t col = (t.tile % tiles_per_row) * kCodecTile;
    const uint8_t* in = packed + t.tile * kCodecTileBytes;
    const uint32_t base = bases[t.tile];
    uint4 out;
    if (base == kCodecMisfit) {
        out = make_uint4(0xffffffffu, 0xffffffffu, 0xffffffffu, 0xffffffffu);
    } else {
        const uint2 low = *reinterpret_cast<const uint2*>(in + low_offset(t));
        const uint32_t codes = *reinterpret_cast<const uint32_t*>(in + code_offset(t));
        out = codec_decode8(low.x, low.y, codes, base * 0x01010101u);
    }
    *reinterpret_cast<uint4*>(w + row * cols + col + 8 * t.g + 32 * t.s) = out;
}

}  // namespace

hipError_t launch_codec_pack(const uint16_t* w, int64_t rows, int cols, uint8_t* packed, uint8_t* bases,
                             unsigned long long* misfit, hipStream_t stream) {
    const int tiles_per_row = cols / kCodecTile;
    const int64_t total = rows * tiles_per_row;
    if (total == 0) return hipSuccess;
    const int64_t blocks = (total + kTilesPerBlock - 1) / kTilesPerBlock;
    hipLaunchKernelGGL(codec_pack, dim3(static_cast<unsigned>(blocks)), dim3(kPackThreads), 0, stream, w, total,
                       tiles_per_row, cols, packed, bases, misfit);
    return hipGetLastError();
}

hipError_t launch_codec_unpack(const uint8_t* packed, const uint8_t* bases, int64_t rows, int cols, uint16_t* w,
                               hipStream_t stream) {
    const int tiles_per_row = cols / kCodecTile;
    const int64_t total = rows * tiles_per_row;
    if (total == 0) return hipSuccess;
    const int64_t blocks = (total + kTilesPerBlock - 1) / kTilesPerBlock;
    hipLaunchKernelGGL(codec_unpack, dim3(static_cast<unsigned>(blocks)), dim3(kPackThreads), 0, stream, packed,
                       bases, total, tiles_per_row, cols, w);
    return hipGetLastError();
}

}  // namespace lrmoe
