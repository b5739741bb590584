// Test infrastructure only: exports the reference's tile packer
// (edge35b/cpu_bf16_reads.h:16-52, pack_cpu_read_tiles) with a C symbol so
// that the oracle's codec restatement can be checked against it.  The header
// is compiled where it lies (oracle/Makefile adds its directory to the include
// path); nothing of it is copied.
#include <cstddef>
#include <cstdint>

#include "cpu_bf16_reads.h"

// Returns the number of tiles packed (the rest keep base 255, the raw marker),
// or -1 when the reference's own bit audit rejects a tile.
extern "C" int64_t ref_pack_cpu_read_tiles(const uint16_t* raw, uint8_t* packed, uint8_t* bases, size_t tiles) {
    try {
        return static_cast<int64_t>(freetoken::cpu_moe::pack_cpu_read_tiles(raw, packed, bases, tiles));
    } catch (...) {
        return -1;
    }
}
