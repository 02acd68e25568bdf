// The decode kernels' state in a MoE workspace (kept between calls): launch
// epochs and two parities of the exchange buffers, shared by moe_decode.hip
// (up to 8 tokens per launch) and moe_decode1.hip (one token).
//
// Epoch words: kEpochSlots 64-bit words, all equal after every launch.
// Workgroup b of a launch reads word b at its start and stores the next word
// to every word j with j % G == b at its end.  A word holds the launch count
// (bits 0-39; its parity picks the exchange buffers of the next launch) and
// the footprint of the launch that stored it: how many bytes of its parity's
// activation (bits 40-48) and partial-sum (bits 49-60) buffers it wrote, in
// 256-byte units.  The exchange buffers read "all zero" as "not yet
// written", so each launch clears what the previous launch wrote into the
// other parity (the previous launch has completed: stream order); the
// footprint bounds that clear.
#pragma once

#include <stddef.h>
#include <stdint.h>

namespace gi {
namespace moe_state {

constexpr int kEpochSlots = 1024;  // also the largest grid
constexpr size_t kActParity = (size_t)64 * 768 * 2;        // one activation exchange buffer (bytes)
constexpr size_t kPartParity = (size_t)88 * 8 * 8 * 32 * 4;  // one partial-sum exchange buffer (bytes)
constexpr int kCountBits = 40;
constexpr unsigned long long kCountMask = (1ull << kCountBits) - 1ull;
constexpr uint32_t kUnit = 256;  // footprint granule (bytes)
constexpr uint32_t kActUnitsAll = (uint32_t)(kActParity / kUnit);    // 384: 9 bits
constexpr uint32_t kPartUnitsAll = (uint32_t)(kPartParity / kUnit);  // 2816: 12 bits
static_assert(kActUnitsAll < 512 && kPartUnitsAll < 4096, "footprint fields");

constexpr size_t state_bytes() { return (size_t)kEpochSlots * 8 + 2 * kActParity + 2 * kPartParity; }
constexpr size_t act_offset() { return (size_t)kEpochSlots * 8; }
constexpr size_t part_offset() { return (size_t)kEpochSlots * 8 + 2 * kActParity; }

__host__ __device__ constexpr unsigned long long epoch_word(unsigned long long count, uint32_t act_units,
                                                            uint32_t part_units) {
  return (count & kCountMask) | ((unsigned long long)act_units << kCountBits) |
         ((unsigned long long)part_units << (kCountBits + 9));
}
__host__ __device__ constexpr unsigned long long epoch_count(unsigned long long w) { return w & kCountMask; }
__host__ __device__ constexpr uint32_t epoch_act_units(unsigned long long w) {
  return (uint32_t)(w >> kCountBits) & 511u;
}
__host__ __device__ constexpr uint32_t epoch_part_units(unsigned long long w) {
  return (uint32_t)(w >> (kCountBits + 9)) & 4095u;
}
__host__ __device__ constexpr uint32_t bytes_to_units(size_t bytes) { return (uint32_t)((bytes + kUnit - 1) / kUnit); }

}  // namespace moe_state
}  // namespace gi
