// swamp_items.hpp -- raw loads of one 64-weight "item" of a quantized row.
//
// An item is two Q4_0 blocks (36 B), two Q8_0 blocks (68 B) or one quarter
// of a Q4_K super-block (its 16-byte header + 32 nibble bytes).  Rows of
// n_cols % 64 == 0 (Q4_0/Q8_0) or % 256 == 0 (Q4_K) start at 4-byte (Q4_0,
// Q8_0) or 16-byte (Q4_K) aligned offsets from an aligned base, so every
// access below is a dword-aligned vector load.
#pragma once

#include "swamp_common.hpp"

namespace swamp {

// Raw bytes of one item, loaded with dword-aligned vector loads.
template <int DT>
struct Raw;
template <>
struct Raw<SWAMP_Q4_0> {
  uint32_t d[9];
};
template <>
struct Raw<SWAMP_Q8_0> {
  uint32_t d[17];
};
template <>
struct Raw<SWAMP_Q4_K> {
  uint32_t h[4];  // d, dmin, 12 scale bytes
  uint32_t q[8];  // 32 nibble bytes of the quarter
};

template <int DT>
__device__ __forceinline__ void load_raw(Raw<DT> &r, const uint8_t *row, int item) {
  if constexpr (DT == SWAMP_Q4_0) {
    const uint8_t *p = row + size_t(item) * 36;
    u32x4 a = ld4(p), b = ld4(p + 16);
#pragma unroll
    for (int i = 0; i < 4; i++) { r.d[i] = a.v[i]; r.d[4 + i] = b.v[i]; }
    r.d[8] = ld1(p + 32);
  } else if constexpr (DT == SWAMP_Q8_0) {
    const uint8_t *p = row + size_t(item) * 68;
#pragma unroll
    for (int j = 0; j < 4; j++) {
      u32x4 a = ld4(p + 16 * j);
#pragma unroll
      for (int i = 0; i < 4; i++) r.d[4 * j + i] = a.v[i];
    }
    r.d[16] = ld1(p + 64);
  } else {
    const uint8_t *blk = row + size_t(item >> 2) * 144;
    const uint8_t *qs = blk + 16 + 32 * (item & 3);
    uint4 h = *reinterpret_cast<const uint4 *>(blk);
    uint4 a = *reinterpret_cast<const uint4 *>(qs);
    uint4 b = *reinterpret_cast<const uint4 *>(qs + 16);
    r.h[0] = h.x; r.h[1] = h.y; r.h[2] = h.z; r.h[3] = h.w;
    r.q[0] = a.x; r.q[1] = a.y; r.q[2] = a.z; r.q[3] = a.w;
    r.q[4] = b.x; r.q[5] = b.y; r.q[6] = b.z; r.q[7] = b.w;
  }
}

__device__ __forceinline__ uint32_t shr16(uint32_t hi, uint32_t lo) {
  return __builtin_amdgcn_alignbyte(hi, lo, 2);  // bytes lo[2..3], hi[0..1]
}

// Q4_K sub-block scale/min codes for sub-blocks j and j+1 (j even) from the
// 12 packed bytes (q4_k.rs:37-53).
__device__ __forceinline__ void q4k_scales(const uint32_t *h, int j, uint32_t &sc0,
                                           uint32_t &m0, uint32_t &sc1, uint32_t &m1) {
  const uint32_t s03 = h[1], s47 = h[2], s811 = h[3];
  auto get = [&](int sb, uint32_t &sc, uint32_t &mn) {
    if (sb < 4) {
      sc = (s03 >> (8 * sb)) & 63u;
      mn = (s47 >> (8 * sb)) & 63u;
    } else {
      const int k = sb - 4;
      const uint32_t b8 = (s811 >> (8 * k)) & 0xFFu;
      sc = (b8 & 0xFu) | (((s03 >> (8 * k)) & 0xC0u) >> 2);
      mn = (b8 >> 4) | (((s47 >> (8 * k)) & 0xC0u) >> 2);
    }
  };
  get(j, sc0, m0);
  get(j + 1, sc1, m1);
}

}  // namespace swamp
