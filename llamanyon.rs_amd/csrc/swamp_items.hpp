// swamp_items.hpp -- raw loads of one 64-weight "item" of a quantized row.
//
// An item is two Q4_0 blocks (36 B), two Q8_0 blocks (68 B), one quarter
// of a Q4_K super-block (its 16-byte header + 32 nibble bytes) or one
// quarter of a Q6_K block.  Rows of n_cols % 64 == 0 (Q4_0/Q8_0), % 256 == 0
// (Q4_K) or % 512 == 0 (Q6_K) start at 4-byte (Q4_0, Q8_0, Q6_K) or 16-byte
// (Q4_K) aligned offsets from an aligned base, so every access below is a
// dword-aligned vector load.
#pragma once

#include "swamp_common.hpp"

namespace swamp {

// A Q6_K block is 210 bytes, so in a row of an even number of blocks (a
// 4-byte aligned row) the odd blocks start 2 bytes past a dword boundary.
// A Q6_K item (block b, quarter q: half h = q >> 1, columns i = q & 1)
// loads dword-aligned windows that start at (field address) & ~3 and are
// one dword longer than the field; item_dot shifts them by the block's
// misalignment (0 or 2 bytes, from b's parity).  Fields of the item, as
// byte offsets in the block:
//   qlA = 64h + 16i (16 B)   low nibbles: q1, high nibbles: q3
//   qlB = qlA + 32  (16 B)   low nibbles: q2, high nibbles: q4
//   qh  = 128 + 32h + 16i (16 B)
//   sc  = 192 + 8h  (8 B: the item uses sc[8h + i + 2j], j < 4; 12-byte window)
//   d   = 208 (2 B)
// Every window lies inside the block, or for an even block inside the
// next one, which exists because the row has an even number of blocks.

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
template <>
struct Raw<SWAMP_Q6_K> {
  uint32_t a[5];  // qlA window
  uint32_t b[5];  // qlB window
  uint32_t h[5];  // qh window
  uint32_t s[3];  // scale window
  uint32_t d;     // the dword holding d
};

// Byte offset of item `item` within its row (32-bit: rows are < 4 GiB), so
// that loads take the uniform row pointer as a scalar base plus this
// per-lane offset (global_load ... saddr), keeping no 64-bit address VGPRs.
template <int DT>
__device__ __forceinline__ uint32_t item_offset(int item) {
  if constexpr (DT == SWAMP_Q4_0) return uint32_t(item) * 36u;
  else if constexpr (DT == SWAMP_Q8_0) return uint32_t(item) * 68u;
  else if constexpr (DT == SWAMP_Q4_K) return uint32_t(item >> 2) * 144u + 16u + 32u * uint32_t(item & 3);
  else  // Q6_K: the aligned start of the item's qlA window
    return (uint32_t(item >> 2) * 210u & ~3u) + 64u * uint32_t((item >> 1) & 1) +
           16u * uint32_t(item & 1);
}

// Raw bytes of the item at byte offset `off` of `row` (from item_offset).
template <int DT>
__device__ __forceinline__ void load_raw_at(Raw<DT> &r, const uint8_t *row, uint32_t off, int item) {
  static_assert(DT != SWAMP_Q6_K, "Q6_K items are loaded through buffer resources");
  if constexpr (DT == SWAMP_Q4_0) {
    const uint8_t *p = row + off;
    u32x4 a = ld4(p), b = ld4(p + 16);
#pragma unroll
    for (int i = 0; i < 4; i++) { r.d[i] = a.v[i]; r.d[4 + i] = b.v[i]; }
    r.d[8] = ld1(p + 32);
  } else if constexpr (DT == SWAMP_Q8_0) {
    const uint8_t *p = row + off;
#pragma unroll
    for (int j = 0; j < 4; j++) {
      u32x4 a = ld4(p + 16 * j);
#pragma unroll
      for (int i = 0; i < 4; i++) r.d[4 * j + i] = a.v[i];
    }
    r.d[16] = ld1(p + 64);
  } else {
    const uint8_t *qs = row + off;
    const uint8_t *blk = row + (off - 16u - 32u * uint32_t(item & 3));
    uint4 h = *reinterpret_cast<const uint4 *>(blk);
    uint4 a = *reinterpret_cast<const uint4 *>(qs);
    uint4 b = *reinterpret_cast<const uint4 *>(qs + 16);
    r.h[0] = h.x; r.h[1] = h.y; r.h[2] = h.z; r.h[3] = h.w;
    r.q[0] = a.x; r.q[1] = a.y; r.q[2] = a.z; r.q[3] = a.w;
    r.q[4] = b.x; r.q[5] = b.y; r.q[6] = b.z; r.q[7] = b.w;
  }
}

// Buffer resource over [base, base + bytes): raw (untyped) dword loads,
// 32-bit data format (the gfx9 word-3 value), out-of-range reads return 0.
__device__ __forceinline__ __amdgpu_buffer_rsrc_t make_rsrc(const void *base, uint32_t bytes) {
  return __builtin_amdgcn_make_buffer_rsrc(const_cast<void *>(base), 0, int(bytes), 0x00020000);
}

typedef uint32_t u32x4v __attribute__((ext_vector_type(4)));
typedef uint32_t u32x3v __attribute__((ext_vector_type(3)));

// Raw bytes of one item through a buffer resource: the per-lane item offset
// in a VGPR (voff) and the per-row offset in an SGPR (soff), so one row
// pointer per tile (in the descriptor) serves every load of the tile.
template <int DT>
__device__ __forceinline__ void load_raw_buf(Raw<DT> &r, __amdgpu_buffer_rsrc_t rs, uint32_t voff,
                                             uint32_t soff, int item) {
  if constexpr (DT == SWAMP_Q4_0) {
    const u32x4v a = __builtin_amdgcn_raw_buffer_load_b128(rs, voff, soff, 0);
    const u32x4v b = __builtin_amdgcn_raw_buffer_load_b128(rs, voff + 16, soff, 0);
#pragma unroll
    for (int i = 0; i < 4; i++) { r.d[i] = a[i]; r.d[4 + i] = b[i]; }
    r.d[8] = __builtin_amdgcn_raw_buffer_load_b32(rs, voff + 32, soff, 0);
  } else if constexpr (DT == SWAMP_Q8_0) {
#pragma unroll
    for (int j = 0; j < 4; j++) {
      const u32x4v a = __builtin_amdgcn_raw_buffer_load_b128(rs, voff + 16 * j, soff, 0);
#pragma unroll
      for (int i = 0; i < 4; i++) r.d[4 * j + i] = a[i];
    }
    r.d[16] = __builtin_amdgcn_raw_buffer_load_b32(rs, voff + 64, soff, 0);
  } else if constexpr (DT == SWAMP_Q4_K) {
    const uint32_t hoff = voff - 16u - 32u * uint32_t(item & 3);
    const u32x4v h = __builtin_amdgcn_raw_buffer_load_b128(rs, hoff, soff, 0);
    const u32x4v a = __builtin_amdgcn_raw_buffer_load_b128(rs, voff, soff, 0);
    const u32x4v b = __builtin_amdgcn_raw_buffer_load_b128(rs, voff + 16, soff, 0);
#pragma unroll
    for (int i = 0; i < 4; i++) { r.h[i] = h[i]; r.q[i] = a[i]; r.q[4 + i] = b[i]; }
  } else {
    // voff = aligned block start ab + 64h + 16i (item_offset)
    const uint32_t hh = uint32_t((item >> 1) & 1), ii = uint32_t(item & 1);
    const uint32_t ab = voff - 64u * hh - 16u * ii;
    const uint32_t qh = ab + 128u + 32u * hh + 16u * ii;
    const u32x4v a = __builtin_amdgcn_raw_buffer_load_b128(rs, voff, soff, 0);
    const uint32_t a4 = __builtin_amdgcn_raw_buffer_load_b32(rs, voff + 16, soff, 0);
    const u32x4v b = __builtin_amdgcn_raw_buffer_load_b128(rs, voff + 32, soff, 0);
    const uint32_t b4 = __builtin_amdgcn_raw_buffer_load_b32(rs, voff + 48, soff, 0);
    const u32x4v h = __builtin_amdgcn_raw_buffer_load_b128(rs, qh, soff, 0);
    const uint32_t h4 = __builtin_amdgcn_raw_buffer_load_b32(rs, qh + 16, soff, 0);
    const u32x3v sw = __builtin_amdgcn_raw_buffer_load_b96(rs, ab + 192u + 8u * hh, soff, 0);
    r.d = __builtin_amdgcn_raw_buffer_load_b32(rs, ab + 208u, soff, 0);
#pragma unroll
    for (int i = 0; i < 4; i++) { r.a[i] = a[i]; r.b[i] = b[i]; r.h[i] = h[i]; }
    r.a[4] = a4; r.b[4] = b4; r.h[4] = h4;
    r.s[0] = sw[0]; r.s[1] = sw[1]; r.s[2] = sw[2];
  }
}

template <int DT>
__device__ __forceinline__ void load_raw(Raw<DT> &r, const uint8_t *row, int item) {
  load_raw_at<DT>(r, row, item_offset<DT>(item), item);
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
