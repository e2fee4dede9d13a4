// gemm.hip -- prefill GEMM on the matrix cores, and on-device Q8_0
// activation quantization.
//
// Replaces the prefill use of forward_linear_batch
// (swamp-engine/src/executor.rs:106-110 -> linear.rs:176-239): the reference
// runs the batched CPU GEMV token block by token block; here one launch
// computes y[m][r] = sum_k W[r,k] x[m][k] for the whole prompt.
//
// bf16 path (MFMA-bound: 2*M*N*K flops over ~0.56 B/weight + 2 B/act):
//  * Workgroup tile 256 tokens x 256 weight rows (or a 128-token half tile,
//    below), K step 64 (one 64-weight item per row), 8 waves = two per
//    SIMD.  Wave w owns weight rows [32w, 32w + 32) and every token of the
//    tile: 8 V_MFMA_F32_32X32X16_BF16 tiles, 128 fp32 accumulators.
//  * Weights never touch LDS.  Each wave loads its own rows' items two K
//    steps ahead and dequantizes them one step ahead straight into the
//    B-operand layout (lane l: row 32w + l%32, in a k order -- shared with
//    the activation reads -- that lets a lane load only the part of the
//    item it uses: one Q4_0 / Q8_0 block, half a Q4_K quarter with its
//    header; 2, 3, 2 loads per step), and every weight is converted once
//    per tile.  With two
//    waves per SIMD, one wave's dequantization issues while the other's
//    MFMAs run (vector ALU work issued by the wave that also issues the
//    MFMAs stretches the MFMA cadence; another wave's does not).
//  * Activations: five LDS stages filled by direct-to-LDS DMA
//    (buffer_load ... lds, no VGPRs) four K steps ahead; 128-byte rows
//    with 16-byte chunks XOR-swizzled by (row / 2) % 8.  Each A fragment
//    is re-read into its register right after the MFMA that consumed it.
//    One barrier per K step; its wait covers the loads issued before the
//    previous step (the memory counter is in order), so two steps of
//    loads stay in flight.
//  * Dequantization is q * s + o rounded once in fp32 by an fma (exact up
//    to that rounding) and then to bf16: the same B values as the
//    dequantization kernels produce, rounded to bf16.  Nibble codes reach
//    fp32 two per instruction through gfx950's scaled fp8 convert (a byte
//    below 16 read as E4M3 is the integer times 2^-9; the scale operand
//    supplies 2^9): low nibbles masked in place, high ones shifted down.
//  * Tile order: groups of 4 token tiles, consecutive tiles walking the
//    weight columns of a group; workgroup ids are remapped so each XCD
//    (ids i, i+8, ...) runs a contiguous run of that order.  A round of an
//    XCD's 32 CUs then shares 4 activation slabs and 8 weight columns in
//    its L2.
//  * Decomposition: at most 64 tokens run as 64-token tiles (a quarter of
//    the MFMA work per weight stream), split along K while they fill at
//    most half the CUs.  Otherwise complete rounds of full tiles; a last round at most
//    half full runs as twice as many 128-token half tiles (no partial
//    sums).  Problems of at most half a round split full tiles along K
//    into up to 8 pieces whose partial tiles go to the stream's workspace
//    and are summed in piece order by a second kernel (short K: half
//    tiles; without a workspace: pieces added into zeroed y with float
//    atomics).
#include "swamp_common.hpp"
#include "swamp_items.hpp"

#include <algorithm>
#include <mutex>

namespace {

using swamp::q4k_scales;
using swamp::shr16;

typedef __bf16 bf16x8_t __attribute__((ext_vector_type(8)));
typedef __bf16 bf16x2_t __attribute__((ext_vector_type(2)));
typedef float f32x16_t __attribute__((ext_vector_type(16)));
typedef uint32_t u32x4v_t __attribute__((ext_vector_type(4)));

constexpr int kBM = 256, kBN = 256, kBK = 64;  // full tile and K step
constexpr int kThreads = 512, kWaves = 8;
constexpr int kStages = 5;                     // activation stages
constexpr int kGroup = 4;                      // token tiles per order group

// Per-shape constants: kTok token tiles of 32 per wave (8: full tile,
// 4: half tile).
template <int DT, int kTok>
struct Cfg {
  static constexpr int kRows = 32 * kTok;              // tokens of the tile
  static constexpr int kXStage = kRows * kBK * 2;      // bytes of one stage
  static constexpr int kSmem = kStages * kXStage;      // 160 KB / 80 KB
  static constexpr int kDma = kRows * 128 / 1024 / kWaves;  // 1 KB DMAs per wave and step
  static constexpr int kWLoads = DT == SWAMP_Q8_0 ? 3 : 2;  // weight loads per item
  static constexpr int kVmem = kDma + kWLoads;         // vector-memory ops per step
};

__device__ __forceinline__ int swz(int row, int chunk) {
  return row * 128 + ((chunk ^ ((row >> 1) & 7)) << 4);
}

__device__ __forceinline__ uint32_t pack_bf16(float a, float b) {
  bf16x2_t v;
  v[0] = (__bf16)a;
  v[1] = (__bf16)b;
  return __builtin_bit_cast(uint32_t, v);
}

// One 16-byte-per-lane DMA into LDS (lane L writes lds + 16 L).  Not a
// template: the host compilation pass rejects the LDS address-space cast
// inside a template instantiation.
__device__ __forceinline__ void dma16(__amdgpu_buffer_rsrc_t r, uint8_t *lds, uint32_t voff,
                                      uint32_t soff) {
  __builtin_amdgcn_raw_ptr_buffer_load_lds(r, (__attribute__((address_space(3))) void *)lds, 16,
                                           voff, soff, 0, 0);
}

typedef float f32x2_t __attribute__((ext_vector_type(2)));

// Two nibble codes c0, c1 (bytes 2 sel, 2 sel + 1 of a word whose bytes are
// all below 16) as fp32: a byte below 16 read as OCP E4M3 is the integer
// times 2^-9 (the denormals run on linearly into the first binade), and the
// convert's scale operand, of which only the power of two counts, supplies
// 2^9 -- exact, two codes per instruction.
template <bool kSel>
__device__ __forceinline__ f32x2_t nib_pair(uint32_t w) {
  return __builtin_amdgcn_cvt_scalef32_pk_f32_fp8(w, 512.0f, kSel);
}

// Eight weights from the four bytes of w: byte p holds elements 2p (low
// nibble) and 2p + 1 (high nibble); value q * s + o, one fp32 rounding,
// then bf16.
__device__ __forceinline__ u32x4v_t deq_pairs(uint32_t w, float s, float o) {
  const uint32_t lo = w & 0x0F0F0F0Fu, hi = (w >> 4) & 0x0F0F0F0Fu;
  const f32x2_t l0 = nib_pair<false>(lo), l1 = nib_pair<true>(lo);
  const f32x2_t h0 = nib_pair<false>(hi), h1 = nib_pair<true>(hi);
  u32x4v_t out;
  out[0] = pack_bf16(__builtin_fmaf(l0[0], s, o), __builtin_fmaf(h0[0], s, o));
  out[1] = pack_bf16(__builtin_fmaf(l0[1], s, o), __builtin_fmaf(h0[1], s, o));
  out[2] = pack_bf16(__builtin_fmaf(l1[0], s, o), __builtin_fmaf(h1[0], s, o));
  out[3] = pack_bf16(__builtin_fmaf(l1[1], s, o), __builtin_fmaf(h1[1], s, o));
  return out;
}

// Eight consecutive weights from the bytes of two words w0, w1 (byte i of
// w0 is weight i), each byte u the weight's code; value u * s + o.
__device__ __forceinline__ u32x4v_t deq_bytes(uint32_t w0, uint32_t w1, float s, float o) {
  asm("" : "+v"(w0), "+v"(w1));
  u32x4v_t out;
#pragma unroll
  for (int p = 0; p < 2; p++) {
    out[p] = pack_bf16(__builtin_fmaf(float((w0 >> (16 * p)) & 0xFFu), s, o),
                       __builtin_fmaf(float((w0 >> (16 * p + 8)) & 0xFFu), s, o));
    out[2 + p] = pack_bf16(__builtin_fmaf(float((w1 >> (16 * p)) & 0xFFu), s, o),
                           __builtin_fmaf(float((w1 >> (16 * p + 8)) & 0xFFu), s, o));
  }
  return out;
}

// The same for bytes that are all below 16 (nibble codes), through nib_pair.
__device__ __forceinline__ u32x4v_t deq_nibbles(uint32_t w0, uint32_t w1, float s, float o) {
  const f32x2_t a = nib_pair<false>(w0), b = nib_pair<true>(w0);
  const f32x2_t c = nib_pair<false>(w1), d = nib_pair<true>(w1);
  u32x4v_t out;
  out[0] = pack_bf16(__builtin_fmaf(a[0], s, o), __builtin_fmaf(a[1], s, o));
  out[1] = pack_bf16(__builtin_fmaf(b[0], s, o), __builtin_fmaf(b[1], s, o));
  out[2] = pack_bf16(__builtin_fmaf(c[0], s, o), __builtin_fmaf(c[1], s, o));
  out[3] = pack_bf16(__builtin_fmaf(d[0], s, o), __builtin_fmaf(d[1], s, o));
  return out;
}

// Item weights (and activation k) that lane half h = lane / 32 supplies to
// the MFMA of substep s, as the 8-weight chunk 0..7 of the K step.  Any
// order works if A and B agree; this one makes a lane need 36 B or less of
// the item.  Q4_0 / Q8_0: chunk s + 4h, weights 32h .. 32h + 31 -- block h
// of the item.  Q4_K: chunk 4(s/2) + 2h + s%2, i.e. low nibbles (sub-block
// A) of quarter bytes 16h + 8(s%2) .. +7 for s < 2 and the high nibbles
// (sub-block B) of the same bytes for s >= 2 -- 16 bytes of the quarter,
// with the sub-block and its scale constants of the substep.
template <int DT>
__host__ __device__ constexpr int k_chunk(int s, int h) {
  return DT == SWAMP_Q4_K ? 4 * (s >> 1) + 2 * h + (s & 1) : s + 4 * h;
}

// A lane's share of one weight item (64 weights of its row for one K
// step): block h of a Q4_0 / Q8_0 item, loaded with the dword around its
// start (block 1 starts 2 bytes into a dword); header and bytes 16h ..
// 16h + 15 of a Q4_K quarter.
template <int DT>
struct WItem;
template <>
struct WItem<SWAMP_Q4_0> {
  uint32_t d[5];  // d[0]: item bytes 16..19; d[1..4]: bytes 0..15 (h = 0) or 20..35 (h = 1)
};
template <>
struct WItem<SWAMP_Q8_0> {
  uint32_t d[9];  // d[0]: item bytes 32..35; d[1..8]: bytes 0..31 (h = 0) or 36..67 (h = 1)
};
template <>
struct WItem<SWAMP_Q4_K> {
  uint32_t h[4];  // d, dmin, 12 scale bytes
  uint32_t q[4];  // nibble bytes 16h .. 16h + 15 of the quarter
};

// Per-lane byte offset (within the item) of the first 16-byte load.
template <int DT>
__host__ __device__ constexpr uint32_t half_offset(bool h) {
  return !h ? 0u : DT == SWAMP_Q4_0 ? 20u : DT == SWAMP_Q8_0 ? 36u : 16u;
}

// B fragment of substep S for the lane's row: chunk k_chunk(S, h) of the
// item.  S is a template argument so every index into the
// item is a constant and the item stays in registers; the lane's half
// only selects between two registers.  Q = item % 4 (the Q4_K quarter,
// whose sub-block scales the item uses) is one too, so the scale
// unpacking has no branch.
template <int DT, int S, int Q>
__device__ __forceinline__ u32x4v_t b_frag(const WItem<DT> &r, bool h) {
  // block 0's quants start 2 bytes into their dwords, block 1's on a dword:
  // one byte-align per dword with a per-lane shift (2 or 0) serves both
  const uint32_t sh = h ? 0u : 2u;
  if constexpr (DT == SWAMP_Q4_0) {
    // block h: d, then 16 nibble bytes (byte b holds elements 2b and 2b + 1,
    // q4_0.rs:30-35); chunk S is quant bytes 4S .. 4S + 3.  Block 0's quants
    // start at byte 2 of d[1] (its bytes 16, 17 sit in d[0]); block 1's d is
    // the high half of d[0] and its quants are d[1..4].
    const uint32_t hi0 = S < 3 ? r.d[S + 2] : r.d[0];
    const uint32_t w = __builtin_amdgcn_alignbyte(hi0, r.d[S + 1], sh);
    const float d = swamp::f16_bits_to_f32(h ? r.d[0] >> 16 : r.d[1] & 0xFFFFu);
    return deq_pairs(w, d, -8.0f * d);
  } else if constexpr (DT == SWAMP_Q8_0) {
    // block h: d, then 32 int8; chunk S is quant bytes 8S .. 8S + 7.  Block
    // 0's quants start at byte 2 of d[1] (bytes 32, 33 sit in d[0]); block
    // 1's d is the high half of d[0] and its quants are d[1..8].  Bytes
    // carry q + 128 after the xor: (q + 128) d - 128 d = q d exactly.
    constexpr int j = 2 * S;
    const uint32_t e2 = j + 2 < 9 ? r.d[j + 2] : r.d[0];
    const uint32_t e3 = j + 3 < 9 ? r.d[j + 3] : r.d[0];
    const uint32_t w0 = __builtin_amdgcn_alignbyte(e2, r.d[j + 1], sh);
    const uint32_t w1 = __builtin_amdgcn_alignbyte(e3, e2, sh);
    const float d = swamp::f16_bits_to_f32(h ? r.d[0] >> 16 : r.d[1] & 0xFFFFu);
    return deq_bytes(w0 ^ 0x80808080u, w1 ^ 0x80808080u, d, -128.0f * d);
  } else {
    (void)sh;
    // Q4_K quarter: sub-block A = low nibbles of the 32 bytes (S < 2),
    // sub-block B = high nibbles (S >= 2) (layout A, q4_k.rs:290-319), of
    // the lane's bytes 8(S%2) .. +7.  The sub-block, its mask and scale are
    // constants of the substep.
    const float dd = swamp::f16_bits_to_f32(r.h[0] & 0xFFFFu);
    const float dmin = swamp::f16_bits_to_f32(r.h[0] >> 16);
    uint32_t sc0, m0, sc1, m1;
    q4k_scales(r.h, 2 * Q, sc0, m0, sc1, m1);  // Q: the item's quarter, a constant
    constexpr bool hb = S >= 2;
    const float sc = dd * float(hb ? sc1 : sc0), o = -(dmin * float(hb ? m1 : m0));
    (void)h;
    constexpr int t = 2 * (S & 1);
    const uint32_t w0 = r.q[t], w1 = r.q[t + 1];
    // low nibbles: bytes of w & 0x0F0F0F0F; high: of (w >> 4) & 0x0F0F0F0F
    const uint32_t a0 = hb ? w0 >> 4 : w0, a1 = hb ? w1 >> 4 : w1;
    return deq_nibbles(a0 & 0x0F0F0F0Fu, a1 & 0x0F0F0F0Fu, sc, o);
  }
}

// A lane's share of one weight item through a buffer resource: the lane's
// row in the VGPR offset vrow (vhalf = vrow + half_offset), the item's byte
// offset within a row in the (uniform) SGPR offset.  Reads past the
// descriptor's range return zeros.
template <int DT>
__device__ __forceinline__ void load_item(WItem<DT> &r, __amdgpu_buffer_rsrc_t rs, uint32_t vrow,
                                          uint32_t vhalf, int item) {
  if constexpr (DT == SWAMP_Q4_0) {
    const uint32_t so = uint32_t(item) * 36u;
    r.d[0] = __builtin_amdgcn_raw_buffer_load_b32(rs, vrow + 16, so, 0);
    const u32x4v_t a = __builtin_amdgcn_raw_buffer_load_b128(rs, vhalf, so, 0);
#pragma unroll
    for (int i = 0; i < 4; i++) r.d[1 + i] = a[i];
  } else if constexpr (DT == SWAMP_Q8_0) {
    const uint32_t so = uint32_t(item) * 68u;
    r.d[0] = __builtin_amdgcn_raw_buffer_load_b32(rs, vrow + 32, so, 0);
#pragma unroll
    for (int j = 0; j < 2; j++) {
      const u32x4v_t a = __builtin_amdgcn_raw_buffer_load_b128(rs, vhalf + 16 * j, so, 0);
#pragma unroll
      for (int i = 0; i < 4; i++) r.d[1 + 4 * j + i] = a[i];
    }
  } else {
    const uint32_t hb = uint32_t(item >> 2) * 144u;
    const uint32_t so = hb + 16u + 32u * uint32_t(item & 3);
    const u32x4v_t hd = __builtin_amdgcn_raw_buffer_load_b128(rs, vrow, hb, 0);
    const u32x4v_t a = __builtin_amdgcn_raw_buffer_load_b128(rs, vhalf, so, 0);
#pragma unroll
    for (int i = 0; i < 4; i++) { r.h[i] = hd[i]; r.q[i] = a[i]; }
  }
}

// Per-lane load geometry.  DMA instruction i of wave w fills stage bytes
// [1024 (kDma w + i), +1024) = tile rows 8(kDma w + i) .. +7: lane L writes
// row 8(kDma w + i) + L/8, physical chunk L%8, and fetches the logical chunk
// the swizzle puts there, (L%8) ^ ((row / 2) % 8) = (L%8) ^ ((4p + L/16) % 8)
// with p = (kDma w + i) % 2: xv[p].  The weight item of the lane is row 32w + L%32.
struct Geo {
  __amdgpu_buffer_rsrc_t xr, wr;
  uint32_t xv[2];  // per-lane DMA offsets for even / odd instructions
  uint32_t xs;     // m0 * K * 2 (scalar)
  uint32_t xinst;  // 8 * K * 2: scalar step between instructions
  uint32_t wv;     // per-lane weight row offset
  uint32_t wvh;    // wv + half_offset (the lane's first 16-byte weight load)
  int wave;
};

template <int kDma>
__device__ __forceinline__ void xdma(uint8_t *stage, const Geo &g, int kt) {
#pragma unroll
  for (int i = 0; i < kDma; i++)  // the swizzle of rows 8(kDma w + i) .. +7 has parity kDma w + i
    dma16(g.xr, stage + 1024 * (kDma * g.wave + i), ((kDma * g.wave + i) & 1) ? g.xv[1] : g.xv[0],
          g.xs + uint32_t(i) * g.xinst + uint32_t(kt) * 128u);
}

// A fragment of token tile i, substep ks: the 16-byte chunk
// k_chunk(ks, l/32) of the token's row, the k order of b_frag.
template <int DT>
__device__ __forceinline__ bf16x8_t a_frag(const uint8_t *stg, int ks, int i, int lane) {
  return *reinterpret_cast<const bf16x8_t *>(
      stg + swz(32 * i + (lane & 31), k_chunk<DT>(ks, lane >> 5)));
}

// Substep KS of a K step (k = 16 KS .. 16 KS + 15): the MFMAs of every
// token tile with B fragment bc[KS]; each A fragment is re-read right after
// the MFMA that consumed it (for substep KS + 1, or the next step's
// substep 0 from `nxt`); step kt+1's B fragment KS is dequantized from
// `nw`.  Substep 0 also issues the step's loads: step kt+4's activations
// into `dma`, step kt+2's weight item into `fetch`.
template <int DT, int kTok, int KS, int Q>
__device__ __forceinline__ void substep(f32x16_t (&acc)[kTok], bf16x8_t (&a)[kTok],
                                        const uint8_t *cur, const uint8_t *nxt, uint8_t *dma,
                                        const u32x4v_t (&bc)[4], u32x4v_t (&bn)[4],
                                        const WItem<DT> &nw, WItem<DT> &fetch, const Geo &g, int kt,
                                        int kt1, int lane) {
  using C = Cfg<DT, kTok>;
  if constexpr (KS == 0) {
    xdma<C::kDma>(dma, g, min(kt + kStages - 1, kt1 - 1));  // past the end: re-read
    load_item<DT>(fetch, g.wr, g.wv, g.wvh, min(kt + 2, kt1 - 1));
  }
#pragma unroll
  for (int i = 0; i < kTok; i++) {
    acc[i] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(a[i], __builtin_bit_cast(bf16x8_t, bc[KS]),
                                                     acc[i], 0, 0, 0);
    a[i] = KS < 3 ? a_frag<DT>(cur, KS + 1, i, lane) : a_frag<DT>(nxt, 0, i, lane);
  }
  bn[KS] = b_frag<DT, KS, Q>(nw, lane >= 32);
#pragma unroll
  for (int m = 0; m < kTok; m++) {
    __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);          // 1 MFMA
    __builtin_amdgcn_sched_group_barrier(0x100, 1, 0);          // 1 DS read
    __builtin_amdgcn_sched_group_barrier(0x002, 32 / kTok, 0);  // VALU
    if constexpr (KS == 0)
      __builtin_amdgcn_sched_group_barrier(0x010, (C::kVmem + kTok - 1) / kTok, 0);  // VMEM
  }
  __builtin_amdgcn_sched_barrier(0);
}

// One K step.  a[] holds substep 0's A fragments on entry (read before the
// previous barrier) and the next step's on return.  Q = (kt + 1) % 4, the
// quarter of the item dequantized in this step (used by Q4_K; past the last
// step the re-read item's B fragments are never used).
template <int DT, int kTok, int Q>
__device__ __forceinline__ void kstep(f32x16_t (&acc)[kTok], bf16x8_t (&a)[kTok],
                                      const uint8_t *cur, const uint8_t *nxt, uint8_t *dma,
                                      const u32x4v_t (&bc)[4], u32x4v_t (&bn)[4],
                                      const WItem<DT> &nw, WItem<DT> &fetch, const Geo &g, int kt,
                                      int kt1, int lane) {
  using C = Cfg<DT, kTok>;
  substep<DT, kTok, 0, Q>(acc, a, cur, nxt, dma, bc, bn, nw, fetch, g, kt, kt1, lane);
  substep<DT, kTok, 1, Q>(acc, a, cur, nxt, dma, bc, bn, nw, fetch, g, kt, kt1, lane);
  substep<DT, kTok, 2, Q>(acc, a, cur, nxt, dma, bc, bn, nw, fetch, g, kt, kt1, lane);
  substep<DT, kTok, 3, Q>(acc, a, cur, nxt, dma, bc, bn, nw, fetch, g, kt, kt1, lane);
  // The loads issued before the previous step -- among them step kt+2's
  // activations -- are complete; the last kTok fragment reads (of `nxt`)
  // stay in flight across the barrier.
  asm volatile("s_waitcnt vmcnt(%0)\n\ts_waitcnt lgkmcnt(%1)\n\ts_barrier" ::"n"(2 * C::kVmem),
               "n"(kTok)
               : "memory");
}

// Tile t of the grouped order -> (token tile, weight tile).
__host__ __device__ inline void tile_coords(int t, int tiles_m, int tiles_n, int &mt, int &nt) {
  const int grp = t / (kGroup * tiles_n), first = grp * kGroup;
  const int gs = min(tiles_m - first, kGroup), r = t % (kGroup * tiles_n);
  mt = first + r % gs;
  nt = r / gs;
}

// Work of one launch: tiles [first, first + count) of the grouped order,
// each as `parts` token parts (1: full tile, 2: halves) x `splits` K pieces.
struct Work {
  int tiles_m, tiles_n, first, parts, splits, kt_per_split;
  float *part;  // splits > 1: partial sums [piece][M][N] (else added into y atomically)
};

template <int DT, int kTok>
__global__ void __launch_bounds__(kThreads, 1)
    gemm_bf16_kernel(const uint8_t *w, const uint16_t *x, float *__restrict__ y, int M, int N,
                     int K, size_t row_bytes, Work wk) {
  // w and x carry no __restrict__: the hand-counted waits assume every load
  // is issued where the code places it, and with the weights known to be
  // read-only the compiler may move their loads across the barriers (whose
  // memory clobber then no longer orders them).
  using C = Cfg<DT, kTok>;
  extern __shared__ __attribute__((aligned(16))) uint8_t smem[];
  const int tid = threadIdx.x;
  const int wave = tid >> 6, lane = tid & 63;

  // XCD-aware unit order: hardware ids i, i+8, ... run on one XCD; each
  // XCD takes a contiguous run of units.
  const int n_units = int(gridDim.x);
  int u = blockIdx.x;
  if (n_units % 8 == 0) u = (u % 8) * (n_units / 8) + u / 8;
  const int per_tile = wk.parts * wk.splits;
  const int t = wk.first + u / per_tile, part = (u % per_tile) / wk.splits;
  const int piece = u % wk.splits;
  int mt, nt;
  tile_coords(t, wk.tiles_m, wk.tiles_n, mt, nt);
  const int m0 = mt * kBM + part * C::kRows, n0 = nt * kBN;
  if (m0 >= M) return;  // second half of a short last token tile (uniform)
  const int KT = K / kBK;
  const int kt0 = piece * wk.kt_per_split, kt1 = min(KT, kt0 + wk.kt_per_split);
  const bool atomic = wk.splits > 1;

  Geo g;
  g.wave = __builtin_amdgcn_readfirstlane(wave);
  g.xr = swamp::make_rsrc(x, uint32_t(size_t(M) * K * 2));
  {
    const int rl = 8 * C::kDma * wave + (lane >> 3);
#pragma unroll
    for (int par = 0; par < 2; par++) {
      const int c = (lane & 7) ^ ((4 * par + (lane >> 4)) & 7);
      g.xv[par] = uint32_t((rl * K + 8 * c) * 2);
    }
  }
  g.xs = uint32_t(size_t(m0) * K * 2);
  g.xinst = uint32_t(8 * K * 2);
  const int nrows = min(kBN, N - n0);
  g.wr = swamp::make_rsrc(w + size_t(n0) * row_bytes, uint32_t(size_t(nrows) * row_bytes));
  g.wv = uint32_t(size_t(32 * wave + (lane & 31)) * row_bytes);
  g.wvh = g.wv + half_offset<DT>(lane >= 32);

  f32x16_t acc[kTok];
#pragma unroll
  for (int i = 0; i < kTok; i++)
#pragma unroll
    for (int e = 0; e < 16; e++) acc[i][e] = 0.f;

  auto st = [&](int s) { return smem + C::kXStage * ((s - kt0) % kStages); };
  WItem<DT> ra, rb;
  u32x4v_t ba[4], bb[4];
  bf16x8_t a[kTok];
  const bool h = lane >= 32;
  // Prologue in the steady-state order: x(kt0), x(kt0+1), x(kt0+2), w(kt0),
  // x(kt0+3), w(kt0+1) (steps kt0-4 .. kt0-1 of the loop's pattern).
  xdma<C::kDma>(st(kt0), g, kt0);
  __builtin_amdgcn_sched_barrier(0);
  xdma<C::kDma>(st(kt0 + 1), g, min(kt0 + 1, kt1 - 1));
  __builtin_amdgcn_sched_barrier(0);
  xdma<C::kDma>(st(kt0 + 2), g, min(kt0 + 2, kt1 - 1));
  __builtin_amdgcn_sched_barrier(0);
  load_item<DT>(ra, g.wr, g.wv, g.wvh, kt0);
  __builtin_amdgcn_sched_barrier(0);
  xdma<C::kDma>(st(kt0 + 3), g, min(kt0 + 3, kt1 - 1));
  __builtin_amdgcn_sched_barrier(0);
  load_item<DT>(rb, g.wr, g.wv, g.wvh, min(kt0 + 1, kt1 - 1));
  __builtin_amdgcn_sched_barrier(0);
  ba[0] = b_frag<DT, 0, 0>(ra, h);  // kt0 % 4 == 0 for Q4_K
  ba[1] = b_frag<DT, 1, 0>(ra, h);  // kt0 % 4 == 0 for Q4_K
  ba[2] = b_frag<DT, 2, 0>(ra, h);  // kt0 % 4 == 0 for Q4_K
  ba[3] = b_frag<DT, 3, 0>(ra, h);  // kt0 % 4 == 0 for Q4_K
  // x(kt0) and x(kt0+1) complete: 2 kVmem loads were issued after x(kt0+1)
  asm volatile("s_waitcnt vmcnt(%0)\n\ts_barrier" ::"n"(2 * C::kVmem) : "memory");
#pragma unroll
  for (int i = 0; i < kTok; i++) a[i] = a_frag<DT>(st(kt0), 0, i, lane);

  constexpr int D = kStages - 1;
  int kt = kt0;
  if constexpr (DT == SWAMP_Q4_K) {
    // Four steps per trip: the item quarters are constants (kt0 and kt1 are
    // multiples of 4 for Q4_K, whose rows are whole 256-weight blocks).
    for (; kt < kt1; kt += 4) {
      kstep<DT, kTok, 1>(acc, a, st(kt), st(kt + 1), st(kt + D), ba, bb, rb, ra, g, kt, kt1, lane);
      kstep<DT, kTok, 2>(acc, a, st(kt + 1), st(kt + 2), st(kt + 1 + D), bb, ba, ra, rb, g,
                         kt + 1, kt1, lane);
      kstep<DT, kTok, 3>(acc, a, st(kt + 2), st(kt + 3), st(kt + 2 + D), ba, bb, rb, ra, g,
                         kt + 2, kt1, lane);
      kstep<DT, kTok, 0>(acc, a, st(kt + 3), st(kt + 4), st(kt + 3 + D), bb, ba, ra, rb, g,
                         kt + 3, kt1, lane);
    }
  } else {
    // Two steps per trip so the register buffers keep static roles.
    for (; kt + 1 < kt1; kt += 2) {
      kstep<DT, kTok, 0>(acc, a, st(kt), st(kt + 1), st(kt + D), ba, bb, rb, ra, g, kt, kt1, lane);
      kstep<DT, kTok, 0>(acc, a, st(kt + 1), st(kt + 2), st(kt + 1 + D), bb, ba, ra, rb, g,
                         kt + 1, kt1, lane);
    }
    if (kt < kt1)
      kstep<DT, kTok, 0>(acc, a, st(kt), st(kt + 1), st(kt + D), ba, bb, rb, ra, g, kt, kt1, lane);
  }

  // C layout of a 32x32 tile: lane holds column (lane & 31), rows
  // 8*(e/4) + 4*(lane/32) + (e%4) for e = 0..15.
  const int fr = lane & 31, fc = lane >> 5;
  const int n = n0 + 32 * wave + fr;
  if (n < N) {
#pragma unroll
    for (int i = 0; i < kTok; i++)
#pragma unroll
      for (int e = 0; e < 16; e++) {
        const int m = m0 + 32 * i + 8 * (e >> 2) + 4 * fc + (e & 3);
        if (m < M) {
          float *dst = y + size_t(m) * N + n;
          if (!atomic) *dst = acc[i][e];
          else if (wk.part) wk.part[(size_t(piece) * M + m) * N + n] = acc[i][e];
          else unsafeAtomicAdd(dst, acc[i][e]);
        }
      }
  }
}

// Zero the y blocks of tiles [first, first + gridDim.x / 64) of the grouped
// order: block b clears 4 rows of tile first + b/64, each thread 4 floats.
__global__ void zero_tiles_kernel(float *__restrict__ y, int M, int N, int tiles_m, int tiles_n,
                                  int first) {
  const int t = first + int(blockIdx.x) / 64;
  int mt, nt;
  tile_coords(t, tiles_m, tiles_n, mt, nt);
  const int m = mt * kBM + 4 * (int(blockIdx.x) % 64) + int(threadIdx.x) / 64;
  const int n = nt * kBN + 4 * (int(threadIdx.x) % 64);
  if (m >= M) return;
  float *row = y + size_t(m) * N;
#pragma unroll
  for (int i = 0; i < 4; i++)
    if (n + i < N) row[n + i] = 0.f;
}

// y = sum of the K pieces' partials, in piece order (deterministic); all
// (at most 8) loads are issued before the adds.
__global__ void split_reduce_kernel(const float *__restrict__ part, float *__restrict__ y,
                                    int splits, size_t n) {
  const size_t i = size_t(blockIdx.x) * blockDim.x + threadIdx.x;
  if (i >= n) return;
  float v[8];
#pragma unroll
  for (int p = 0; p < 8; p++) v[p] = p < splits ? part[size_t(p) * n + i] : 0.f;
  float s = v[0];
#pragma unroll
  for (int p = 1; p < 8; p++) s += v[p];  // missing pieces add 0
  y[i] = s;
}

// The same sums, 4 consecutive elements per thread (16-byte loads and
// stores: part, y and n / 4 16-byte aligned); each element takes the
// scalar kernel's additions in the same order, so y is bit-identical.
__global__ void split_reduce4_kernel(const float4 *__restrict__ part, float4 *__restrict__ y,
                                     int splits, size_t n4) {
  const size_t i = size_t(blockIdx.x) * blockDim.x + threadIdx.x;
  if (i >= n4) return;
  float4 v[8];
#pragma unroll
  for (int p = 0; p < 8; p++)
    v[p] = p < splits ? part[size_t(p) * n4 + i] : make_float4(0.f, 0.f, 0.f, 0.f);
  float4 s = v[0];
#pragma unroll
  for (int p = 1; p < 8; p++) {
    s.x += v[p].x;
    s.y += v[p].y;
    s.z += v[p].z;
    s.w += v[p].w;
  }
  y[i] = s;
}

// ---- Q8_0 activation quantization ------------------------------------------
// The arithmetic of one block, shared by both kernels: amax over the block,
// d = amax / 127, q = round(v / d) clamped to [-127, 127], d stored as fp16
// (the host quantizer's, byte for byte).
__device__ __forceinline__ float q8_scale(float amax) { return amax / 127.0f; }
__device__ __forceinline__ int q8_code(float v, float d) {
  const float id = d != 0.f ? 1.0f / d : 0.f;
  const float q = fminf(127.f, fmaxf(-127.f, roundf(v * id)));
  return int(q);
}

// Any alignment of dst: one element per thread, 32 lanes per block, byte
// stores.  Also quantizes the blocks [first, n_blocks) left over by the
// vector kernel below.
template <bool kBf16>
__global__ void quantize_q8_0_kernel(const void *__restrict__ src, uint8_t *__restrict__ dst,
                                     size_t first, size_t n_blocks) {
  const size_t gid = first * 32 + size_t(blockIdx.x) * blockDim.x + threadIdx.x;
  const size_t blk = gid >> 5;
  const int i = int(gid & 31);
  const bool ok = blk < n_blocks;
  float v = 0.f;
  if (ok) {
    if (kBf16) v = __uint_as_float(uint32_t(static_cast<const uint16_t *>(src)[gid]) << 16);
    else v = static_cast<const float *>(src)[gid];
  }
  float a = fabsf(v);
#pragma unroll
  for (int off = 16; off >= 1; off >>= 1) a = fmaxf(a, __shfl_xor(a, off, 32));
  const float d = q8_scale(a);
  const int q = q8_code(v, d);
  if (ok) {
    uint8_t *b = dst + blk * 34;
    b[2 + i] = uint8_t(int8_t(q));
    if (i == 0) {
      const uint16_t h = __builtin_bit_cast(uint16_t, _Float16(d));
      b[0] = uint8_t(h & 0xFF);
      b[1] = uint8_t(h >> 8);
    }
  }
}

// 4-byte aligned dst: a wave quantizes 8 whole blocks, 4 consecutive
// elements per lane (one 16-byte or 8-byte load), the block's amax over its
// 8 lanes.  The wave's 8 output blocks are 272 contiguous bytes at a 4-byte
// aligned offset (272 = 4 * 68): they are assembled in LDS with 2-byte
// stores (a lane's 4 codes sit at 34 k + 2 + 4 j, 2 mod 4 for even blocks)
// and written out as 68 dwords.  Only whole groups of 8 blocks come here.
template <bool kBf16>
__global__ void __launch_bounds__(256) quantize_q8_0_x8_kernel(const void *__restrict__ src,
                                                               uint8_t *__restrict__ dst,
                                                               size_t n_groups) {
  __shared__ uint32_t stage[4][68];
  const int lane = threadIdx.x & 63, w = threadIdx.x >> 6;
  const size_t grp = size_t(blockIdx.x) * 4 + size_t(w);
  const bool ok = grp < n_groups;  // uniform per wave
  const int k = lane >> 3, j = lane & 7;
  // this workgroup's groups as one buffer range (out-of-range loads read 0)
  const size_t g0 = size_t(blockIdx.x) * 4;
  const uint32_t ebytes = kBf16 ? 2u : 4u;
  const uint32_t range = uint32_t(min(n_groups - g0, size_t(4)) * 256u * ebytes);
  const __amdgpu_buffer_rsrc_t r = swamp::make_rsrc(
      static_cast<const uint8_t *>(src) + g0 * 256u * ebytes, range);
  const uint32_t voff = (uint32_t(w) * 256u + uint32_t(lane) * 4u) * ebytes;
  float v[4];
  if constexpr (kBf16) {
    typedef uint32_t u32x2v_t __attribute__((ext_vector_type(2)));
    const u32x2v_t h = __builtin_amdgcn_raw_buffer_load_b64(r, voff, 0, 0);
    v[0] = __uint_as_float(h[0] << 16);
    v[1] = __uint_as_float(h[0] & 0xFFFF0000u);
    v[2] = __uint_as_float(h[1] << 16);
    v[3] = __uint_as_float(h[1] & 0xFFFF0000u);
  } else {
    const u32x4v_t a = __builtin_amdgcn_raw_buffer_load_b128(r, voff, 0, 0);
#pragma unroll
    for (int i = 0; i < 4; i++) v[i] = __uint_as_float(a[i]);
  }
  float a = fmaxf(fmaxf(fabsf(v[0]), fabsf(v[1])), fmaxf(fabsf(v[2]), fabsf(v[3])));
#pragma unroll
  for (int off = 4; off >= 1; off >>= 1) a = fmaxf(a, __shfl_xor(a, off, 8));
  const float d = q8_scale(a);
  uint32_t packed = 0;
#pragma unroll
  for (int i = 0; i < 4; i++) packed |= (uint32_t(q8_code(v[i], d)) & 0xFFu) << (8 * i);
  typedef uint16_t __attribute__((may_alias)) u16_alias_t;  // 2-byte view of the dword stage
  u16_alias_t *st = reinterpret_cast<u16_alias_t *>(stage[w]);
  const int o = 17 * k + 1 + 2 * j;  // in 2-byte units: byte 34 k + 2 + 4 j
  st[o] = uint16_t(packed & 0xFFFFu);
  st[o + 1] = uint16_t(packed >> 16);
  if (j == 0) st[17 * k] = __builtin_bit_cast(uint16_t, _Float16(d));
  __syncthreads();
  if (ok) {
    uint32_t *out = reinterpret_cast<uint32_t *>(dst + grp * 272u);
    out[lane] = stage[w][lane];
    if (lane < 4) out[64 + lane] = stage[w][64 + lane];
  }
}

template <int DT, int kTok>
int launch_tiles(const uint8_t *w, const uint16_t *x, float *y, int m, int n_rows, int n_cols,
                 const Work &wk, int count, hipStream_t s) {
  using C = Cfg<DT, kTok>;
  static std::once_flag once;
  static hipError_t err = hipSuccess;
  std::call_once(once, [] {
    err = hipFuncSetAttribute(reinterpret_cast<const void *>(&gemm_bf16_kernel<DT, kTok>),
                              hipFuncAttributeMaxDynamicSharedMemorySize, C::kSmem);
  });
  if (err != hipSuccess) return SWAMP_ELAUNCH;
  const unsigned units = unsigned(count * wk.parts * wk.splits);
  gemm_bf16_kernel<DT, kTok><<<units, kThreads, C::kSmem, s>>>(
      w, x, y, m, n_rows, n_cols, swamp::row_bytes(DT, size_t(n_cols)), wk);
  return hipGetLastError() == hipSuccess ? SWAMP_OK : SWAMP_ELAUNCH;
}

// Work decomposition of one bf16 GEMM call (the choice follows measured
// step times of one tile on one CU -- full 2.0 us, half 1.3 us at 8B
// shapes -- and 6 TB/s for the partial sums: written, read, y written).
//  kSmall  at most 64 tokens: 64-token tiles (a quarter of the MFMA work of
//          a full tile for the same weight stream), split along K into up
//          to 8 pieces while they fill at most half the CUs;
//  kSplit  at most half a round of tiles: full tiles split along K into up
//          to 8 pieces, or 128-token halves (split into up to 4 pieces when
//          they fill at most half the CUs);
//  kRounds full tiles in complete rounds, a last round at most half full as
//          128-token halves (no partial sums).
// Split pieces write partial tiles to scratch, summed in piece order by a
// second kernel (deterministic).  Without scratch the pieces add into
// zeroed y with float atomics (and kSplit takes halves).
struct GemmPlan {
  enum Kind { kSmall, kSplit, kRounds } kind;
  bool full;      // kSplit: full tiles (else halves)
  int pieces;     // K pieces (1: none)
  int kps;        // K steps per piece
  int half_pieces, half_kps;  // kSplit fallback without scratch: halves
  size_t part_bytes;          // scratch for the pieces' partial sums
};

template <int DT>
GemmPlan plan_bf16(int m, int n_rows, int n_cols) {
  const int tiles_m = (m + kBM - 1) / kBM, tiles_n = (n_rows + kBN - 1) / kBN;
  const int tiles = tiles_m * tiles_n, KT = n_cols / kBK;
  const int cus = swamp::device_info().num_cus;
  const size_t mn = size_t(m) * size_t(n_rows);
  auto piece_len = [&](int splits) {  // K steps per piece (whole Q4_K blocks)
    int kps = (KT + splits - 1) / splits;
    if (DT == SWAMP_Q4_K) kps = (kps + 3) / 4 * 4;
    return kps;
  };
  GemmPlan p{GemmPlan::kRounds, true, 1, KT, 1, KT, 0};
  if (m <= kBM / 4) {
    p.kind = GemmPlan::kSmall;
    int pieces = 2 * tiles <= cus ? std::max(1, std::min({cus / tiles, 8, KT / 8})) : 1;
    p.kps = piece_len(pieces);
    p.pieces = (KT + p.kps - 1) / p.kps;
  } else if (2 * tiles <= cus) {
    p.kind = GemmPlan::kSplit;
    auto est_us = [&](double step_us, int pieces) {
      double t_us = double(piece_len(pieces)) * step_us;
      if (pieces > 1) t_us += (2.0 * pieces + 1.0) * double(mn) * 4.0 / 6e6;
      return t_us;
    };
    const int fs = std::min({cus / tiles, 8, KT / 8});
    const int hs = 4 * tiles <= cus ? std::max(1, std::min({cus / (2 * tiles), 4, KT / 8})) : 1;
    p.half_kps = piece_len(hs);
    p.half_pieces = (KT + p.half_kps - 1) / p.half_kps;
    p.full = fs >= 2 && est_us(2.0, fs) < est_us(1.3, hs);
    if (p.full) {
      p.kps = piece_len(fs);
      p.pieces = (KT + p.kps - 1) / p.kps;
    } else {
      p.kps = p.half_kps;
      p.pieces = p.half_pieces;
    }
  }
  p.part_bytes = p.pieces > 1 ? size_t(p.pieces) * mn * sizeof(float) : 0;
  return p;
}

template <int DT>
int launch_bf16(const uint8_t *w, const uint16_t *x, float *y, int m, int n_rows, int n_cols,
                swamp::Scratch &sc, hipStream_t s) {
  const int tiles_m = (m + kBM - 1) / kBM, tiles_n = (n_rows + kBN - 1) / kBN;
  const int tiles = tiles_m * tiles_n, KT = n_cols / kBK;
  const int cus = swamp::device_info().num_cus;
  const size_t mn = size_t(m) * size_t(n_rows);
  const GemmPlan p = plan_bf16<DT>(m, n_rows, n_cols);
  float *part = p.part_bytes ? static_cast<float *>(sc.get(p.part_bytes)) : nullptr;
  if (p.kind == GemmPlan::kSmall) {
    if (p.pieces > 1 && !part)
      zero_tiles_kernel<<<unsigned(tiles * 64), 256, 0, s>>>(y, m, n_rows, tiles_m, tiles_n, 0);
    const Work wk{tiles_m, tiles_n, 0, 1, p.pieces, p.kps, part};
    if (int rc = launch_tiles<DT, 2>(w, x, y, m, n_rows, n_cols, wk, tiles, s)) return rc;
    if (p.pieces > 1 && part) return swamp_launch_split_reduce(part, y, p.pieces, mn, s);
    return SWAMP_OK;
  }
  if (p.kind == GemmPlan::kSplit) {
    if (p.full && part) {
      const Work wk{tiles_m, tiles_n, 0, 1, p.pieces, p.kps, part};
      if (int rc = launch_tiles<DT, 8>(w, x, y, m, n_rows, n_cols, wk, tiles, s)) return rc;
      return swamp_launch_split_reduce(part, y, p.pieces, mn, s);
    }
    // halves: their pieces go to scratch when it is there, else add into
    // zeroed y
    const bool use_part = !p.full && part;
    const int pieces = p.full ? p.half_pieces : p.pieces;
    const int kps = p.full ? p.half_kps : p.kps;
    if (pieces > 1 && !use_part)
      zero_tiles_kernel<<<unsigned(tiles * 64), 256, 0, s>>>(y, m, n_rows, tiles_m, tiles_n, 0);
    const Work wk{tiles_m, tiles_n, 0, 2, pieces, kps, use_part ? part : nullptr};
    if (int rc = launch_tiles<DT, 4>(w, x, y, m, n_rows, n_cols, wk, tiles, s)) return rc;
    if (pieces > 1 && use_part) return swamp_launch_split_reduce(part, y, pieces, mn, s);
    return SWAMP_OK;
  }
  // Full tiles in complete rounds; a last round at most half full as
  // 128-token halves (twice the workgroups, no partial sums).
  int n_half = 0;
  if (tiles >= cus) {
    const int rem = tiles % cus;
    if (rem > 0 && 2 * rem <= cus) n_half = rem;
  }
  const int n_full = tiles - n_half;
  {
    const Work wk{tiles_m, tiles_n, 0, 1, 1, KT, nullptr};
    if (int rc = launch_tiles<DT, 8>(w, x, y, m, n_rows, n_cols, wk, n_full, s)) return rc;
  }
  if (n_half > 0) {
    const Work wk{tiles_m, tiles_n, n_full, 2, 1, KT, nullptr};
    if (int rc = launch_tiles<DT, 4>(w, x, y, m, n_rows, n_cols, wk, n_half, s)) return rc;
  }
  return SWAMP_OK;
}

}  // namespace

int swamp_launch_split_reduce(const float *d_part, float *d_y, int pieces, size_t n,
                              hipStream_t s) {
  if (pieces < 1 || pieces > 8) return SWAMP_EINVAL;
  if (n % 4 == 0 && reinterpret_cast<uintptr_t>(d_part) % 16 == 0 &&
      reinterpret_cast<uintptr_t>(d_y) % 16 == 0) {
    const size_t n4 = n / 4;
    split_reduce4_kernel<<<unsigned((n4 + 255) / 256), 256, 0, s>>>(
        reinterpret_cast<const float4 *>(d_part), reinterpret_cast<float4 *>(d_y), pieces, n4);
  } else {
    split_reduce_kernel<<<unsigned((n + 255) / 256), 256, 0, s>>>(d_part, d_y, pieces, n);
  }
  return hipGetLastError() == hipSuccess ? SWAMP_OK : SWAMP_ELAUNCH;
}

size_t swamp_gemm_scratch_bytes(uint32_t dtype, uint32_t x_type, int m, int n_rows, int n_cols,
                                size_t limit) {
  if (m <= 0 || n_rows <= 0 || n_cols <= 0) return 0;
  if (x_type == SWAMP_Q8_0) return swamp_gemm_i8_scratch_bytes(dtype, m, n_rows, n_cols);
  if (x_type != SWAMP_BF16 || n_cols % kBK != 0) return 0;
  if (swamp_gemm_dq_route(dtype, m, n_rows, n_cols)) {
    const size_t dq = swamp_gemm_dq_scratch_bytes(m, n_rows, n_cols);
    if (dq <= limit || dtype == SWAMP_Q6_K) return dq;
  }
  switch (dtype) {
    case SWAMP_Q4_0: return plan_bf16<SWAMP_Q4_0>(m, n_rows, n_cols).part_bytes;
    case SWAMP_Q8_0: return plan_bf16<SWAMP_Q8_0>(m, n_rows, n_cols).part_bytes;
    case SWAMP_Q4_K: return plan_bf16<SWAMP_Q4_K>(m, n_rows, n_cols).part_bytes;
    default: return 0;
  }
}

int swamp_launch_gemm(uint32_t dtype, const void *d_w, const void *d_x, uint32_t x_type,
                      float *d_y, int m, int n_rows, int n_cols, swamp::Scratch &sc,
                      hipStream_t s) {
  if (m == 0 || n_rows == 0) return SWAMP_OK;
  if (x_type == SWAMP_Q8_0)
    return swamp_launch_gemm_i8(dtype, d_w, d_x, d_y, m, n_rows, n_cols, sc, s);
  if (x_type != SWAMP_BF16) return SWAMP_EDTYPE;
  if (n_cols % kBK != 0) return SWAMP_ESHAPE;
  // activation offsets are 32-bit (buffer descriptors)
  if (size_t(m) * size_t(n_cols) * 2 > size_t(UINT32_MAX)) return SWAMP_ESHAPE;
  // long prompts: dequantize once to bf16 and run a plain bf16 GEMM, when
  // the scratch for it is there (else the fused kernel below)
  if (swamp_gemm_dq_route(dtype, m, n_rows, n_cols) &&
      sc.cap - sc.used >= swamp_gemm_dq_scratch_bytes(m, n_rows, n_cols)) {
    const size_t used = sc.used;
    const int rc = swamp_launch_gemm_dq(dtype, d_w, d_x, d_y, m, n_rows, n_cols, sc, s);
    if (rc != kDqUnavailable) return rc;
    sc.used = used;
  }
  if (dtype == SWAMP_Q6_K) return SWAMP_EWORKSPACE;  // the route above is its only one
  const uint8_t *w = static_cast<const uint8_t *>(d_w);
  const uint16_t *x = static_cast<const uint16_t *>(d_x);
  switch (dtype) {
    case SWAMP_Q4_0: return launch_bf16<SWAMP_Q4_0>(w, x, d_y, m, n_rows, n_cols, sc, s);
    case SWAMP_Q8_0: return launch_bf16<SWAMP_Q8_0>(w, x, d_y, m, n_rows, n_cols, sc, s);
    case SWAMP_Q4_K: return launch_bf16<SWAMP_Q4_K>(w, x, d_y, m, n_rows, n_cols, sc, s);
    default: return SWAMP_EDTYPE;
  }
}

int swamp_launch_quantize_q8_0(const void *d_x, uint32_t x_type, void *d_q, size_t n,
                               hipStream_t s) {
  const size_t nb = n / 32;
  if (nb == 0) return SWAMP_OK;
  if (x_type != SWAMP_BF16 && x_type != SWAMP_F32) return SWAMP_EDTYPE;
  const bool bf = x_type == SWAMP_BF16;
  uint8_t *q = static_cast<uint8_t *>(d_q);
  // whole groups of 8 blocks by the vector kernel when dst is 4-byte
  // aligned; the rest (and any block of an unaligned dst) one element per thread
  const size_t groups = reinterpret_cast<uintptr_t>(d_q) % 4 == 0 ? nb / 8 : 0;
  if (groups > 0) {
    const unsigned grid = unsigned((groups + 3) / 4);
    if (bf) quantize_q8_0_x8_kernel<true><<<grid, 256, 0, s>>>(d_x, q, groups);
    else quantize_q8_0_x8_kernel<false><<<grid, 256, 0, s>>>(d_x, q, groups);
  }
  const size_t first = groups * 8;
  if (first < nb) {
    const unsigned grid = unsigned(((nb - first) * 32 + 255) / 256);
    if (bf) quantize_q8_0_kernel<true><<<grid, 256, 0, s>>>(d_x, q, first, nb);
    else quantize_q8_0_kernel<false><<<grid, 256, 0, s>>>(d_x, q, first, nb);
  }
  return hipGetLastError() == hipSuccess ? SWAMP_OK : SWAMP_ELAUNCH;
}
