// gemv_batched.hip -- small-batch (2..64 tokens per pass; Q6_K 2..32)
// quantized GEMV on the matrix cores, for speculative verify and
// continuous batching.  Q4_0, Q8_0, Q4_K and Q6_K weights.
//
// Replaces forward_linear_batch (swamp-engine/src/linear.rs:176-239) and
// fused_gemv_q4k_batched (swamp-kernels/src/fused_gemv_q4k.rs:527-554,
// scalar body :650-698).
//
// Still HBM-bound (at 16 tokens a Q4 weight byte feeds ~57 FLOP, at 64
// ~230, the chip's balance is ~300), so the weights must stream exactly once
// per pass, with enough bytes in flight per CU to cover HBM latency.
//  * V_MFMA_F32_16X16X32_F16 with A = activations (16 tokens x 32 k) and
//    B = weights (32 k x 16 rows); C = 16 tokens x 16 rows, 4 VGPRs.  Passes
//    of 17..64 tokens run 2 or 4 token groups: every dequantized B fragment
//    feeds one MFMA per group, each group with its own accumulators.
//  * One workgroup of 16 waves per CU.  Its waves form Wt tile lanes x Wk
//    K slices (Wt * Wk = 16): Wk = 1 for matrices with many tiles (each
//    wave streams whole rows), up to 16 for the small ones, so that every
//    CU has weight bytes in flight.  Lane (r = l%16, g = l/16) of a wave
//    reads items g, g+4, g+8, ... (64 weights each) of row r in its slice.
//  * Activations are staged in LDS, rounded to fp16 and stored in MFMA
//    fragment order: one ds_read_b128 per lane and step.  The k order inside
//    each MFMA is permuted so that a lane's 8 weights come from ONE nibble
//    dword (Q4) or two int8 dwords (Q8_0); the staged activations use the
//    same permutation.  When K x tokens exceeds 128 KB of LDS, K runs in
//    phases, restaged between barriers, while the accumulators of up to 2
//    tiles per wave stay in registers.
//  * Weight bytes stream through buffer loads (one descriptor per tile, the
//    chunk offset in an SGPR) into two register chunks: chunk s+1 is in
//    flight while chunk s is dequantized (nibble -> fp16 1024+q with one
//    and-or per pair, packed fp16 offset and scale) and multiplied.
//  * With Wk > 1 the K slices of a tile are summed through LDS in slice
//    order (deterministic) after a barrier; nothing crosses workgroups.
#include <cstdlib>
#include <mutex>

#include "swamp_common.hpp"
#include "swamp_items.hpp"

namespace {

using swamp::Raw;
using swamp::shr16;

typedef _Float16 half8_t __attribute__((ext_vector_type(8)));
typedef _Float16 half2_t __attribute__((ext_vector_type(2)));
typedef float float4_t __attribute__((ext_vector_type(4)));

constexpr int kWaves = 16;      // waves per workgroup, one workgroup per CU
constexpr int kThreads = kWaves * 64;
constexpr int kTok = 64;        // tokens per pass: up to 4 groups of 16 (MFMA M)
constexpr int kRowsTile = 16;   // rows per tile (MFMA N)
constexpr int kJmax = 2;        // tiles per wave whose accumulators stay in registers
constexpr int kXLdsMax = 139264;             // activation bytes in LDS (one K phase)
constexpr int kSlotBytes = kWaves * 16 * 16 * 4;  // one 16x16 fp32 partial per wave
constexpr uint32_t kF16Magic = 0x64006400u;  // fp16 pair (1024, 1024)
constexpr uint32_t kOob = 0x80000000u;       // buffer offset past any descriptor: reads 0

__device__ __forceinline__ half2_t as_h2(uint32_t u) { return __builtin_bit_cast(half2_t, u); }
__device__ __forceinline__ uint32_t as_u(half2_t h) { return __builtin_bit_cast(uint32_t, h); }

// Element (0..63 of the item) that operand slot i (0..7) of MFMA step st
// (0..7) multiplies.  Q4: a step's nibble dword splits into the bytes'
// low nibbles (slots 0..3) and high nibbles (slots 4..7), two fp16 pairs
// each, in byte order.  Q8_0: pair p of the step's two int8 dwords holds
// bytes (0, 2) or (1, 3) of one dword.
template <int DT>
__host__ __device__ constexpr int slot_elem(int st, int i) {
  // Q6_K: step st takes group k = st / 2 (16 weights, one scale) and its
  // half st % 2, 8 consecutive weights; numbered by x offset from the
  // item's first weight (32 k + c)
  if (DT == SWAMP_Q6_K) return 32 * (st / 2) + 8 * (st % 2) + i;
  if (DT == SWAMP_Q8_0) {
    const int p = i / 2, h = i % 2;
    // two int8 dwords per step; pair 0/1 of dword 0 -> bytes (0,2), (1,3)
    const int dw = p / 2, pb = p % 2;
    const int byte = pb + 2 * h;
    return 32 * (st / 4) + 8 * (st % 4) + 4 * dw + byte;
  }
  const int hi = i / 4, byte = i % 4;
  // Q4_0: nibble n of a dword is element n (low nibble of byte b: 2b)
  if (DT == SWAMP_Q4_0) return 32 * (st / 4) + 8 * (st % 4) + 2 * byte + hi;
  // Q4_K quarter: dword st = bytes 4st..4st+3; low nibble -> sub-block A
  // element 4st + byte, high nibble -> sub-block B (item elements 32..63)
  return 32 * hi + 4 * st + byte;
}

// The 8 elements of step st, as loaded by the activation staging: Q4_0 and
// Q8_0 read elements base(st)+0..7; Q4_K reads 4st+0..3 and 32+4st+0..3;
// Q6_K reads x offsets 32(st/2) + 8(st%2) + 0..7 from the item's first
// weight (x_item_base).  slot_local gives the index (0..7) of slot i in
// that 8-float group.
template <int DT>
__host__ __device__ constexpr int stage_elem(int st, int v) {
  if (DT == SWAMP_Q6_K) return 32 * (st / 2) + 8 * (st % 2) + v;
  if (DT == SWAMP_Q4_K) return (v < 4 ? 0 : 32) + 4 * st + (v & 3);
  return 32 * (st / 4) + 8 * (st % 4) + v;
}
template <int DT>
__host__ __device__ constexpr int slot_local(int i) {
  if (DT == SWAMP_Q6_K) return i;
  if (DT == SWAMP_Q8_0) {
    const int p = i / 2, h = i % 2;
    return 4 * (p / 2) + (p % 2) + 2 * h;
  }
  if (DT == SWAMP_Q4_0) return 2 * (i % 4) + i / 4;
  return i;
}
template <int DT>
constexpr bool staging_matches_slots() {
  for (int st = 0; st < 8; st++)
    for (int i = 0; i < 8; i++)
      if (stage_elem<DT>(st, slot_local<DT>(i)) != slot_elem<DT>(st, i)) return false;
  return true;
}
static_assert(staging_matches_slots<SWAMP_Q4_0>(), "Q4_0 staging order");
static_assert(staging_matches_slots<SWAMP_Q8_0>(), "Q8_0 staging order");
static_assert(staging_matches_slots<SWAMP_Q4_K>(), "Q4_K staging order");
static_assert(staging_matches_slots<SWAMP_Q6_K>(), "Q6_K staging order");

// Offset in x of an item's first weight: items are 64 consecutive weights,
// except Q6_K, whose item (block b, half h, columns i) holds 4 runs of 16:
// x[256b + 128h + 16i + 32k + c], k < 4, c < 16 (q6_k.rs:28-44).
template <int DT>
__device__ __forceinline__ size_t x_item_base(int item) {
  if constexpr (DT == SWAMP_Q6_K)
    return size_t(item >> 2) * 256 + 128 * ((item >> 1) & 1) + 16 * (item & 1);
  else
    return size_t(item) * 64;
}

// Q4_K per-item scales as fp16 pairs: sub-block A (item elements 0..31)
// and B (32..63) of quarter `quarter`, W = q * s - m.
struct Q4kScales {
  half2_t sa, ma, sb, mb;
};

// Scales of sub-blocks 2*quarter and 2*quarter+1 (q4_k.rs:37-53), branch
// free: quarters 0/1 read the low 6 bits of bytes 0..3, quarters 2/3 the
// packed high form; bytes 2*(quarter&1) and +1 in both cases.  d*sc and
// dmin*m are exact products of an fp16 and a 6-bit integer, rounded once
// to fp16 by the packed multiply (the same value as rounding the fp32
// product).
__device__ __forceinline__ Q4kScales q4k_item_scales(const Raw<SWAMP_Q4_K> &r, int quarter) {
  const uint32_t sh = 16u * uint32_t(quarter & 1);
  const uint32_t b03 = r.h[1] >> sh, b47 = r.h[2] >> sh, b811 = r.h[3] >> sh;
  uint32_t sm0, sm1;  // (sc | m << 16) of the two sub-blocks
  if (quarter < 2) {  // lane-constant select, compiled to v_cndmask
    sm0 = (b03 & 63u) | ((b47 & 63u) << 16);
    sm1 = ((b03 >> 8) & 63u) | (((b47 >> 8) & 63u) << 16);
  } else {
    sm0 = ((b811 & 0xFu) | ((b03 >> 2) & 0x30u)) |
          ((((b811 >> 4) & 0xFu) | ((b47 >> 2) & 0x30u)) << 16);
    sm1 = (((b811 >> 8) & 0xFu) | ((b03 >> 10) & 0x30u)) |
          ((((b811 >> 12) & 0xFu) | ((b47 >> 10) & 0x30u)) << 16);
  }
  const half2_t off = {_Float16(-1024.0f), _Float16(-1024.0f)};
  const half2_t dd = as_h2(r.h[0]);  // (d, dmin)
  const half2_t p0 = (as_h2(sm0 | kF16Magic) + off) * dd;  // (d*sc0, dmin*m0)
  const half2_t p1 = (as_h2(sm1 | kF16Magic) + off) * dd;
  Q4kScales s;
  s.sa = half2_t{p0[0], p0[0]};
  s.ma = half2_t{p0[1], p0[1]};
  s.sb = half2_t{p1[0], p1[0]};
  s.mb = half2_t{p1[1], p1[1]};
  return s;
}

// The nibbles 0..15 of a dword's four bytes as exact fp16 pairs: the
// low nibbles (lo[0] = bytes 0,1; lo[1] = bytes 2,3), then the high ones.
// A byte below 16 read as OCP fp8 E4M3 is that integer times 2^-9 (the
// denormals run on linearly into the first binade); the convert's scale
// operand contributes its power of two, 2^9, so the pairs are the nibbles
// themselves: 4 converts and 3 bit operations per 8 weights.
struct Nib8 {
  half2_t lo[2], hi[2];
};
__device__ __forceinline__ Nib8 nibbles_f16(uint32_t w) {
  const uint32_t l = w & 0x0F0F0F0Fu, h = (w >> 4) & 0x0F0F0F0Fu;
  Nib8 n;
  n.lo[0] = __builtin_amdgcn_cvt_scalef32_pk_f16_fp8(l, 512.0f, false);
  n.lo[1] = __builtin_amdgcn_cvt_scalef32_pk_f16_fp8(l, 512.0f, true);
  n.hi[0] = __builtin_amdgcn_cvt_scalef32_pk_f16_fp8(h, 512.0f, false);
  n.hi[1] = __builtin_amdgcn_cvt_scalef32_pk_f16_fp8(h, 512.0f, true);
  return n;
}

// 8 fp16 weights (4 packed dwords) of MFMA step st from one item (for
// Q4_K with its scales from q4k_item_scales), in slot_elem order.
template <int DT>
__device__ __forceinline__ half8_t weights_step(const Raw<DT> &r, int st, const Q4kScales &ks) {
  uint32_t o[4];
  if constexpr (DT == SWAMP_Q4_0) {
    const int blk = st / 4, t = st % 4;
    const uint32_t w = blk == 0 ? shr16(r.d[t + 1], r.d[t]) : r.d[5 + t];
    const uint32_t dbits = blk == 0 ? (r.d[0] & 0xFFFFu) : (r.d[4] >> 16);
    const half2_t d2 = as_h2(dbits | (dbits << 16));
    const half2_t m8 = d2 * half2_t{_Float16(-8.0f), _Float16(-8.0f)};  // exact
    const Nib8 n = nibbles_f16(w);
    // (q - 8) * d rounded once, as fma(q, d, -8d)
    o[0] = as_u(__builtin_elementwise_fma(n.lo[0], d2, m8));
    o[1] = as_u(__builtin_elementwise_fma(n.lo[1], d2, m8));
    o[2] = as_u(__builtin_elementwise_fma(n.hi[0], d2, m8));
    o[3] = as_u(__builtin_elementwise_fma(n.hi[1], d2, m8));
  } else if constexpr (DT == SWAMP_Q8_0) {
    const int blk = st / 4, t = st % 4;
    uint32_t w0, w1, dbits;
    if (blk == 0) {
      w0 = shr16(r.d[2 * t + 1], r.d[2 * t]);
      w1 = shr16(r.d[2 * t + 2], r.d[2 * t + 1]);
      dbits = r.d[0] & 0xFFFFu;
    } else {
      w0 = r.d[9 + 2 * t];
      w1 = r.d[10 + 2 * t];
      dbits = r.d[8] >> 16;
    }
    const half2_t d2 = as_h2(dbits | (dbits << 16));
    const half2_t off = {_Float16(-1152.0f), _Float16(-1152.0f)};
    const uint32_t u0 = w0 ^ 0x80808080u, u1 = w1 ^ 0x80808080u;  // q + 128
    // fp16 pairs (1024 + byte) built by one byte permute each: bytes 0 and
    // 2 (or 1 and 3) of u under 0x64 high bytes from the magic word
    constexpr uint32_t kSelEven = 0x07020500u, kSelOdd = 0x07030501u;
    const uint32_t mg = 0x64646464u;
    o[0] = as_u((as_h2(__builtin_amdgcn_perm(mg, u0, kSelEven)) + off) * d2);
    o[1] = as_u((as_h2(__builtin_amdgcn_perm(mg, u0, kSelOdd)) + off) * d2);
    o[2] = as_u((as_h2(__builtin_amdgcn_perm(mg, u1, kSelEven)) + off) * d2);
    o[3] = as_u((as_h2(__builtin_amdgcn_perm(mg, u1, kSelOdd)) + off) * d2);
  } else {
    const Nib8 n = nibbles_f16(r.q[st]);
    // q * s - m rounded once per weight; low nibbles sub-block A, high B
    o[0] = as_u(__builtin_elementwise_fma(n.lo[0], ks.sa, -ks.ma));
    o[1] = as_u(__builtin_elementwise_fma(n.lo[1], ks.sa, -ks.ma));
    o[2] = as_u(__builtin_elementwise_fma(n.hi[0], ks.sb, -ks.mb));
    o[3] = as_u(__builtin_elementwise_fma(n.hi[1], ks.sb, -ks.mb));
  }
  half8_t v;
#pragma unroll
  for (int p = 0; p < 4; p++) {
    half2_t h = as_h2(o[p]);
    v[2 * p] = h[0];
    v[2 * p + 1] = h[1];
  }
  return v;
}

// The group scales of a Q6_K item, d * sc[8h + i + 2k] for k < 4, as fp16
// pairs (one rounding of the exact product).  The item's windows start at
// the block's dword-aligned address; sh (0 or 2 bytes, the block's parity)
// realigns them.
struct Q6kScales {
  half2_t s[4];
};
__device__ __forceinline__ Q6kScales q6k_item_scales(const Raw<SWAMP_Q6_K> &r, int g,
                                                     uint32_t sh) {
  Q6kScales q;
  const uint32_t ii = uint32_t(g & 1);
  const uint32_t s01 = __builtin_amdgcn_alignbyte(r.s[1], r.s[0], sh);
  const uint32_t s23 = __builtin_amdgcn_alignbyte(r.s[2], r.s[1], sh);
  const float d = swamp::f16_bits_to_f32(__builtin_amdgcn_alignbyte(0u, r.d, sh) & 0xFFFFu);
  // int8 scales: bytes i and 2 + i of each scale dword (groups 0..3)
  const int sc[4] = {int(s01 << (24 - 8 * ii)) >> 24, int(s01 << (8 - 8 * ii)) >> 24,
                     int(s23 << (24 - 8 * ii)) >> 24, int(s23 << (8 - 8 * ii)) >> 24};
#pragma unroll
  for (int k = 0; k < 4; k++) {
    const _Float16 v = _Float16(d * float(sc[k]));  // exact product, rounded once
    q.s[k] = half2_t{v, v};
  }
  return q;
}

// 8 fp16 weights of MFMA step st of a Q6_K item, in slot_elem order: group
// k = st / 2, columns c = 8 (st % 2) + 0..7 (dwords t0, t0 + 1 of the ql
// and qh windows, realigned here rather than kept realigned for the whole
// item, which would hold 12 more registers).  The 6-bit codes (low or high
// nibble of ql, two bits of qh) become fp16 1024 + q by one byte permute
// per pair, q - 32 exactly by the packed subtraction, then one rounding in
// the multiply by the group scale.
__device__ __forceinline__ half8_t weights_step_q6k(const Raw<SWAMP_Q6_K> &r, const Q6kScales &q,
                                                    uint32_t sh, int st) {
  const int k = st / 2, t0 = 2 * (st % 2);
  const half2_t off = {_Float16(-1056.0f), _Float16(-1056.0f)};
  constexpr uint32_t kSelLo = 0x04010400u, kSelHi = 0x04030402u;  // bytes (0,1) / (2,3)
  const uint32_t mg = 0x64646464u;
  uint32_t o[4];
#pragma unroll
  for (int j = 0; j < 2; j++) {
    const int t = t0 + j;
    const uint32_t l = (k & 1) ? __builtin_amdgcn_alignbyte(r.b[t + 1], r.b[t], sh)
                               : __builtin_amdgcn_alignbyte(r.a[t + 1], r.a[t], sh);
    const uint32_t h = __builtin_amdgcn_alignbyte(r.h[t + 1], r.h[t], sh);
    const uint32_t nib = k < 2 ? (l & 0x0F0F0F0Fu) : ((l >> 4) & 0x0F0F0F0Fu);
    const uint32_t hb = k == 0   ? (h << 4) & 0x30303030u
                        : k == 1 ? (h << 2) & 0x30303030u
                        : k == 2 ? h & 0x30303030u
                                 : (h >> 2) & 0x30303030u;
    const uint32_t code = nib | hb;  // bytes q, 0..63
    o[2 * j] = as_u((as_h2(__builtin_amdgcn_perm(mg, code, kSelLo)) + off) * q.s[k]);
    o[2 * j + 1] = as_u((as_h2(__builtin_amdgcn_perm(mg, code, kSelHi)) + off) * q.s[k]);
  }
  half8_t v;
#pragma unroll
  for (int p = 0; p < 4; p++) {
    half2_t h = as_h2(o[p]);
    v[2 * p] = h[0];
    v[2 * p + 1] = h[1];
  }
  return v;
}

// Bytes of 4 consecutive items (one item per lane group) and the offset of
// a lane's item inside such a group of 4.
template <int DT>
__host__ __device__ constexpr uint32_t quad_bytes() {
  return DT == SWAMP_Q4_0 ? 144u : DT == SWAMP_Q8_0 ? 272u : DT == SWAMP_Q6_K ? 210u : 144u;
}
template <int DT>
__device__ __forceinline__ uint32_t lane_item_offset(int g) {
  if constexpr (DT == SWAMP_Q4_K) return 16u + 32u * uint32_t(g);  // quarter g after the header
  // Q6_K: item g's ql window from the block's dword-aligned start (64 h + 16 i)
  else if constexpr (DT == SWAMP_Q6_K) return 64u * uint32_t((g >> 1) & 1) + 16u * uint32_t(g & 1);
  else return uint32_t(g) * (quad_bytes<DT>() / 4);
}

// Raw bytes of one item: voff = per-lane offset (row + item), soff = the
// chunk's offset (uniform).  Q4_K also loads the super-block header, which
// sits 16 + 32*g bytes before the lane's quarter.
template <int DT>
__device__ __forceinline__ void load_item(Raw<DT> &r, __amdgpu_buffer_rsrc_t rs, uint32_t voff,
                                          uint32_t soff, int g) {
  if constexpr (DT == SWAMP_Q4_K) {
    const uint32_t hoff = voff - 16u - 32u * uint32_t(g);
    const swamp::u32x4v h = __builtin_amdgcn_raw_buffer_load_b128(rs, hoff, soff, 0);
    const swamp::u32x4v a = __builtin_amdgcn_raw_buffer_load_b128(rs, voff, soff, 0);
    const swamp::u32x4v b = __builtin_amdgcn_raw_buffer_load_b128(rs, voff + 16, soff, 0);
#pragma unroll
    for (int i = 0; i < 4; i++) { r.h[i] = h[i]; r.q[i] = a[i]; r.q[4 + i] = b[i]; }
  } else {
    swamp::load_raw_buf<DT>(r, rs, voff, soff, 0);
  }
}

struct Args {
  const uint8_t *w;
  const float *x;
  float *y;
  int n_tok, n_rows, n_cols;
  uint32_t row_bytes;
  int ipr;         // items (64 weights) per row
  int ipw;         // items per wave and phase (multiple of 4 * kChunk)
  int lwk;         // log2 of Wk, the waves that share one tile (K slices)
  int wtu;         // tile lanes in use (<= 16 / Wk): a tile group's tiles
  int phases;      // K phases; phase p covers items [p*ipp, p*ipp + ipp), ipp = ipw * Wk
  int accumulate;  // y += W x instead of y = W x
  int nkg;         // K groups: workgroups split the row's items into nkg ranges
  int ipk;         // items per K group (one phase each when nkg > 1)
  float *ws;       // nkg > 1: partial sums [nkg][n_tok][n_rows], reduced afterwards
};

// Output of a workgroup: y itself, or with K groups the K group's slice
// of the workspace, which has y's layout [n_tok][n_rows]; partials are
// stored, never accumulated.  One store path keeps the register count
// under the 128 that 16 waves per CU allow.
struct Out {
  float *y;
  int accumulate;
};
__device__ __forceinline__ Out out_of(const Args &a, int kg) {
  if (a.nkg > 1) return {a.ws + size_t(kg) * a.n_tok * a.n_rows, 0};
  return {a.y, a.accumulate};
}

// y[t][row] += / = v for the tokens and rows that exist.
__device__ __forceinline__ void put_y(const Args &a, const Out &o, int t, int row, float v) {
  if (t < a.n_tok && row < a.n_rows) {
    float *d = o.y + size_t(t) * a.n_rows + row;
    *d = o.accumulate ? *d + v : v;
  }
}

// Workgroup barrier that orders LDS only: the weight loads in flight and
// the y stores need not drain (__syncthreads would wait for the stores and,
// the memory counter being in order, for every load issued before them).
__device__ __forceinline__ void lds_barrier() {
  __builtin_amdgcn_fence(__ATOMIC_RELEASE, "workgroup", "local");
  __builtin_amdgcn_s_barrier();
  __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "workgroup", "local");
}

// Stage the activations of items [item0, item0 + n_items) into LDS as
// fragments: entry (item, step, token) holds the 8 fp16 values one lane
// feeds one MFMA, at row 8 * item + step, slot token; rows are TOK + 1
// slots long (one slot of padding), which spreads both the staging writes
// (consecutive rows) and the MFMA reads (consecutive tokens) over the banks.
// Thread e takes step e % 8 of item (e / 8) % n_items of token e / (8 *
// n_items): consecutive threads read consecutive 32-byte runs of one
// token's x, so a wave's loads cover whole cache lines (the token-fastest
// order read 16 rows per instruction, 64 bytes of each line, and staging
// took most of a 16-token pass).  Missing tokens and items past the row
// are zero.  kU entries per thread are loaded before any is written, so the
// loads overlap (fewer inside the main loop, where both weight chunks hold
// registers).
template <int TOK>
constexpr int frag_row() { return TOK + 1; }  // 16-byte slots per fragment row
// Token groups of 16 a pass of TOK tokens runs per weight fragment (4, 8
// and 16 tokens: one, with empty token rows below 16).
template <int TOK>
constexpr int token_groups() { return TOK > 16 ? TOK / 16 : 1; }
template <int NG>
struct Acc {
  float4_t v[NG];
};
// r / n for r < 2^24, n > 0: the float quotient is within one of the
// integer one, which one correction each way makes exact (no integer
// division sequence, whose temporaries would hold registers while the
// first weight chunk is in flight).
__device__ __forceinline__ int div_small(int r, int n, float inv_n) {
  int q = int(float(r) * inv_n);
  q -= q * n > r ? 1 : 0;
  q += (q + 1) * n <= r ? 1 : 0;
  return q;
}
template <int DT, int TOK, int kU>
__device__ __forceinline__ void stage_x(const Args &a, half8_t *xl, int item0, int n_items, int tid) {
  const int n_ent = n_items * 8 * TOK;
  const float inv_n = 1.0f / float(n_items);
  for (int e0 = tid; e0 < n_ent; e0 += kU * kThreads) {
    float4 v0[kU], v1[kU];
#pragma unroll
    for (int u = 0; u < kU; u++) {
      const int e = e0 + u * kThreads;
      const int st = e & 7, r = e >> 3, tok = div_small(r, n_items, inv_n);
      const int item = item0 + (r - tok * n_items);
      v0[u] = v1[u] = make_float4(0.f, 0.f, 0.f, 0.f);
      if (e < n_ent && tok < a.n_tok && item < a.ipr) {
        const float *xp = a.x + size_t(tok) * a.n_cols + x_item_base<DT>(item);
        v0[u] = *reinterpret_cast<const float4 *>(xp + stage_elem<DT>(st, 0));
        v1[u] = *reinterpret_cast<const float4 *>(xp + stage_elem<DT>(st, 4));
      }
    }
#pragma unroll
    for (int u = 0; u < kU; u++) {
      const int e = e0 + u * kThreads;
      if (e < n_ent) {
        const float v[8] = {v0[u].x, v0[u].y, v0[u].z, v0[u].w, v1[u].x, v1[u].y, v1[u].z, v1[u].w};
        half8_t h;
#pragma unroll
        for (int i = 0; i < 8; i++) h[i] = _Float16(v[slot_local<DT>(i)]);
        const int r = e >> 3, tok = div_small(r, n_items, inv_n);
        xl[(8 * (r - tok * n_items) + (e & 7)) * frag_row<TOK>() + tok] = h;
      }
    }
  }
}

// Position of a chunk in a wave's sequence: tile batch, K phase, tile in
// the batch, chunk in the wave's K slice.
struct Pos {
  int batch, p, j, c;
};

// Workgroup b owns tile groups b, b + G, b + 2G, ... (G = gridDim.x); tile
// group q is tiles q*Wt .. q*Wt + Wt-1, one per tile lane.  Wave w is tile
// lane w / Wk and K slice w % Wk.  Tile groups are taken kJmax at a time
// (a batch); per batch the K phases run in order and, inside each, the
// batch's tiles, so each tile's accumulator stays in registers across
// phases.  All waves of a workgroup run the same sequence, which keeps the
// barriers (phase staging, K-slice reduction) uniform.
template <int DT, int TOK, int kChunk, bool kRagged>
__global__ void __launch_bounds__(kThreads, 1) gemv_batched_kernel(Args a) {
  extern __shared__ half8_t xl[];  // [ipp][8 steps][TOK] fragments, then reduction slots
  const int tid = threadIdx.x;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6), lane = tid & 63;
  const int r16 = lane & 15, g = lane >> 4;
  // tile lanes in use: wt = 16 / Wk, or fewer so that the tile groups of
  // one round cover every CU; the waves of a lane past wt load nothing and
  // store nothing (they keep pace with the barriers)
  const int wk = 1 << a.lwk, wt = a.wtu;
  const int tl = wave >> a.lwk, ks = wave & (wk - 1);
  const bool lane_used = tl < wt;
  const int ipp = a.ipw << a.lwk;
  const int n_tiles = (a.n_rows + kRowsTile - 1) / kRowsTile;
  const int n_tg = (n_tiles + wt - 1) / wt;
  // with K groups the grid is nkg blocks of G workgroups; workgroup b of
  // K group kg covers items [kg * ipk, kg * ipk + ipk) of its tiles
  const int G = gridDim.x / a.nkg, b = blockIdx.x % G, kg = blockIdx.x / G;
  const int kitem0 = kg * a.ipk;
  const Out out = out_of(a, kg);
  const int J = (n_tg - 1 - b) / G + 1;  // tile groups of this workgroup (b < n_tg)
  const int cpw = a.ipw / (4 * kChunk);  // chunks per wave, tile and phase
  const int n_chunks = a.phases * cpw * J;
  const int P = a.phases;
  const uint32_t rb = a.row_bytes;
  const uint32_t lane_off = uint32_t(r16) * rb + lane_item_offset<DT>(g);
  const uint32_t chunk_bytes = kChunk * quad_bytes<DT>();
  float *slots = reinterpret_cast<float *>(xl + ipp * 8 * frag_row<TOK>());  // [16 waves][16 tok][16 rows]

  // tiles per batch: one with four token groups (their accumulators take
  // the registers of a second tile)
  constexpr int kJ = token_groups<TOK>() > 2 ? 1 : kJmax;
  auto tile_of = [&](int batch, int j) { return (b + (batch * kJ + j) * G) * wt + tl; };
  auto batch_len = [&](int batch) { return min(kJ, J - batch * kJ); };
  auto advance = [&](Pos &q) {
    if (++q.c < cpw) return;
    q.c = 0;
    if (++q.j < batch_len(q.batch)) return;
    q.j = 0;
    if (++q.p < P) return;
    q.p = 0;
    q.batch++;
  };

  auto issue = [&](Raw<DT> (&r)[kChunk], const Pos &q) {
    // Tiles past the matrix (the last tile group, the issue past the end)
    // re-read the last tile, whose results are never stored.  Every term of
    // the descriptor stays a scalar min/select: a two-sided clamp becomes
    // v_med3, a VGPR temporary that can alias a register an in-flight load
    // still writes, and the wait for it drains the prefetch.
    const int tile = min(tile_of(q.batch, q.j), n_tiles - 1);
    const int row0 = tile * kRowsTile;
    // this wave's items in the chunk: base + g + 4*(c*kChunk + i)
    const int base = kitem0 + q.p * ipp + ks * a.ipw;
    const int first = base + 4 * q.c * kChunk;  // first item of the chunk
    const uint32_t soff = uint32_t(base / 4) * quad_bytes<DT>() + uint32_t(q.c) * chunk_bytes;
    if constexpr (DT == SWAMP_Q6_K) {
      // rows are whole 512-weight pairs of blocks (never ragged); item i of
      // the chunk is in block soff / 210 + i, loaded from its dword-aligned
      // start (the windows are realigned by q6k_item)
      const int nr = first < a.ipr && lane_used ? min(kRowsTile, a.n_rows - row0) : 0;
      const __amdgpu_buffer_rsrc_t rs = swamp::make_rsrc(a.w + size_t(row0) * rb, uint32_t(nr) * rb);
#pragma unroll
      for (int i = 0; i < kChunk; i++)
        swamp::load_raw_buf<DT>(r[i], rs, lane_off, (soff + uint32_t(i) * 210u) & ~3u, g);
    } else if constexpr (!kRagged) {
      // ipr is a multiple of 4 * kChunk: a chunk lies wholly inside the
      // row or wholly past it (then the descriptor has no records and the
      // loads return zeros); no per-lane select before the loads
      const int nr = first < a.ipr && lane_used ? min(kRowsTile, a.n_rows - row0) : 0;
      const __amdgpu_buffer_rsrc_t rs = swamp::make_rsrc(a.w + size_t(row0) * rb, uint32_t(nr) * rb);
#pragma unroll
      for (int i = 0; i < kChunk; i++)
        load_item<DT>(r[i], rs, lane_off + uint32_t(i) * quad_bytes<DT>(), soff, g);
    } else {
      const int nr = lane_used ? min(kRowsTile, a.n_rows - row0) : 0;
      const __amdgpu_buffer_rsrc_t rs = swamp::make_rsrc(a.w + size_t(row0) * rb, uint32_t(nr) * rb);
#pragma unroll
      for (int i = 0; i < kChunk; i++) {
        const bool ok = first + 4 * i + g < a.ipr;
        const uint32_t voff = ok ? lane_off + uint32_t(i) * quad_bytes<DT>() : kOob;
        load_item<DT>(r[i], rs, voff, soff, g);
      }
    }
  };

  Raw<DT> ra[kChunk], rbuf[kChunk];
  Pos qi{0, 0, 0, 0};  // next chunk to issue
  issue(ra, qi);
  advance(qi);
  __builtin_amdgcn_sched_barrier(0);
  stage_x<DT, TOK, 4>(a, xl, kitem0, ipp, tid);
  __syncthreads();

  // this lane's fragments: rows 8 * item + step of its items (item
  // ks * ipw + g + 4 j), slot r16 % TOK, plus 16 per token group
  constexpr int FR = frag_row<TOK>();
  constexpr int NG = token_groups<TOK>();
  const half8_t *xlane = xl + (ks * a.ipw + g) * 8 * FR + (TOK >= 16 ? r16 : r16 % TOK);
  // accumulators of the batch's tiles, one 16x16 block per token group
  // (registers: every index is a constant; an indexed array would live in
  // scratch, whose accesses share the vector memory counter with the
  // weight prefetch and drain it)
  Acc<NG> acc0{}, acc1{};
  Pos qc{0, 0, 0, 0};  // chunk being consumed

  // Result of tile k of a batch: direct stores when a wave owns its tile's
  // whole K range, else a K-slice reduction through LDS.
  auto emit_tile = [&](int batch, int k, const Acc<NG> &v) {
    const int tile = tile_of(batch, k);
    if (wk == 1) {
      if (tile < n_tiles && lane_used) {
#pragma unroll
        for (int gi = 0; gi < NG; gi++)
#pragma unroll
          for (int i = 0; i < 4; i++)
            put_y(a, out, 16 * gi + 4 * g + i, tile * kRowsTile + r16, v.v[gi][i]);
      }
      return;
    }
    // K slices summed through LDS, one token group at a time (each group
    // passed by a constant index: a loop over the groups around the
    // barriers would index the accumulators at run time, in scratch)
    float *mine = slots + wave * 256;
    auto reduce_group = [&](const float4_t &vg, int gi) {
#pragma unroll
      for (int i = 0; i < 4; i++) mine[(4 * g + i) * 16 + r16] = vg[i];
      lds_barrier();
      for (int o = tid; o < wt * 256; o += kThreads) {
        const int otl = o >> 8, e = o & 255;
        const float *src = slots + (otl << a.lwk) * 256 + e;
        float sum = 0.f;
        for (int s2 = 0; s2 < wk; s2++) sum += src[s2 * 256];
        const int otile = (b + (batch * kJ + k) * G) * wt + otl;
        if (otile < n_tiles) put_y(a, out, 16 * gi + (e >> 4), otile * kRowsTile + (e & 15), sum);
      }
      lds_barrier();
    };
    reduce_group(v.v[0], 0);
    if constexpr (NG > 1) reduce_group(v.v[1], 1);
    if constexpr (NG > 2) {
      reduce_group(v.v[2], 2);
      reduce_group(v.v[3], 3);
    }
  };
  auto emit = [&](int batch) {
    const int jb = batch_len(batch);
    emit_tile(batch, 0, acc0);
    if (jb > 1) emit_tile(batch, 1, acc1);
    acc0 = acc1 = Acc<NG>{};
  };

  auto consume = [&](const Raw<DT> (&r)[kChunk]) {
    if (P > 1 && qc.c == 0 && qc.j == 0 && (qc.p | qc.batch) != 0) {
      lds_barrier();  // every wave is done with the previous phase
      stage_x<DT, TOK, 1>(a, xl, kitem0 + qc.p * ipp, ipp, tid);
      lds_barrier();
    }
    const half8_t *xc = xlane + qc.c * kChunk * 32 * FR;
    Acc<NG> c = acc0;
    // Q6_K: block of the chunk's first item (its parity gives each block's
    // misalignment)
    [[maybe_unused]] const int blk0 = (kitem0 + qc.p * ipp + ks * a.ipw) / 4 + qc.c * kChunk;
#pragma unroll
    for (int i = 0; i < kChunk; i++) {
      Q4kScales kq{};
      if constexpr (DT == SWAMP_Q4_K) kq = q4k_item_scales(r[i], g);
      Q6kScales q6{};
      [[maybe_unused]] const uint32_t sh6 = 2u * uint32_t((blk0 + i) & 1);
      if constexpr (DT == SWAMP_Q6_K) q6 = q6k_item_scales(r[i], g, sh6);
#pragma unroll
      for (int st = 0; st < 8; st++) {
        half8_t wb;
        if constexpr (DT == SWAMP_Q6_K) wb = weights_step_q6k(r[i], q6, sh6, st);
        else wb = weights_step<DT>(r[i], st, kq);
        // one dequantized B fragment feeds every token group
#pragma unroll
        for (int gi = 0; gi < NG; gi++) {
          const half8_t xa = xc[(i * 32 + st) * FR + 16 * gi];
          c.v[gi] = __builtin_amdgcn_mfma_f32_16x16x32_f16(xa, wb, c.v[gi], 0, 0, 0);
        }
      }
    }
    acc0 = c;
    if (qc.c == cpw - 1) {
      // next tile of the batch into acc0: rotate by the batch length
      // (selects, not branches: the optimizer turns the branchy form into a
      // store at a dynamic index, i.e. into scratch memory)
      const int jb = batch_len(qc.batch);
#pragma unroll
      for (int gi = 0; gi < NG; gi++) {
        acc0.v[gi] = jb > 1 ? acc1.v[gi] : c.v[gi];
        acc1.v[gi] = c.v[gi];
      }
      if (qc.j == jb - 1 && qc.p == P - 1) emit(qc.batch);
    }
    advance(qc);
  };

  for (int s = 0;;) {
    issue(rbuf, qi);  // past the end: re-reads the last tile
    advance(qi);
    __builtin_amdgcn_sched_barrier(0);
    consume(ra);
    if (++s >= n_chunks) break;
    issue(ra, qi);
    advance(qi);
    __builtin_amdgcn_sched_barrier(0);
    consume(rbuf);
    if (++s >= n_chunks) break;
  }
}

// Sum of the K groups' partials, in K-group order (deterministic):
// y = sum, or y += sum with accumulate.  Up to 16 partials are loaded
// before any is added, so their latencies overlap.
__global__ void kgroup_reduce_kernel(const float *__restrict__ ws, float *__restrict__ y, int nkg,
                                     size_t n, int accumulate) {
  const size_t i = size_t(blockIdx.x) * blockDim.x + threadIdx.x;
  if (i >= n) return;
  float s = 0.f;
  for (int k0 = 0; k0 < nkg; k0 += 16) {
    float v[16];
#pragma unroll
    for (int j = 0; j < 16; j++) v[j] = k0 + j < nkg ? ws[size_t(k0 + j) * n + i] : 0.f;
#pragma unroll
    for (int j = 0; j < 16; j++) s += v[j];  // adding 0 past nkg leaves s unchanged
  }
  y[i] = accumulate ? y[i] + s : s;
}

// Launch geometry: tokens in LDS, items per register chunk, waves per tile,
// K phases (nkg == 1) or K groups (nkg > 1: every workgroup owns one tile
// group and one K range, staged once; the partials go to a.ws).
template <int DT, int TOK, int kChunk, bool kRagged>
int launch_geo(Args a, int lwk, int nkg, hipStream_t s) {
  auto kern = gemv_batched_kernel<DT, TOK, kChunk, kRagged>;
  static std::once_flag once;
  std::call_once(once, [&] {
    (void)hipFuncSetAttribute(reinterpret_cast<const void *>(kern),
                              hipFuncAttributeMaxDynamicSharedMemorySize, kXLdsMax + kSlotBytes);
  });
  const int q = 4 * kChunk;                           // item granule of a wave's K slice
  const int xcap = kXLdsMax / (frag_row<TOK>() * 8 * 16);  // items of activations in LDS
  const int wk = 1 << lwk;
  const int gran = q * wk;
  int ipp;
  if (nkg > 1) {
    a.ipk = ((a.ipr + nkg - 1) / nkg + gran - 1) / gran * gran;
    if (a.ipk > xcap / gran * gran) return SWAMP_ESHAPE;  // chosen so that it fits
    a.nkg = (a.ipr + a.ipk - 1) / a.ipk;
    a.phases = 1;
    ipp = a.ipk;
  } else {
    const int ipp_max = xcap / gran * gran;
    a.nkg = 1;
    a.ipk = 0;
    a.phases = (a.ipr + ipp_max - 1) / ipp_max;
    const int per_phase = (a.ipr + a.phases - 1) / a.phases;
    ipp = (per_phase + gran - 1) / gran * gran;
  }
  a.ipw = ipp / wk;
  a.lwk = lwk;
  const int n_tiles = (a.n_rows + kRowsTile - 1) / kRowsTile;
  const int cus = swamp::device_info().num_cus;
  // Tile groups of 16 / Wk tiles; when one round of them leaves CUs idle
  // (8B gate+up: 224 groups of 8), groups of fewer tiles spread the round
  // over every CU (256 of 7).  K-group plans keep their 16-tile groups.
  a.wtu = kWaves >> lwk;
  if (a.nkg == 1 && (n_tiles + a.wtu - 1) / a.wtu < cus) a.wtu = (n_tiles + cus - 1) / cus;
  const int n_tg = (n_tiles + a.wtu - 1) / a.wtu;
  const int grid = (a.nkg > 1 ? n_tg : std::min(n_tg, cus)) * a.nkg;
  const size_t lds = size_t(ipp) * 8 * frag_row<TOK>() * 16 + (wk > 1 ? kSlotBytes : 0);
  kern<<<unsigned(grid), kThreads, lds, s>>>(a);
  if (hipGetLastError() != hipSuccess) return SWAMP_ELAUNCH;
  if (a.nkg > 1) {
    const size_t n = size_t(a.n_tok) * a.n_rows;
    kgroup_reduce_kernel<<<unsigned((n + 255) / 256), 256, 0, s>>>(a.ws, a.y, a.nkg, n,
                                                                   a.accumulate);
    if (hipGetLastError() != hipSuccess) return SWAMP_ELAUNCH;
  }
  return SWAMP_OK;
}

// launch_geo with the ragged form when a row's items are not a multiple of
// the chunk granule (Q6_K rows never are: whole pairs of blocks).
template <int DT, int TOK, int kChunk>
int launch_geo_r(Args a, int lwk, int nkg, hipStream_t s) {
  if constexpr (DT == SWAMP_Q6_K) {
    return launch_geo<DT, TOK, kChunk, false>(a, lwk, nkg, s);
  } else {
    return a.ipr % (4 * kChunk) ? launch_geo<DT, TOK, kChunk, true>(a, lwk, nkg, s)
                                : launch_geo<DT, TOK, kChunk, false>(a, lwk, nkg, s);
  }
}

// K-group plan of a pass: with one wave per tile (Wk = 1) a workgroup
// covers 16 tiles; when those tile groups fill at most half the CUs and the
// pass's activations are not small (n_tok * K >= 16384 fp32, which the
// K-phase form would stage whole into every workgroup), the row's items are
// split over workgroups instead, each staging only its range: as many
// groups as fill the CUs (at least 4), each a multiple of the chunk granule
// q (8 items, or 4 when that fills more CUs) and within the LDS.  nkg = 1:
// no split.
struct KgPlan {
  int nkg, q;
};
constexpr long kKgMinX = 16384;  // n_tok * K from which K groups pay (measured)
constexpr int kKgMin = 4;        // fewer groups do not pay for the reduction (measured)
KgPlan kg_plan(int n_tok, int n_rows, int n_cols, int tok) {
  static const int forced = [] {  // tuning override: SWAMP_BATCHED_NKG (1 = off)
    const char *e = std::getenv("SWAMP_BATCHED_NKG");
    return e ? std::atoi(e) : 0;
  }();
  const int ipr = (n_cols + 63) / 64;
  const int cus = swamp::device_info().num_cus;
  const int n_tg0 = ((n_rows + kRowsTile - 1) / kRowsTile + kWaves - 1) / kWaves;
  const int xcap_items = kXLdsMax / ((tok + 1) * 8 * 16);
  if (forced == 1) return {1, 8};
  if (forced <= 0 && (2 * n_tg0 > cus || long(n_tok) * n_cols < kKgMinX)) return {1, 8};
  KgPlan best{1, 8};
  for (int q : {8, 4}) {
    const int xcap = xcap_items / q * q;
    if (q > xcap || q > ipr) continue;
    int nkg = forced > 0 ? std::min(forced, ipr / q) : std::min(cus / n_tg0, ipr / q);
    while (nkg >= 1 && nkg < ipr / q && (ipr + nkg - 1) / nkg > xcap) nkg++;
    if (nkg < 2 || (forced <= 0 && (n_tg0 * nkg > cus || nkg < kKgMin))) continue;
    // the groups actually launched (ranges rounded up to the granule)
    const int ipk = ((ipr + nkg - 1) / nkg + q - 1) / q * q;
    const int used = (ipr + ipk - 1) / ipk;
    if (used > best.nkg) best = {used, q};
  }
  return best;
}

// Waves per tile: the power of two that minimises the estimated time,
// rounds of tile groups x (K per wave + the K-slice reduction, costed as
// 1/20 of a full row), the smaller one on ties.
template <int DT, int TOK>
int launch_pass_tok(Args a, hipStream_t s) {
  const int cus = swamp::device_info().num_cus;
  const int n_tiles = (a.n_rows + kRowsTile - 1) / kRowsTile;
  const int xcap = kXLdsMax / (frag_row<TOK>() * 8 * 16);
  if (a.ws) {
    const KgPlan kp = kg_plan(a.n_tok, a.n_rows, a.n_cols, TOK);
    const int nkg = kp.nkg, q = kp.q;
    if (nkg > 1) {
      if constexpr (token_groups<TOK>() == 1 && DT != SWAMP_Q6_K) {
        if (q == 8) return launch_geo_r<DT, TOK, 2>(a, 0, nkg, s);
      }
      return launch_geo_r<DT, TOK, 1>(a, 0, nkg, s);
    }
  }
  static const int forced = [] {  // tuning override: SWAMP_BATCHED_LWK (0..4)
    const char *e = std::getenv("SWAMP_BATCHED_LWK");
    return e ? std::atoi(e) : -1;
  }();
  int best = 0;
  double best_cost = 1e30;
  for (int lwk = 0; lwk <= 4; lwk++) {
    const int wt = kWaves >> lwk;
    const int n_tg = (n_tiles + wt - 1) / wt;
    const int rounds = (n_tg + cus - 1) / cus;
    const double cost = double(rounds) * (1.0 / double(1 << lwk) + (lwk ? 0.05 : 0.0));
    if (cost < best_cost - 1e-9) {
      best_cost = cost;
      best = lwk;
    }
  }
  if (forced >= 0 && forced <= 4) best = forced;
  // The Wk K slices of one phase hold a granule of 4 * kChunk items each:
  // two-item chunks when that fits LDS and the row, else one-item chunks,
  // else fewer slices.
  while (best > 0 && ((4 << best) > xcap || (4 << best) > a.ipr)) best--;
  // token groups keep one-item chunks: their accumulators take the registers
  // a second item would; so does Q6_K (19 registers of raw bytes per item)
  if constexpr (token_groups<TOK>() == 1 && DT != SWAMP_Q6_K) {
    if ((8 << best) <= xcap && (8 << best) <= a.ipr) return launch_geo_r<DT, TOK, 2>(a, best, 1, s);
  }
  return launch_geo_r<DT, TOK, 1>(a, best, 1, s);
}

// Token count of the pass's activation layout (4, 8 or 16).
int pass_tok(int n_tok) {
  return n_tok <= 4 ? 4 : n_tok <= 8 ? 8 : n_tok <= 16 ? 16 : n_tok <= 32 ? 32 : 64;
}

// K groups a pass of n_tok tokens will use (the plan launch_pass_tok follows).
int pass_kgroups(int n_tok, int n_rows, int n_cols) {
  return kg_plan(n_tok, n_rows, n_cols, pass_tok(n_tok)).nkg;
}

template <int DT>
int launch_pass(Args a, hipStream_t s) {
  if (a.n_tok <= 4) return launch_pass_tok<DT, 4>(a, s);
  if (a.n_tok <= 8) return launch_pass_tok<DT, 8>(a, s);
  if (a.n_tok <= 16) return launch_pass_tok<DT, 16>(a, s);
  if (a.n_tok <= 32 || DT == SWAMP_Q6_K) return launch_pass_tok<DT, 32>(a, s);
  if constexpr (DT != SWAMP_Q6_K) return launch_pass_tok<DT, 64>(a, s);
  return SWAMP_ESHAPE;
}

}  // namespace

namespace {

// Tokens per pass of the small-batch kernel: up to 64 (four token groups
// per weight fragment); Q6_K up to 32 (four groups of Q6_K items do not fit
// the 128 registers a lane has at 16 waves per CU).
int pass_len(uint32_t dtype) { return dtype == SWAMP_Q6_K ? 32 : kTok; }

// The GEMM route of a call: more than 64 tokens written over y, on x rounded
// to bf16 (in scratch).  Q6_K stays on the passes at any count: its GEMM
// needs a bf16 copy of the weights in scratch, which the passes do not.
bool gemm_route(uint32_t dtype, int n_tok, int n_cols, int accumulate) {
  return dtype != SWAMP_Q6_K && n_tok > kTok && !accumulate && n_cols % 64 == 0 &&
         size_t(n_tok) * size_t(n_cols) * 2 <= size_t(UINT32_MAX);
}

// Q6_K rows the passes take: whole pairs of blocks (4-byte aligned rows);
// other rows run the decode GEMV per token.
bool q6k_passes(int n_cols) { return n_cols % 512 == 0; }

// Scratch of the small-batch passes: the largest K-group partial block.
size_t kgroup_bytes(uint32_t dtype, int n_tok, int n_rows, int n_cols, int accumulate) {
  size_t ws = 0;
  const int pl = pass_len(dtype);
  for (int t0 = 0; t0 < n_tok; t0 += pl) {
    const int nt = std::min(pl, n_tok - t0);
    if (nt == 1 && !accumulate) continue;  // the decode GEMV
    if (!accumulate && swamp_gemv_tokens_ok(dtype, nt, n_cols)) continue;  // 2 tokens
    const int nkg = pass_kgroups(nt, n_rows, n_cols);
    if (nkg > 1) ws = std::max(ws, size_t(nkg) * nt * n_rows * sizeof(float));
  }
  return ws;
}

}  // namespace

size_t swamp_batched_scratch_bytes(uint32_t dtype, int n_tok, int n_rows, int n_cols,
                                   int accumulate, size_t limit) {
  if (n_tok <= 0 || n_rows <= 0 || n_cols <= 0) return 0;
  if (dtype != SWAMP_Q4_0 && dtype != SWAMP_Q8_0 && dtype != SWAMP_Q4_K && dtype != SWAMP_Q6_K)
    return 0;
  if (dtype == SWAMP_Q6_K && (accumulate || !q6k_passes(n_cols))) return 0;
  if (gemm_route(dtype, n_tok, n_cols, accumulate)) {
    const size_t xb = (size_t(n_tok) * size_t(n_cols) * 2 + 255) & ~size_t(255);
    return xb + swamp_gemm_scratch_bytes(dtype, SWAMP_BF16, n_tok, n_rows, n_cols,
                                         limit > xb ? limit - xb : 0);
  }
  return kgroup_bytes(dtype, n_tok, n_rows, n_cols, accumulate);
}

int swamp_launch_gemv_batched(uint32_t dtype, const void *d_w, const float *d_x, float *d_y,
                              int n_tok, int n_rows, int n_cols, int accumulate,
                              swamp::Scratch &sc, hipStream_t s) {
  if (n_rows == 0 || n_tok == 0) return SWAMP_OK;
  if (dtype == SWAMP_Q6_K && accumulate) return SWAMP_EDTYPE;
  if (dtype == SWAMP_Q6_K && !q6k_passes(n_cols)) {
    // rows of an odd number of blocks: the decode GEMV per token, written
    // over y, as forward_linear_batch's fallback_gemv does for every Q6_K
    // row (linear.rs:336-364)
    for (int t = 0; t < n_tok; t++) {
      const int rc = swamp_launch_gemv(dtype, d_w, d_x + size_t(t) * n_cols,
                                       d_y + size_t(t) * n_rows, n_rows, n_cols, s);
      if (rc) return rc;
    }
    return SWAMP_OK;
  }
  // Batches of more than 64 tokens written over y run as the prefill GEMM
  // on x rounded to bf16 (in scratch).  Without scratch the passes below
  // run instead.
  if (gemm_route(dtype, n_tok, n_cols, accumulate)) {
    const size_t n = size_t(n_tok) * size_t(n_cols);
    if (void *xb = sc.get(n * 2)) {
      int rc = swamp_launch_f32_to_bf16(d_x, xb, n, s);
      if (rc == SWAMP_OK)
        rc = swamp_launch_gemm(dtype, d_w, xb, SWAMP_BF16, d_y, n_tok, n_rows, n_cols, sc, s);
      return rc;
    }
  }
  Args a{};
  a.w = static_cast<const uint8_t *>(d_w);
  a.n_rows = n_rows;
  a.n_cols = n_cols;
  a.row_bytes = uint32_t(swamp::row_bytes(int(dtype), size_t(n_cols)));
  a.ipr = (n_cols + 63) / 64;
  a.accumulate = accumulate;
  // 16 rows of a tile are addressed by one buffer descriptor (32-bit range)
  if (size_t(a.row_bytes) * kRowsTile >= (size_t(1) << 30)) return SWAMP_ESHAPE;
  if (dtype != SWAMP_Q4_0 && dtype != SWAMP_Q8_0 && dtype != SWAMP_Q4_K && dtype != SWAMP_Q6_K)
    return SWAMP_EDTYPE;
  // scratch for the passes that split K over workgroups; without it the
  // passes run as K phases
  const size_t ws_bytes = kgroup_bytes(dtype, n_tok, n_rows, n_cols, accumulate);
  a.ws = ws_bytes ? static_cast<float *>(sc.get(ws_bytes)) : nullptr;
  int rc = SWAMP_OK;
  const int pl = pass_len(dtype);
  for (int t0 = 0; t0 < n_tok && rc == SWAMP_OK; t0 += pl) {
    a.n_tok = std::min(pl, n_tok - t0);
    a.x = d_x + size_t(t0) * n_cols;
    a.y = d_y + size_t(t0) * n_rows;
    // a pass of one token written over y is a GEMV: the one-token kernel
    // streams the weights faster (8B Q4_K gate+up 15 us against 21 us here)
    if (a.n_tok == 1 && !accumulate) {
      rc = swamp_launch_gemv(dtype, d_w, a.x, a.y, n_rows, n_cols, s);
      continue;
    }
    // 2 tokens written over y: the GEMV over both at once, each weight
    // item dequantized once (fp16 x, as the passes below)
    if (!accumulate && swamp_gemv_tokens_ok(dtype, a.n_tok, n_cols)) {
      rc = swamp_launch_gemv_tokens(dtype, d_w, a.x, a.y, a.n_tok, n_rows, n_cols, s);
      continue;
    }
    switch (dtype) {
    case SWAMP_Q4_0: rc = launch_pass<SWAMP_Q4_0>(a, s); break;
    case SWAMP_Q8_0: rc = launch_pass<SWAMP_Q8_0>(a, s); break;
    case SWAMP_Q6_K: rc = launch_pass<SWAMP_Q6_K>(a, s); break;
    default: rc = launch_pass<SWAMP_Q4_K>(a, s); break;
    }
  }
  return rc;
}
