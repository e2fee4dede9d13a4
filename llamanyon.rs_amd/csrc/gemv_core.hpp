// gemv_core.hpp -- the item GEMV kernel and its launch helpers, shared by
// gemv.hip (plain decode GEMV) and gemv_fused.hip (GEMV with the RMSNorm or
// SiLU*up prologue).  The design notes are at the top of gemv.hip.  Each
// including translation unit gets its own instantiations (anonymous
// namespace); the two units compile in parallel.
#pragma once

#include "swamp_common.hpp"
#include "swamp_items.hpp"

#include <algorithm>
#include <cstdlib>
#include <type_traits>

namespace {

using swamp::Raw;
using swamp::load_raw;
using swamp::q4k_scales;
using swamp::shr16;

typedef _Float16 half2_t __attribute__((ext_vector_type(2)));

// Prologue applied to x as the workgroup loads it: the f32 step the engine
// runs between the previous kernel and this GEMV.
//   kProRmsNorm: x <- (x * inv_rms) * w_norm, inv_rms = 1 / sqrt(sum x^2 / n
//                + eps)                       (rmsnorm, swamp-engine/src/ops.rs:188-201)
//   kProSwiGLU:  x <- silu(x) * up, silu(v) = v / (1 + exp(-v))
//                                             (silu, mul_in_place, ops.rs:203-214)
// Both use the hardware reciprocal square root / exp2 / reciprocal (about
// 1 ulp), well inside what the fp16 rounding of x already costs.
//   kProSwiGLUAcc: as kProSwiGLU, and y += W x (the residual add) instead
//                of y = W x
enum { kProNone = 0, kProRmsNorm = 1, kProSwiGLU = 2, kProSwiGLUAcc = 3 };
struct Pro {
  const float *x2 = nullptr;  // kProRmsNorm: w_norm; kProSwiGLU*: up (x is gate)
  float eps = 0.f;            // kProRmsNorm: epsilon
};

__device__ __forceinline__ float dot2(uint32_t a, uint32_t b, float c) {
  return __builtin_amdgcn_fdot2(__builtin_bit_cast(half2_t, a), __builtin_bit_cast(half2_t, b), c,
                                false);
}

// Two floats -> packed fp16 pair, round to nearest even (V_CVT_PK_F16_F32).
__device__ __forceinline__ uint32_t pack_f16(float lo, float hi) {
  half2_t v;
  v[0] = (_Float16)lo;
  v[1] = (_Float16)hi;
  return __builtin_bit_cast(uint32_t, v);
}

// fp16 pair (1024, 1024) in a VGPR the compiler cannot see through, so that
// (w & mask) | magic selects V_AND_OR_B32 with the mask in an SGPR (gfx9
// VOP3 encodings take no literal).
__device__ __forceinline__ uint32_t f16_magic() {
  uint32_t m;
  asm("v_mov_b32 %0, 0x64006400" : "=v"(m));
  return m;
}

// Four fp16 pairs of one nibble dword w:
//   P0 = lo(b0), lo(b2)   P1 = lo(b1), lo(b3)     (value 1024 + q)
//   P2 = hi(b0), hi(b2)   P3 = hi(b1), hi(b3)     (value 1024 + 16 q)
__device__ __forceinline__ void nib_pairs(uint32_t w, uint32_t m, uint32_t (&P)[4]) {
  const uint32_t s = w >> 8;
  P[0] = (w & 0x000F000Fu) | m;
  P[1] = (s & 0x000F000Fu) | m;
  P[2] = (w & 0x00F000F0u) | m;
  P[3] = (s & 0x00F000F0u) | m;
}

// Element (0..63 within the item) that half h of pair p of nibble dword t
// multiplies.  Nibble n of dword t (n = 0..7, bit offset 4n) is:
//   Q4_0: byte n/2 of the dword, element 8t' + 2(n/2) + (n%2) of block t/4
//         (interleaved layout, q4_0.rs:30-35), t' = t%4;
//   Q4_K: low nibble of byte b -> sub-block A element 4t+b,
//         high nibble -> sub-block B (item elements 32..63) element 4t+b.
// Pairs p = 2, 3 hold high nibbles (their x is divided by 16).
template <int DT>
__host__ __device__ constexpr int nib_elem(int t, int p, int h) {
  const int byte = (p & 1) + 2 * h;  // P0: b0,b2  P1: b1,b3  P2: b0,b2  P3: b1,b3
  const int high = p >= 2;
  if (DT == SWAMP_Q4_0) return 32 * (t / 4) + 8 * (t % 4) + 2 * byte + high;
  return 32 * high + 4 * t + byte;  // Q4_K
}

// Element of half h of pair j (0, 1) of int8 dword t of a Q8_0 item (after
// the block-0 bytes are realigned): bytes j and j + 2.
__host__ __device__ constexpr int q8_elem(int t, int j, int h) { return 4 * t + j + 2 * h; }

// Per-lane x fragment for one item: fp16 pairs in the order the weight
// pairs are formed, the offset corrections, and the item's scale 2^e.
template <int DT>
struct XFrag;

template <>
struct XFrag<SWAMP_Q4_0> {
  uint32_t p[32];  // 8 nibble dwords x 4 pairs
  float c[2];      // per block: sum of 1032 x (low) + 1152 x/16 (high)
  float scale;
};
template <>
struct XFrag<SWAMP_Q4_K> {
  uint32_t p[32];
  float sa;    // sum of x over sub-block A (low nibbles)
  float sb16;  // sum of x/16 over sub-block B (high nibbles)
  float scale;
};
template <>
struct XFrag<SWAMP_Q8_0> {
  uint32_t p[32];  // 16 int8 dwords x 2 pairs
  float c[2];      // per block: 1152 * sum of x
  float scale;
};
template <>
struct XFrag<SWAMP_Q6_K> {
  uint32_t p[32];  // pair 8t + 2j + e: group j, dword t, bytes (e, e + 2)
  float c[4];      // per group: the offset sum (1056 x or 1536 x/16)
  float scale;
};

// Issue the loads of one item's 64 x values (clamped item: always in
// bounds; a lane past the row end zeroes its values afterwards).  A Q6_K
// item of block b, half h, columns i has x[256b + 128h + 32j + 16i + c] for
// j < 4, c < 16 in xv[4j + c/4].
template <int DT>
__device__ __forceinline__ void load_x(float4 (&xv)[16], const float *__restrict__ x, int item) {
  if constexpr (DT == SWAMP_Q6_K) {
    const float *xb = x + size_t(item >> 2) * 256 + 128 * ((item >> 1) & 1) + 16 * (item & 1);
#pragma unroll
    for (int j = 0; j < 4; j++) {
      const float4 *xp = reinterpret_cast<const float4 *>(xb + 32 * j);
#pragma unroll
      for (int k = 0; k < 4; k++) xv[4 * j + k] = xp[k];
    }
  } else {
    const float4 *xp = reinterpret_cast<const float4 *>(x + size_t(item) * 64);
#pragma unroll
    for (int i = 0; i < 16; i++) xv[i] = xp[i];
  }
}

template <int DT>
__device__ __forceinline__ void build_xfrag(XFrag<DT> &xf, const float4 (&x4)[16], bool valid) {
  float xv[64];
#pragma unroll
  for (int i = 0; i < 16; i++) {
    xv[4 * i] = x4[i].x; xv[4 * i + 1] = x4[i].y; xv[4 * i + 2] = x4[i].z; xv[4 * i + 3] = x4[i].w;
  }
  float amax = 0.f;
#pragma unroll
  for (int i = 0; i < 64; i++) {
    xv[i] = valid ? xv[i] : 0.f;
    amax = fmaxf(amax, fabsf(xv[i]));
  }
  // scale 2^(141 - E) maps amax (biased exponent E) into [2^14, 2^15)
  int E = int((__float_as_uint(amax) >> 23) & 0xFFu);
  E = E < 15 ? 15 : E > 254 ? 254 : E;
  const float down = __uint_as_float(uint32_t(268 - E) << 23);
  xf.scale = __uint_as_float(uint32_t(E - 14) << 23);
  const float down16 = down * 0.0625f;
  const uint32_t k_lo = 0x64086408u;  // fp16 pair (1032, 1032)
  const uint32_t k_hi = 0x64806480u;  // fp16 pair (1152, 1152)
  const uint32_t k_one = 0x3C003C00u;  // fp16 pair (1, 1)
  if constexpr (DT == SWAMP_Q6_K) {
    // groups j = 0, 1 hold 1024 + q (x scaled by down), groups 2, 3 hold
    // 1024 + 16 q (x scaled by down/16); sum (q - 32) x = S - c with
    // c = 1056 sum x (j < 2) or 1536 sum x/16 (j >= 2)
    const uint32_t k_c01 = 0x64206420u;  // fp16 pair (1056, 1056)
    const uint32_t k_c23 = 0x66006600u;  // fp16 pair (1536, 1536)
#pragma unroll
    for (int j = 0; j < 4; j++) {
      const float f = j >= 2 ? down16 : down;
      float c = 0.f;
#pragma unroll
      for (int t = 0; t < 4; t++) {
        const float *v = xv + 16 * j + 4 * t;
        const uint32_t p0 = pack_f16(v[0] * f, v[2] * f);
        const uint32_t p1 = pack_f16(v[1] * f, v[3] * f);
        xf.p[8 * t + 2 * j] = p0;
        xf.p[8 * t + 2 * j + 1] = p1;
        c = dot2(j >= 2 ? k_c23 : k_c01, p0, c);
        c = dot2(j >= 2 ? k_c23 : k_c01, p1, c);
      }
      xf.c[j] = c;
    }
  } else if constexpr (DT == SWAMP_Q8_0) {
    float c0 = 0.f, c1 = 0.f;
#pragma unroll
    for (int t = 0; t < 16; t++)
#pragma unroll
      for (int j = 0; j < 2; j++) {
        const uint32_t pr = pack_f16(xv[q8_elem(t, j, 0)] * down, xv[q8_elem(t, j, 1)] * down);
        xf.p[2 * t + j] = pr;
        if (t < 8) c0 = dot2(k_hi, pr, c0);
        else c1 = dot2(k_hi, pr, c1);
      }
    xf.c[0] = c0;
    xf.c[1] = c1;
  } else {
    float s0 = 0.f, s1 = 0.f;
#pragma unroll
    for (int t = 0; t < 8; t++)
#pragma unroll
      for (int p = 0; p < 4; p++) {
        const float f = p >= 2 ? down16 : down;
        const uint32_t pr = pack_f16(xv[nib_elem<DT>(t, p, 0)] * f, xv[nib_elem<DT>(t, p, 1)] * f);
        xf.p[4 * t + p] = pr;
        if constexpr (DT == SWAMP_Q4_0) {
          // both halves of a pair lie in block t / 4
          if (t < 4) s0 = dot2(p >= 2 ? k_hi : k_lo, pr, s0);
          else s1 = dot2(p >= 2 ? k_hi : k_lo, pr, s1);
        } else {
          if (p < 2) s0 = dot2(k_one, pr, s0);
          else s1 = dot2(k_one, pr, s1);
        }
      }
    if constexpr (DT == SWAMP_Q4_0) {
      xf.c[0] = s0;
      xf.c[1] = s1;
    } else {
      xf.sa = s0;
      xf.sb16 = s1;
    }
  }
}

template <int DT>
__device__ __forceinline__ float item_dot(const Raw<DT> &r, const XFrag<DT> &xf, int item,
                                          uint32_t m) {
  if constexpr (DT == SWAMP_Q4_0) {
    const float d0 = swamp::f16_bits_to_f32(r.d[0] & 0xFFFFu);
    const float d1 = swamp::f16_bits_to_f32(r.d[4] >> 16);
    float s0 = 0.f, s1 = 0.f;
#pragma unroll
    for (int t = 0; t < 8; t++) {
      const uint32_t w = t < 4 ? shr16(r.d[t + 1], r.d[t]) : r.d[t + 1];
      uint32_t P[4];
      nib_pairs(w, m, P);
#pragma unroll
      for (int p = 0; p < 4; p++) {
        if (t < 4) s0 = dot2(P[p], xf.p[4 * t + p], s0);
        else s1 = dot2(P[p], xf.p[4 * t + p], s1);
      }
    }
    return (d0 * (s0 - xf.c[0]) + d1 * (s1 - xf.c[1])) * xf.scale;
  } else if constexpr (DT == SWAMP_Q8_0) {
    const float d0 = swamp::f16_bits_to_f32(r.d[0] & 0xFFFFu);
    const float d1 = swamp::f16_bits_to_f32(r.d[8] >> 16);
    float s0 = 0.f, s1 = 0.f;
#pragma unroll
    for (int t = 0; t < 16; t++) {
      const uint32_t w = (t < 8 ? shr16(r.d[t + 1], r.d[t]) : r.d[t + 1]) ^ 0x80808080u;
      const uint32_t P0 = (w & 0x00FF00FFu) | m;
      const uint32_t P1 = ((w >> 8) & 0x00FF00FFu) | m;
      if (t < 8) {
        s0 = dot2(P0, xf.p[2 * t], s0);
        s0 = dot2(P1, xf.p[2 * t + 1], s0);
      } else {
        s1 = dot2(P0, xf.p[2 * t], s1);
        s1 = dot2(P1, xf.p[2 * t + 1], s1);
      }
    }
    return (d0 * (s0 - xf.c[0]) + d1 * (s1 - xf.c[1])) * xf.scale;
  } else if constexpr (DT == SWAMP_Q6_K) {
    // realign the windows of an odd block by 2 bytes (item bit 2 = block
    // parity; rows start 4-byte aligned)
    const uint32_t sh = uint32_t(item & 4) >> 1;
    const uint32_t ii = uint32_t(item & 1);
    const uint32_t s01 = __builtin_amdgcn_alignbyte(r.s[1], r.s[0], sh);  // sc[8h .. 8h+3]
    const uint32_t s23 = __builtin_amdgcn_alignbyte(r.s[2], r.s[1], sh);  // sc[8h+4 .. 8h+7]
    const float d = swamp::f16_bits_to_f32(__builtin_amdgcn_alignbyte(0u, r.d, sh) & 0xFFFFu);
    // group j uses sc[8h + i + 2j]: byte i + 2j of s01:s23
    const float sc0 = float(int(s01 << (24 - 8 * ii)) >> 24);
    const float sc1 = float(int(s01 << (8 - 8 * ii)) >> 24);
    const float sc2 = float(int(s23 << (24 - 8 * ii)) >> 24);
    const float sc3 = float(int(s23 << (8 - 8 * ii)) >> 24);
    const uint32_t lo = 0x000F000Fu, hi = 0x00F000F0u, b45 = 0x00300030u, b89 = 0x03000300u;
    float g0 = 0.f, g1 = 0.f, g2 = 0.f, g3 = 0.f;
#pragma unroll
    for (int t = 0; t < 4; t++) {
      const uint32_t A = __builtin_amdgcn_alignbyte(r.a[t + 1], r.a[t], sh);
      const uint32_t B = __builtin_amdgcn_alignbyte(r.b[t + 1], r.b[t], sh);
      const uint32_t H = __builtin_amdgcn_alignbyte(r.h[t + 1], r.h[t], sh);
      // qh fields moved to bits 4-5 (low-nibble groups) and 8-9 (high-
      // nibble groups, whose nibble stays at bits 4-7): bytes 0, 2 first
      const uint32_t hA = H << 4, hB = H >> 4, hC = H << 2, hD = H >> 6;
      const uint32_t sA = A >> 8, sB = B >> 8;
      g0 = dot2((A & lo) | (hA & b45) | m, xf.p[8 * t + 0], g0);
      g0 = dot2((sA & lo) | (hB & b45) | m, xf.p[8 * t + 1], g0);
      g1 = dot2((B & lo) | (hC & b45) | m, xf.p[8 * t + 2], g1);
      g1 = dot2((sB & lo) | (hD & b45) | m, xf.p[8 * t + 3], g1);
      g2 = dot2((A & hi) | (hA & b89) | m, xf.p[8 * t + 4], g2);
      g2 = dot2((sA & hi) | (hB & b89) | m, xf.p[8 * t + 5], g2);
      g3 = dot2((B & hi) | (hC & b89) | m, xf.p[8 * t + 6], g3);
      g3 = dot2((sB & hi) | (hD & b89) | m, xf.p[8 * t + 7], g3);
    }
    return d * (sc0 * (g0 - xf.c[0]) + sc1 * (g1 - xf.c[1]) + sc2 * (g2 - xf.c[2]) +
                sc3 * (g3 - xf.c[3])) *
           xf.scale;
  } else {
    const float d = swamp::f16_bits_to_f32(r.h[0] & 0xFFFFu);
    const float dmin = swamp::f16_bits_to_f32(r.h[0] >> 16);
    uint32_t sc0, m0, sc1, m1;
    q4k_scales(r.h, 2 * (item & 3), sc0, m0, sc1, m1);
    float sa = 0.f, sb = 0.f;
#pragma unroll
    for (int t = 0; t < 8; t++) {
      uint32_t P[4];
      nib_pairs(r.q[t], m, P);
      sa = dot2(P[0], xf.p[4 * t + 0], sa);
      sa = dot2(P[1], xf.p[4 * t + 1], sa);
      sb = dot2(P[2], xf.p[4 * t + 2], sb);
      sb = dot2(P[3], xf.p[4 * t + 3], sb);
    }
    // sum (d*sc*q - dmin*m) x = d*sc*(S - 1024 Sx) - dmin*m*Sx, with B's x
    // carried as x/16
    const float qa = sa - 1024.0f * xf.sa, qb = sb - 1024.0f * xf.sb16;
    return (d * (float(sc0) * qa + float(sc1) * qb) -
            dmin * (float(m0) * xf.sa + float(m1) * 16.0f * xf.sb16)) *
           xf.scale;
  }
}

// ---- fp32 x: the reference's arithmetic ------------------------------------
// The default GEMV multiplies the exact weight codes by unrounded fp32 x and
// sums in fp32, as forward_linear (linear.rs:81-85) and the scalar Q4_K
// GEMV (fused_gemv_q4k.rs:484-504) do.  Q4_0 and Q4_K nibbles become their
// exact codes q as fp16 pairs through the fp8 convert (nib4_f16); Q6_K
// pairs take one and-or onto the fp16 magic (1024 + q, or 1024 + 16 q for a
// nibble left in place) and one packed fp16 add or fma that removes it,
// exactly, leaving q - 32.  V_FMA_MIX_F32 converts each half to fp32
// (exact) and fuses it with the fp32 x value and the fp32 partial sum: one
// rounding per weight, as in an fp32 FMA.  Q8_0 bytes are converted with a
// sign-extending sub-dword convert.  The block scales and offsets are
// applied per block: Q4_0 d (sum(q x) - 8 sum(x)); Q8_0, Q6_K d * sum;
// Q4_K (d sc) sum(q x) - (dmin m) sum(x); sum(x) per block or sub-block is
// taken once per lane, x being the same for every row it streams.
// Per 8 nibbles (Q4): 3 bit operations + 4 converts + 8 fma_mix.

template <int DT>
struct XFrag32 {
  float x[64];   // the item's x in the order item_dot forms its weight pairs
  float sa, sb;  // Q4_0: sum of x over block 0 (elements 0..31) and block 1 (32..63);
                 // Q4_K: over sub-block A (0..31) and B (32..63)
};

__device__ __forceinline__ half2_t h2(uint32_t v) { return __builtin_bit_cast(half2_t, v); }
__device__ __forceinline__ half2_t h2c(float c) { return half2_t{(_Float16)c, (_Float16)c}; }

// The eight nibbles of a dword as exact fp16 pairs: pair 0 = low nibbles of
// bytes 0, 1; pair 1 = bytes 2, 3; pairs 2, 3 the high nibbles.  A byte below
// 16 read as OCP fp8 E4M3 is that integer times 2^-9 (the denormals run on
// linearly into the first binade); the convert's scale operand contributes
// its power of two, 2^9: 3 bit operations and 4 converts per 8 weights.
__device__ __forceinline__ void nib4_f16(uint32_t w, half2_t (&E)[4]) {
  const uint32_t l = w & 0x0F0F0F0Fu, h = (w >> 4) & 0x0F0F0F0Fu;
  E[0] = __builtin_amdgcn_cvt_scalef32_pk_f16_fp8(l, 512.0f, false);
  E[1] = __builtin_amdgcn_cvt_scalef32_pk_f16_fp8(l, 512.0f, true);
  E[2] = __builtin_amdgcn_cvt_scalef32_pk_f16_fp8(h, 512.0f, false);
  E[3] = __builtin_amdgcn_cvt_scalef32_pk_f16_fp8(h, 512.0f, true);
}
// Element (0..63 of the item) that half h of pair p of nibble dword t holds
// in nib4_f16's order: byte 2 (p % 2) + h, low nibble for p < 2.
template <int DT>
__host__ __device__ constexpr int cvt_elem(int t, int p, int h) {
  const int byte = 2 * (p & 1) + h, high = p >> 1;
  if (DT == SWAMP_Q4_0) return 32 * (t / 4) + 8 * (t % 4) + 2 * byte + high;
  return 32 * high + 4 * t + byte;  // Q4_K
}
// every element of the item exactly once
template <int DT>
constexpr bool cvt_elem_is_permutation() {
  bool seen[64] = {};
  for (int t = 0; t < 8; t++)
    for (int p = 0; p < 4; p++)
      for (int h = 0; h < 2; h++) {
        const int e = cvt_elem<DT>(t, p, h);
        if (e < 0 || e >= 64 || seen[e]) return false;
        seen[e] = true;
      }
  return true;
}
static_assert(cvt_elem_is_permutation<SWAMP_Q4_0>(), "Q4_0 fp32-x element order");
static_assert(cvt_elem_is_permutation<SWAMP_Q4_K>(), "Q4_K fp32-x element order");

// a += e.lo * x0, b += e.hi * x1 (two V_FMA_MIX_F32 with op_sel)
__device__ __forceinline__ void fma2(half2_t e, float x0, float x1, float &a, float &b) {
  a = __builtin_fmaf(float(e[0]), x0, a);
  b = __builtin_fmaf(float(e[1]), x1, b);
}

template <int DT>
__device__ __forceinline__ void build_xfrag(XFrag32<DT> &xf, const float4 (&x4)[16], bool valid) {
  float xv[64];
#pragma unroll
  for (int i = 0; i < 16; i++) {
    xv[4 * i] = x4[i].x; xv[4 * i + 1] = x4[i].y; xv[4 * i + 2] = x4[i].z; xv[4 * i + 3] = x4[i].w;
  }
#pragma unroll
  for (int i = 0; i < 64; i++) xv[i] = valid ? xv[i] : 0.f;
  if constexpr (DT == SWAMP_Q6_K) {
    // pair 8t + 2j + e (group j, dword t, bytes e and e + 2) -> x[16t + 4j + 2e + h]
#pragma unroll
    for (int t = 0; t < 4; t++)
#pragma unroll
      for (int j = 0; j < 4; j++)
#pragma unroll
        for (int e = 0; e < 2; e++)
#pragma unroll
          for (int h = 0; h < 2; h++) xf.x[16 * t + 4 * j + 2 * e + h] = xv[16 * j + 4 * t + e + 2 * h];
  } else if constexpr (DT == SWAMP_Q8_0) {
#pragma unroll
    for (int i = 0; i < 64; i++) xf.x[i] = xv[i];  // byte b of dword t is element 4t + b
  } else {
#pragma unroll
    for (int t = 0; t < 8; t++)
#pragma unroll
      for (int p = 0; p < 4; p++)
#pragma unroll
        for (int h = 0; h < 2; h++) xf.x[8 * t + 2 * p + h] = xv[cvt_elem<DT>(t, p, h)];
    float sa = 0.f, sb = 0.f;
#pragma unroll
    for (int i = 0; i < 32; i++) {
      sa += xv[i];
      sb += xv[32 + i];
    }
    xf.sa = sa;
    xf.sb = sb;
  }
}

template <int DT>
__device__ __forceinline__ float item_dot(const Raw<DT> &r, const XFrag32<DT> &xf, int item,
                                          uint32_t m) {
  if constexpr (DT == SWAMP_Q4_0) {
    const float d0 = swamp::f16_bits_to_f32(r.d[0] & 0xFFFFu);
    const float d1 = swamp::f16_bits_to_f32(r.d[4] >> 16);
    float s0a = 0.f, s0b = 0.f, s1a = 0.f, s1b = 0.f;
#pragma unroll
    for (int t = 0; t < 8; t++) {
      const uint32_t w = t < 4 ? shr16(r.d[t + 1], r.d[t]) : r.d[t + 1];
      half2_t E[4];
      nib4_f16(w, E);  // the codes q, exact
      const float *x = xf.x + 8 * t;
#pragma unroll
      for (int p = 0; p < 4; p++) {
        if (t < 4) fma2(E[p], x[2 * p], x[2 * p + 1], s0a, s0b);
        else fma2(E[p], x[2 * p], x[2 * p + 1], s1a, s1b);
      }
    }
    // sum (q - 8) x = sum(q x) - 8 sum(x), per block; 8 sum(x) is exact
    return d0 * ((s0a + s0b) - 8.0f * xf.sa) + d1 * ((s1a + s1b) - 8.0f * xf.sb);
  } else if constexpr (DT == SWAMP_Q8_0) {
    const float d0 = swamp::f16_bits_to_f32(r.d[0] & 0xFFFFu);
    const float d1 = swamp::f16_bits_to_f32(r.d[8] >> 16);
    float s0a = 0.f, s0b = 0.f, s1a = 0.f, s1b = 0.f;
#pragma unroll
    for (int t = 0; t < 16; t++) {
      const uint32_t w = t < 8 ? shr16(r.d[t + 1], r.d[t]) : r.d[t + 1];
      const float *x = xf.x + 4 * t;
      float &a = t < 8 ? s0a : s1a;
      float &b = t < 8 ? s0b : s1b;
      a = __builtin_fmaf(float(int8_t(w)), x[0], a);
      b = __builtin_fmaf(float(int8_t(w >> 8)), x[1], b);
      a = __builtin_fmaf(float(int8_t(w >> 16)), x[2], a);
      b = __builtin_fmaf(float(int32_t(w) >> 24), x[3], b);
    }
    return d0 * (s0a + s0b) + d1 * (s1a + s1b);
  } else if constexpr (DT == SWAMP_Q6_K) {
    const uint32_t sh = uint32_t(item & 4) >> 1;
    const uint32_t ii = uint32_t(item & 1);
    const uint32_t s01 = __builtin_amdgcn_alignbyte(r.s[1], r.s[0], sh);
    const uint32_t s23 = __builtin_amdgcn_alignbyte(r.s[2], r.s[1], sh);
    const float d = swamp::f16_bits_to_f32(__builtin_amdgcn_alignbyte(0u, r.d, sh) & 0xFFFFu);
    const float sc0 = float(int(s01 << (24 - 8 * ii)) >> 24);
    const float sc1 = float(int(s01 << (8 - 8 * ii)) >> 24);
    const float sc2 = float(int(s23 << (24 - 8 * ii)) >> 24);
    const float sc3 = float(int(s23 << (8 - 8 * ii)) >> 24);
    const uint32_t lo = 0x000F000Fu, hi = 0x00F000F0u, b45 = 0x00300030u, b89 = 0x03000300u;
    // (1024 + q) - 1056 = q - 32;  (1024 + 16 q) / 16 - 96 = q - 32
    const half2_t lo_off = h2c(1056.f), hi_mul = h2c(0.0625f), hi_off = h2c(96.f);
    float g[4][2] = {};
#pragma unroll
    for (int t = 0; t < 4; t++) {
      const uint32_t A = __builtin_amdgcn_alignbyte(r.a[t + 1], r.a[t], sh);
      const uint32_t B = __builtin_amdgcn_alignbyte(r.b[t + 1], r.b[t], sh);
      const uint32_t H = __builtin_amdgcn_alignbyte(r.h[t + 1], r.h[t], sh);
      const uint32_t hA = H << 4, hB = H >> 4, hC = H << 2, hD = H >> 6;
      const uint32_t sA = A >> 8, sB = B >> 8;
      const half2_t E[8] = {
          h2((A & lo) | (hA & b45) | m) - lo_off,           h2((sA & lo) | (hB & b45) | m) - lo_off,
          h2((B & lo) | (hC & b45) | m) - lo_off,           h2((sB & lo) | (hD & b45) | m) - lo_off,
          h2((A & hi) | (hA & b89) | m) * hi_mul - hi_off,  h2((sA & hi) | (hB & b89) | m) * hi_mul - hi_off,
          h2((B & hi) | (hC & b89) | m) * hi_mul - hi_off,  h2((sB & hi) | (hD & b89) | m) * hi_mul - hi_off};
      const float *x = xf.x + 16 * t;
#pragma unroll
      for (int k = 0; k < 8; k++) fma2(E[k], x[2 * k], x[2 * k + 1], g[k >> 1][0], g[k >> 1][1]);
    }
    return d * (sc0 * (g[0][0] + g[0][1]) + sc1 * (g[1][0] + g[1][1]) +
                sc2 * (g[2][0] + g[2][1]) + sc3 * (g[3][0] + g[3][1]));
  } else {
    const float d = swamp::f16_bits_to_f32(r.h[0] & 0xFFFFu);
    const float dmin = swamp::f16_bits_to_f32(r.h[0] >> 16);
    uint32_t sc0, m0, sc1, m1;
    q4k_scales(r.h, 2 * (item & 3), sc0, m0, sc1, m1);
    float sa0 = 0.f, sa1 = 0.f, sb0 = 0.f, sb1 = 0.f;
#pragma unroll
    for (int t = 0; t < 8; t++) {
      half2_t E[4];
      nib4_f16(r.q[t], E);  // the codes q, exact: low nibbles sub-block A, high B
      const float *x = xf.x + 8 * t;
      fma2(E[0], x[0], x[1], sa0, sa1);
      fma2(E[1], x[2], x[3], sa0, sa1);
      fma2(E[2], x[4], x[5], sb0, sb1);
      fma2(E[3], x[6], x[7], sb0, sb1);
    }
    // sum ((d sc) q - dmin m) x = (d sc) sum(q x) - (dmin m) sum(x), per sub-block
    const float sv0 = d * float(sc0), mv0 = dmin * float(m0);
    const float sv1 = d * float(sc1), mv1 = dmin * float(m1);
    return (sv0 * (sa0 + sa1) - mv0 * xf.sa) + (sv1 * (sb0 + sb1) - mv1 * xf.sb);
  }
}

// ---- stage stamps (measurement build) ------------------------------------
// Built with SWAMP_STAGE_STAMPS (libswamp_gpu_stamps.so, bench.py
// --gemv-stages), each wave of the decode GEMV records the real-time
// counter (100 MHz) at five points: kernel entry, x landed in LDS (after
// the staging barrier), x fragment built, first tile stored, last tile
// stored.  The regular build compiles the marks away.
#ifdef SWAMP_STAGE_STAMPS
constexpr int kStampWaves = 16384;
__device__ uint64_t g_gemv_stamps[kStampWaves * 8];
struct Stamps {
  uint64_t t[5] = {};
  __device__ __forceinline__ void mark(int i) { t[i] = __builtin_amdgcn_s_memrealtime(); }
  __device__ __forceinline__ void put(int wave_id, int lane) {
    if (lane == 0 && wave_id < kStampWaves)
      for (int i = 0; i < 5; i++) g_gemv_stamps[size_t(wave_id) * 8 + i] = t[i];
  }
};
#else
struct Stamps {
  __device__ __forceinline__ void mark(int) {}
  __device__ __forceinline__ void put(int, int) {}
};
#endif

// ---- wavefront reduction of kRows partial sums ---------------------------

template <int kCtrl>
__device__ __forceinline__ float dpp(float v) {
  return __builtin_bit_cast(
      float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, v), kCtrl, 0xF, 0xF, false));
}

// One transposed butterfly level on lane bit `off`: lanes with the bit clear
// keep values [0, n/2), lanes with it set keep [n/2, n); each lane adds the
// partner's copy of the values it keeps.
template <int N>
__device__ __forceinline__ void tr_level(float (&v)[N], int n, int off, int lane) {
  const bool up = (lane & off) != 0;
#pragma unroll
  for (int i = 0; i < N / 2; i++) {
    if (i < n / 2) {
      const float send = up ? v[i] : v[i + n / 2];
      const float keep = up ? v[i + n / 2] : v[i];
      v[i] = keep + __shfl_xor(send, off, 64);
    }
  }
}

// After reduce_rows<R>, lane l holds the wavefront total of row
// l >> (6 - log2 R) in v[0].  The xor masks used (32, 16, 15 = row mirror,
// 7 = half-row mirror, 2, 1) are linearly independent over GF(2), so every
// lane's partial is counted exactly once; masks after a transposed level
// never flip that level's bit.
template <int R>
__device__ __forceinline__ void reduce_rows(float (&v)[R], int lane) {
  static_assert(R == 1 || R == 2 || R == 4 || R == 8, "rows per tile");
  if constexpr (R >= 2) tr_level<R>(v, R, 32, lane);
  else v[0] += __shfl_xor(v[0], 32, 64);
  if constexpr (R >= 4) tr_level<R>(v, R / 2, 16, lane);
  else v[0] += __shfl_xor(v[0], 16, 64);
  if constexpr (R >= 8) {
    // bit 3 through the row mirror (lane ^ 15): its bits 0..2 flips are
    // harmless because the later levels reduce over those bits anyway.
    const bool up = (lane & 8) != 0;
    const float send = up ? v[0] : v[1];
    const float keep = up ? v[1] : v[0];
    v[0] = keep + dpp<0x140>(send);
  } else {
    v[0] += dpp<0x140>(v[0]);  // row mirror
  }
  v[0] += dpp<0x141>(v[0]);  // half-row mirror (lane ^ 7)
  v[0] += dpp<0x4E>(v[0]);   // quad_perm [2,3,0,1]
  v[0] += dpp<0xB1>(v[0]);   // quad_perm [1,0,3,2]
}

constexpr int kMaxMats = SWAMP_MULTI_MAX;

struct MatSet {
  const uint8_t *w[kMaxMats];
  float *y[kMaxMats];
  int rows[kMaxMats];
  int tile_end[kMaxMats];  // cumulative tile counts
  int n;
  int wpc;   // waves per CU the persistent grid aims for (launch_items)
  bool sets;  // several row sets per workgroup share x (rows of <= 128 items)
};

struct TileRef {
  const uint8_t *w;
  float *y;
  int row0, nrows;
};

template <int kRows, bool kMulti>
__device__ __forceinline__ TileRef tile_ref(const MatSet &ms, int tile) {
  if constexpr (!kMulti) return TileRef{ms.w[0], ms.y[0], tile * kRows, ms.rows[0]};
  int m = 0;
  while (m + 1 < ms.n && tile >= ms.tile_end[m]) m++;
  const int first = m ? ms.tile_end[m - 1] : 0;
  return TileRef{ms.w[m], ms.y[m], (tile - first) * kRows, ms.rows[m]};
}

// One buffer descriptor per tile (base = the tile's first row); row r of
// the tile is the scalar offset r * row_bytes (rows past the matrix end
// are clamped to its last row, so every load stays in bounds).
template <int DT, int kPPT, int kRows>
__device__ __forceinline__ void issue_tile(Raw<DT> (&raw)[kRows][kPPT], const TileRef &t,
                                           size_t row_bytes, const int (&item)[kPPT],
                                           const uint32_t (&off)[kPPT]) {
  const uint32_t rb = uint32_t(row_bytes);
  const __amdgpu_buffer_rsrc_t rs =
      swamp::make_rsrc(t.w + size_t(t.row0) * row_bytes, rb * kRows);
#pragma unroll
  for (int r = 0; r < kRows; r++) {
    const int rr = min(t.row0 + r, t.nrows - 1) - t.row0;
#pragma unroll
    for (int j = 0; j < kPPT; j++)
      swamp::load_raw_buf<DT>(raw[r][j], rs, off[j], uint32_t(rr) * rb, item[j]);
  }
}

// Row of the tile whose output lane tid stores (kWaves == 1: the first
// lane of each group of 64 / kRows; else lanes tid < kRows), clamped into
// the matrix; the accumulating form loads y there together with the tile's
// weights, so the read-modify-write never waits on memory in the loop.
template <int kRows, int kWaves>
__device__ __forceinline__ int store_row(const TileRef &t, int tid) {
  const int rr = kWaves == 1 ? (tid & 63) / (64 / kRows) : min(tid, kRows - 1);
  return min(t.row0 + rr, t.nrows - 1);
}

// live: the tile is this set's (false: a stand-in tile a row set works
// through so that every wave of the workgroup meets the same barriers; its
// result is not stored).
template <int DT, int kPPT, int kRows, int kWaves, bool kAcc, class XF>
__device__ __forceinline__ void consume_tile(const Raw<DT> (&raw)[kRows][kPPT],
                                             const XF (&xf)[kPPT], const TileRef &t,
                                             const int (&item)[kPPT],
                                             float (*red)[kRows], int tid, uint32_t m,
                                             float out_scale, float y_old, bool live) {
  const int lane = tid & 63, wave = tid >> 6;
  float acc[kRows];
#pragma unroll
  for (int r = 0; r < kRows; r++) {
    acc[r] = 0.f;
#pragma unroll
    for (int j = 0; j < kPPT; j++) acc[r] += item_dot<DT>(raw[r][j], xf[j], item[j], m);
  }
  reduce_rows<kRows>(acc, lane);
  constexpr int kGroup = 64 / kRows;  // lanes holding one row's total
  const int rr = lane / kGroup;
  if constexpr (kWaves == 1) {
    if (live && lane % kGroup == 0 && t.row0 + rr < t.nrows) {
      const float v = acc[0] * out_scale;
      t.y[t.row0 + rr] = kAcc ? y_old + v : v;
    }
  } else {
    if (lane % kGroup == 0) red[wave][rr] = acc[0];
    __syncthreads();
    if (live && tid < kRows && t.row0 + tid < t.nrows) {
      float v = 0.f;
#pragma unroll
      for (int w = 0; w < kWaves; w++) v += red[w][tid];
      v *= out_scale;
      t.y[t.row0 + tid] = kAcc ? y_old + v : v;
    }
  }
}

// ---- x staged through LDS -------------------------------------------------
// With one item per lane, a vector (x, or the prologue operand) reaches the
// workgroup by direct-to-LDS DMA in 1 KB pieces (64 lanes x 16 B, adjacent
// chunks) instead of 16 per-lane loads at a 256-byte lane stride (64 cache
// lines per instruction through the texture path); each lane then reads
// its item's 16 chunks from LDS.  Chunk c of item i sits at 16-byte unit
// 16 i + (c ^ (i & 15)), so eight consecutive lanes reading chunk c hit
// eight different bank groups.

// Byte offset in the vector of chunk c (4 floats) of item `item`, in the
// order load_x fills xv[c].
template <int DT>
__device__ __forceinline__ uint32_t x_chunk_bytes(int item, int c) {
  if constexpr (DT == SWAMP_Q6_K)
    return 4u * (uint32_t(item >> 2) * 256u + 128u * uint32_t((item >> 1) & 1) +
                 16u * uint32_t(item & 1) + 32u * uint32_t(c >> 2) + 4u * uint32_t(c & 3));
  else
    return uint32_t(item) * 256u + 16u * uint32_t(c);
}

// Buffer loads issue_tile makes per item and row (one instruction each).
__host__ __device__ constexpr int loads_per_item(int dt) {
  return dt == SWAMP_Q8_0 ? 5 : dt == SWAMP_Q6_K ? 8 : 3;
}

// DMA of a vector of ipr items into lds: instruction k fills units
// [64k, 64k + 64); wave w issues k = w, w + kWaves, ...  Lanes past the
// vector (the last instruction's tail) read outside the buffer range and
// deposit zeros.
// One 16-byte-per-lane DMA into lds (lane L writes lds + 16 L).  Kept out
// of the templates: the host compilation pass rejects the LDS address-space
// cast inside a template instantiation.
__device__ __forceinline__ void dma16(__amdgpu_buffer_rsrc_t r, uint8_t *lds, uint32_t voff) {
  __builtin_amdgcn_raw_ptr_buffer_load_lds(r, (__attribute__((address_space(3))) void *)lds, 16,
                                           voff, 0, 0, 0);
}

template <int DT, int kWaves>
__device__ __forceinline__ void stage_vec(uint8_t *lds, const float *v, int ipr, int wave,
                                          int lane) {
  const __amdgpu_buffer_rsrc_t r = swamp::make_rsrc(v, uint32_t(ipr) * 256u);
  const int nk = (ipr + 3) >> 2;
  for (int k = wave; k < nk; k += kWaves) {
    const int u = 64 * k + lane;
    const int it = u >> 4;
    const int c = (u & 15) ^ (it & 15);
    dma16(r, lds + 1024 * k, x_chunk_bytes<DT>(it, c));
  }
}

__device__ __forceinline__ void read_vec(float4 (&xv)[16], const uint8_t *lds, int item) {
#pragma unroll
  for (int c = 0; c < 16; c++)
    xv[c] = *reinterpret_cast<const float4 *>(lds + 16 * (16 * item + (c ^ (item & 15))));
}

using swamp::silu_mul;

// One row set = 64 * kWaves lanes; lane j owns items j, j + T, ... (kPPT
// items per lane), covering one row of ipr items.  A workgroup is kSets row
// sets that stage x once and then walk their own tiles: set s of workgroup
// b takes tiles kSets b + s, + kSets gridDim.x, ... of kRows rows each.
// One-wave sets need no barrier per tile and leave when their tiles end.
// Sets of several waves sum a row through LDS behind a workgroup barrier,
// so every set makes as many trips as set 0: a set past the last tile works
// through a stand-in tile and stores nothing.  Since every workgroup holds
// all of x, a prologue that needs the whole vector (the RMSNorm sum of
// squares) is computed by each set for itself.
// kX32: fp32 x (XFrag32, the reference's arithmetic); else x rounded to
// fp16 (XFrag, dot2 arithmetic).
template <int DT, int kPPT, int kRows, int kWaves, bool kMulti, int kPro, bool kX32,
          int kSets = 1>
__global__ void __launch_bounds__(64 * kWaves * kSets)
    gemv_kernel(MatSet ms, const float *__restrict__ x, Pro pro, int ipr, size_t row_bytes,
                int n_tiles) {
  using XF = std::conditional_t<kX32, XFrag32<DT>, XFrag<DT>>;
  constexpr int T = 64 * kWaves;
  constexpr bool kUniform = kSets > 1 && kWaves > 1;  // trips set by set 0
  __shared__ float red[2][kSets][kWaves][kRows];
  const int tid = kSets == 1 ? int(threadIdx.x) : int(threadIdx.x) % T;
  const int set = kSets == 1 ? 0 : __builtin_amdgcn_readfirstlane(int(threadIdx.x) / T);
  Stamps st;
  st.mark(0);

  int item[kPPT];
  bool valid[kPPT];
#pragma unroll
  for (int j = 0; j < kPPT; j++) {
    const int it = tid + j * T;
    valid[j] = it < ipr;
    item[j] = valid[j] ? it : ipr - 1;  // in-bounds stand-in; its x is zero
  }
  uint32_t off[kPPT];
#pragma unroll
  for (int j = 0; j < kPPT; j++) off[j] = swamp::item_offset<DT>(item[j]);

  // A set past the last tile still takes part in staging x (its loads
  // re-read the last tile); a one-wave set then leaves after the staging
  // barrier, a set of several waves keeps pace with set 0 on stand-in tiles.
  const int stride = int(gridDim.x) * kSets;
  int tile = int(blockIdx.x) * kSets + set;
  const bool idle = tile >= n_tiles;
  if (kSets == 1 && idle) return;
  bool live_a = !idle;
  if (idle) tile = n_tiles - 1;
  const uint32_t m = f16_magic();

  // x (and the prologue operand) first, then the first tile's weight loads,
  // then the x conversion (which waits for the x loads only).
  constexpr bool kAcc = kPro == kProSwiGLUAcc;
  [[maybe_unused]] float ya = 0.f, yb = 0.f;  // y of the store rows (kAcc)
  if constexpr (kAcc) {
    const TileRef t0 = tile_ref<kRows, kMulti>(ms, tile);
    ya = t0.y[store_row<kRows, kWaves>(t0, tid)];
  }
  constexpr bool kStage = kPPT == 1;  // x through LDS (item count <= 64 kWaves)
  constexpr bool kTwo = kStage && kPro != kProNone && kWaves <= 4;  // both vectors at once
  constexpr int kRegion = kWaves * 16384;
  __shared__ __align__(16) uint8_t xlds[kStage ? (kTwo ? 2 : 1) * kRegion : 16];
  // waves of the workgroup and this wave's index among them (x staging)
  constexpr int kWgWaves = kWaves * kSets;
  const int wave = __builtin_amdgcn_readfirstlane(int(threadIdx.x >> 6)), lane = tid & 63;
  float4 x4[kPPT][16];
  [[maybe_unused]] float4 v4[kPPT][16];  // prologue operand (w_norm or up)
  if constexpr (kStage) {
    stage_vec<DT, kWgWaves>(xlds, x, ipr, wave, lane);
    if constexpr (kTwo) stage_vec<DT, kWgWaves>(xlds + kRegion, pro.x2, ipr, wave, lane);
  } else {
#pragma unroll
    for (int j = 0; j < kPPT; j++) load_x<DT>(x4[j], x, item[j]);
    if constexpr (kPro != kProNone) {
#pragma unroll
      for (int j = 0; j < kPPT; j++) load_x<DT>(v4[j], pro.x2, item[j]);
    }
  }
  Raw<DT> ra[kRows][kPPT], rb[kRows][kPPT];
  TileRef ta = tile_ref<kRows, kMulti>(ms, tile);
  issue_tile<DT, kPPT, kRows>(ra, ta, row_bytes, item, off);
  // keep every load of the tile ahead of the arithmetic (the scheduler would
  // otherwise sink them into registers freed by the current tile)
  __builtin_amdgcn_sched_barrier(0);
  if constexpr (kStage) {
    // the memory counter is in order: waiting until only the tile's loads
    // are outstanding means every DMA of this wave has landed; the barrier
    // covers the other waves' pieces.  Exactly these loads follow the DMA
    // (the accumulating form's first y load is issued before the staging).
    constexpr int kAfter = kRows * loads_per_item(DT);
    asm volatile("s_waitcnt vmcnt(%0)\n\ts_barrier" ::"n"(kAfter) : "memory");
    st.mark(1);
    read_vec(x4[0], xlds, item[0]);
    if constexpr (kTwo) {
      read_vec(v4[0], xlds + kRegion, item[0]);
    } else if constexpr (kPro != kProNone) {
      // one region: the operand follows once every wave has read x
      asm volatile("s_waitcnt lgkmcnt(0)\n\ts_barrier" ::: "memory");
      stage_vec<DT, kWgWaves>(xlds, pro.x2, ipr, wave, lane);
      asm volatile("s_waitcnt vmcnt(0)\n\ts_barrier" ::: "memory");
      read_vec(v4[0], xlds, item[0]);
    }
  }
  if constexpr (kPro == kProSwiGLU || kPro == kProSwiGLUAcc) {
#pragma unroll
    for (int j = 0; j < kPPT; j++)
#pragma unroll
      for (int i = 0; i < 16; i++) {
        float4 &g = x4[j][i];
        const float4 u = v4[j][i];
        g = make_float4(silu_mul(g.x, u.x), silu_mul(g.y, u.y), silu_mul(g.z, u.z),
                        silu_mul(g.w, u.w));
      }
  }
  // RMSNorm: W ((x * inv_rms) * w) = inv_rms * (W (x * w)), so the fragment
  // is built from x * w at once, the sum of squares finishes behind it and
  // inv_rms scales each output as it is stored.
  [[maybe_unused]] float ss = 0.f;
  if constexpr (kPro == kProRmsNorm) {
#pragma unroll
    for (int j = 0; j < kPPT; j++)
#pragma unroll
      for (int i = 0; i < 16; i++) {
        float4 &g = x4[j][i];
        const float q = g.x * g.x + g.y * g.y + g.z * g.z + g.w * g.w;
        ss += valid[j] ? q : 0.f;
        const float4 w = v4[j][i];
        g = make_float4(g.x * w.x, g.y * w.y, g.z * w.z, g.w * w.w);
      }
  }
  if (kSets > 1 && !kUniform && idle) return;  // after the workgroup's last barrier
  XF xf[kPPT];
#pragma unroll
  for (int j = 0; j < kPPT; j++) build_xfrag<DT>(xf[j], x4[j], valid[j]);
  float out_scale = 1.0f;
  if constexpr (kPro == kProRmsNorm) {
    __shared__ float ssq[kSets][kWaves];
    ss = swamp::wave_sum(ss);
    if (kWaves > 1) {
      if ((tid & 63) == 0) ssq[set][tid >> 6] = ss;
      __syncthreads();
      ss = 0.f;
#pragma unroll
      for (int w = 0; w < kWaves; w++) ss += ssq[set][w];
    }
    out_scale = __builtin_amdgcn_rsqf(ss / float(ipr * 64) + pro.eps);
  }

  // Two tiles per trip so both register buffers have static names.  The
  // next tile's loads are issued unconditionally (past the last tile they
  // re-read the current one, already in cache), so every path through the
  // loop has the same number of loads in flight and the hardware wait
  // counts stay tight.
  // Trip by trip, set s works on tile base + s, base advancing by stride
  // (base is set 0's tile).  A one-wave set stops when its own next tile is
  // past the end; with kUniform every set stops when set 0's is, a set
  // whose tile is past the end working through a stand-in (its current
  // tile, clamped) that it does not store.
  st.mark(2);
  int base = int(blockIdx.x) * kSets;
  bool first_trip = true;
  for (;;) {
    const int cur = tile;  // the tile ra holds (clamped)
    int nb = base + stride;
    bool live_b = nb + set < n_tiles;
    const TileRef tb = tile_ref<kRows, kMulti>(ms, live_b ? nb + set : cur);
    issue_tile<DT, kPPT, kRows>(rb, tb, row_bytes, item, off);
    if constexpr (kAcc) yb = tb.y[store_row<kRows, kWaves>(tb, tid)];
    __builtin_amdgcn_sched_barrier(0);
    consume_tile<DT, kPPT, kRows, kWaves, kAcc>(ra, xf, ta, item, red[0][set], tid, m, out_scale,
                                                ya, live_a);
    if (first_trip) st.mark(3);
    first_trip = false;
    if (kUniform ? nb >= n_tiles : !live_b) break;
    base = __builtin_amdgcn_readfirstlane(nb);  // keep it scalar (no VGPR round trip)
    tile = live_b ? base + set : cur;           // the tile rb holds
    nb = base + stride;
    live_a = nb + set < n_tiles;
    ta = tile_ref<kRows, kMulti>(ms, live_a ? nb + set : tile);
    issue_tile<DT, kPPT, kRows>(ra, ta, row_bytes, item, off);
    if constexpr (kAcc) ya = ta.y[store_row<kRows, kWaves>(ta, tid)];
    __builtin_amdgcn_sched_barrier(0);
    consume_tile<DT, kPPT, kRows, kWaves, kAcc>(rb, xf, tb, item, red[1][set], tid, m, out_scale,
                                                yb, live_b);
    if (kUniform ? nb >= n_tiles : !live_a) break;
    base = __builtin_amdgcn_readfirstlane(nb);  // keep it scalar (no VGPR round trip)
    tile = live_a ? base + set : tile;          // the tile ra holds
  }
  st.mark(4);
  st.put(int(blockIdx.x) * kWaves * kSets + int(threadIdx.x >> 6), int(threadIdx.x & 63));
}


// Rows the item kernel takes: whole items, at most 1024 per row (n_cols <=
// 65536: at most two items per lane, whose two register buffers fit without
// spills), and for Q6_K an even number of blocks (4-byte aligned rows).
bool item_path_ok(uint32_t dt, int n_cols) {
  if (n_cols / 64 > 1024) return false;
  if (dt == SWAMP_Q4_K) return true;
  if (dt == SWAMP_Q6_K) return n_cols % 512 == 0;
  return n_cols % 64 == 0;
}

// Launch shape: waves per CU the persistent grid aims for, and rows per
// tile (SWAMP_GEMV_WAVES_PER_CU / SWAMP_GEMV_ROWS override them).
struct Tuning {
  int waves_per_cu = 0;  // 0: chosen per shape
  int rows = 0;          // 0: chosen per shape
  bool sets = true;      // row sets sharing x (SWAMP_GEMV_SETS=0 turns them off)
  Tuning() {
    if (const char *s = std::getenv("SWAMP_GEMV_WAVES_PER_CU")) {
      int v = std::atoi(s);
      if (v >= 1 && v <= 64) waves_per_cu = v;
    }
    if (const char *s = std::getenv("SWAMP_GEMV_SETS")) sets = std::atoi(s) != 0;
    if (const char *s = std::getenv("SWAMP_GEMV_ROWS")) {
      int v = std::atoi(s);
      if (v == 1 || v == 2 || v == 4) rows = v;
    }
  }
};
const Tuning &tuning() {
  static Tuning t;
  return t;
}

template <int DT, int kPPT, int kRows, int kWaves, int kPro, bool kX32, int kSets = 1>
int launch_items(const MatSet &ms, const float *x, const Pro &pro, int n_cols, hipStream_t s) {
  const int ipr = n_cols / 64;
  if (ipr > kPPT * 64 * kWaves) return SWAMP_ESHAPE;
  const int n_tiles = ms.tile_end[ms.n - 1];
  const int cus = swamp::device_info().num_cus;
  int grid = cus * std::max(1, ms.wpc / (kWaves * kSets));
  const int need = (n_tiles + kSets - 1) / kSets;  // workgroups with a tile for set 0
  if (grid > need) grid = need;
  if (grid < 1) return SWAMP_OK;
  constexpr int kThreads = 64 * kWaves * kSets;
  if (ms.n == 1)
    gemv_kernel<DT, kPPT, kRows, kWaves, false, kPro, kX32, kSets>
        <<<grid, kThreads, 0, s>>>(ms, x, pro, ipr, swamp::row_bytes(DT, n_cols), n_tiles);
  else if constexpr (kPro == kProSwiGLU || kPro == kProSwiGLUAcc)
    return SWAMP_EINVAL;  // single matrix only
  else
    gemv_kernel<DT, kPPT, kRows, kWaves, true, kPro, kX32, kSets>
        <<<grid, kThreads, 0, s>>>(ms, x, pro, ipr, swamp::row_bytes(DT, n_cols), n_tiles);
  return hipGetLastError() == hipSuccess ? SWAMP_OK : SWAMP_ELAUNCH;
}

int build_matset(MatSet &ms, int n, const void *const *ws, float *const *ys, const int *rows,
                 int tile_rows) {
  ms.n = n;
  ms.wpc = 4;
  ms.sets = tuning().sets;
  int acc = 0;
  for (int i = 0; i < n; i++) {
    ms.w[i] = static_cast<const uint8_t *>(ws[i]);
    ms.y[i] = ys[i];
    ms.rows[i] = rows[i];
    acc += (rows[i] + tile_rows - 1) / tile_rows;
    ms.tile_end[i] = acc;
  }
  return acc;
}

// Waves per workgroup for a row of ipr items (matches launch_rows).
int waves_for(int ipr) { return ipr <= 64 ? 1 : ipr <= 128 ? 2 : ipr <= 256 ? 4 : 8; }

// Waves per CU of the persistent grid: 4 (one per SIMD); 8 for the fp32-x
// kernels on the larger matrices, whose heavier arithmetic per weight needs
// a second wave per SIMD to keep loads in flight: Q4_0 / Q4_K from 6144
// rows (with 2-row tiles at most two tiles per wave, all in flight from the
// start), Q6_K from 16384 rows, and all three, and Q8_0, for rows of more
// than 4096 weights.  Measured (bench.py --sweep, us, 4 -> 8 waves per
// CU): Q6_K lm_head 128256 x 4096 84.0 -> 75.4, gate_up 21.6 -> 20.3, down
// 17.0 -> 16.1, qkv 7.6 -> 7.7; Q8_0 lm_head 128256 x 8192 199.4 -> 181.9,
// 128256 x 4096 90.1 -> 92.1.
int waves_per_cu_for(uint32_t dt, int n_cols, int total_rows, bool x32) {
  if (tuning().waves_per_cu) return tuning().waves_per_cu;
  if (!x32) return 4;
  if (n_cols > 4096) return 8;
  // Q4_0 / Q4_K rows of at most 4096 weights, at least 16 four-row tiles
  // per wave at 4 waves per CU (the 8B lm_head, 128256 rows): 4 waves with
  // 4-row tiles stream faster than 8 with 2-row tiles (bench.py decode step,
  // SWAMP_GEMV_WAVES_PER_CU=4 SWAMP_GEMV_ROWS=4 against the default: Q4_0
  // lm_head 49.9 against 51.5 us); shorter matrices lose (gate_up 13.8
  // against 12.6 us), their waves get too few tiles
  if ((dt == SWAMP_Q4_0 || dt == SWAMP_Q4_K) &&
      long(total_rows) >= 64L * 4 * swamp::device_info().num_cus)
    return 4;
  if ((dt == SWAMP_Q4_0 || dt == SWAMP_Q4_K) && total_rows >= 6144) return 8;
  if (dt == SWAMP_Q6_K && total_rows >= 16384) return 8;
  return 4;
}

// Rows per tile: 4 when every wave of the grid gets at least 8 tiles, else
// 2 when it gets at least 1 (8B qkv at 8 waves per CU: 5.15 us against
// 5.6 us with 1-row tiles), else 1; always 1 when a lane holds
// several items (rows of more than 512 items); Q6_K capped lower; at most
// 2 with 8 waves per CU.  Longer tile runs per wave
// hide the first tile's latency and the x prologue; shorter tiles keep
// small matrices spread over the whole chip.
int tile_rows_for(uint32_t dt, int n_cols, int total_rows, bool x32) {
  const int ipr = n_cols / 64;
  int cap = ipr <= 512 ? 4 : 1;
  // Q6_K items carry twice the decode work: 2-row tiles measure fastest, and
  // 1-row tiles for 8-wave workgroups (n_cols > 16384)
  if (dt == SWAMP_Q6_K) cap = ipr <= 256 ? 2 : 1;
  // Q8_0 with fp32 x: the register budget allows 2 rows
  if (dt == SWAMP_Q8_0 && x32) cap = std::min(cap, 2);
  if (tuning().rows) return std::min(tuning().rows, cap);
  const int wpc = waves_per_cu_for(dt, n_cols, total_rows, x32);
  if (wpc >= 8) cap = std::min(cap, 2);
  const int cus = swamp::device_info().num_cus;
  const long slots = long(cus) * std::max(1, wpc / waves_for(ipr));
  int r = 1;
  if (long(total_rows) / 4 >= 8 * slots) r = 4;
  else if (long(total_rows) / 2 >= slots) r = 2;
  return std::min(r, cap);
}

template <int DT, int kRows, int kPro, bool kX32>
int launch_rows(const MatSet &ms, const float *x, const Pro &pro, int n_cols, hipStream_t s) {
  const int ipr = n_cols / 64;
  // tiles of at most 2 rows (tile_rows_for): Q6_K always, Q8_0 with fp32 x
  // (4 double-buffered rows of 68-byte items beside 64 fp32 x values do not
  // fit 256 VGPRs)
  if constexpr (kRows > 2 && (DT == SWAMP_Q6_K || (kX32 && DT == SWAMP_Q8_0))) {
    return SWAMP_ESHAPE;
  } else {
    // row sets sharing x: 4 sets of one wave, 2 of two waves (when the grid
    // aims for 8 waves per CU).  Measured per matrix, fp32 x (us, sets /
    // none): 8B Q4_0 qkv 5.97 / 6.31, o_proj 4.55 / 5.08, gate_up 13.79 /
    // 15.14, lm_head 52.2 / 56.5; 70B Q4_K qkv 12.4 / 13.3, gate_up 52.1 /
    // 58.2.  Two sets of four waves (K = 14336) measured slower (down 10.1
    // / 9.9): their barrier per tile ties the two sets together.
    if (ipr <= 64) {
      if (ms.sets) return launch_items<DT, 1, kRows, 1, kPro, kX32, 4>(ms, x, pro, n_cols, s);
      return launch_items<DT, 1, kRows, 1, kPro, kX32>(ms, x, pro, n_cols, s);
    }
    if (ipr <= 128) {
      if (ms.sets && ms.wpc >= 8) return launch_items<DT, 1, kRows, 2, kPro, kX32, 2>(ms, x, pro, n_cols, s);
      return launch_items<DT, 1, kRows, 2, kPro, kX32>(ms, x, pro, n_cols, s);
    }
    if (ipr <= 256) return launch_items<DT, 1, kRows, 4, kPro, kX32>(ms, x, pro, n_cols, s);
    if (ipr <= 512) return launch_items<DT, 1, kRows, 8, kPro, kX32>(ms, x, pro, n_cols, s);
    // the fused prologues keep one item per lane (n_cols <= 32768)
    if constexpr (kPro != kProNone) return SWAMP_ESHAPE;
    // With two items per lane the tiles are single rows (tile_rows_for caps
    // them) so both register buffers fit without spills; longer rows take
    // the generic kernels (item_path_ok).
    else if constexpr (kRows > 1) return SWAMP_ESHAPE;
    else if (ipr <= 1024) return launch_items<DT, 2, 1, 8, kPro, kX32>(ms, x, pro, n_cols, s);
    return SWAMP_ESHAPE;
  }
}

template <int DT, int kPro, bool kX32>
int launch_dt(const MatSet &ms, const float *x, const Pro &pro, int n_cols, int tile_rows,
              hipStream_t s) {
  switch (tile_rows) {
  case 4: return launch_rows<DT, 4, kPro, kX32>(ms, x, pro, n_cols, s);
  case 2: return launch_rows<DT, 2, kPro, kX32>(ms, x, pro, n_cols, s);
  default: return launch_rows<DT, 1, kPro, kX32>(ms, x, pro, n_cols, s);
  }
}

template <int kPro, bool kX32>
int dispatch(uint32_t dt, const MatSet &ms, const float *x, const Pro &pro, int n_cols,
             int tile_rows, hipStream_t s) {
  switch (dt) {
  case SWAMP_Q4_0: return launch_dt<SWAMP_Q4_0, kPro, kX32>(ms, x, pro, n_cols, tile_rows, s);
  case SWAMP_Q8_0: return launch_dt<SWAMP_Q8_0, kPro, kX32>(ms, x, pro, n_cols, tile_rows, s);
  case SWAMP_Q4_K: return launch_dt<SWAMP_Q4_K, kPro, kX32>(ms, x, pro, n_cols, tile_rows, s);
  case SWAMP_Q6_K: return launch_dt<SWAMP_Q6_K, kPro, kX32>(ms, x, pro, n_cols, tile_rows, s);
  default: return SWAMP_EDTYPE;
  }
}

// Several matrices sharing x: matrices of one dtype share a launch (and
// the x prologue); a different dtype starts another launch on the same
// stream.  Shapes the item kernel does not take go to swamp_launch_gemv
// one matrix at a time (no prologue: the fused forms reject them first).
template <int kPro, bool kX32>
int launch_multi(int n_mats, const uint32_t *dtypes, const void *const *d_ws,
                 const int *row_counts, const float *d_x, const Pro &pro, float *const *d_ys,
                 int n_cols, hipStream_t s) {
  bool done[kMaxMats] = {};
  for (int i = 0; i < n_mats; i++) {
    if (done[i]) continue;
    const uint32_t dt = dtypes[i];
    if (!item_path_ok(dt, n_cols)) {
      if (kPro != kProNone) return SWAMP_ESHAPE;
      for (int j = i; j < n_mats; j++)
        if (!done[j] && dtypes[j] == dt) {
          int rc = swamp_launch_gemv(dt, d_ws[j], d_x, d_ys[j], row_counts[j], n_cols, s);
          if (rc) return rc;
          done[j] = true;
        }
      continue;
    }
    const void *ws[kMaxMats];
    float *ys[kMaxMats];
    int rows[kMaxMats];
    int n = 0, total = 0;
    for (int j = i; j < n_mats; j++)
      if (!done[j] && dtypes[j] == dt && row_counts[j] > 0) {
        ws[n] = d_ws[j];
        ys[n] = d_ys[j];
        rows[n] = row_counts[j];
        total += row_counts[j];
        n++;
        done[j] = true;
      } else if (dtypes[j] == dt) {
        done[j] = true;
      }
    if (n == 0) continue;
    MatSet ms;
    const int tr = tile_rows_for(dt, n_cols, total, kX32);
    build_matset(ms, n, ws, ys, rows, tr);
    ms.wpc = waves_per_cu_for(dt, n_cols, total, kX32);
    int rc = dispatch<kPro, kX32>(dt, ms, d_x, pro, n_cols, tr, s);
    if (rc) return rc;
  }
  return SWAMP_OK;
}


}  // namespace
