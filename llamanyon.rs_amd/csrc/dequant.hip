// dequant.hip -- bit-exact device dequantization (quant::dequantize).
//
// This translation unit is compiled with -ffp-contract=off: the Q4_K value
// (d*sc)*q - dmin*m must round the product and the difference separately,
// as the reference's Rust does (swamp-gguf/src/quant/q4_k.rs:296-316).
// Q4_0 and Q8_0 are one exact-integer-times-scale product each; Q6_K is
// (d*sc)*q, two roundings in that order (q6_k.rs:41-44).
//
// Work split: one thread writes 8 consecutive outputs, so consecutive
// threads store consecutive 32-byte runs (coalesced); the few block bytes
// each thread needs are re-read by its neighbours from L1.
#include "swamp_common.hpp"

namespace {

using swamp::f16_bits_to_f32_exact;

__device__ __forceinline__ uint32_t ld_u16(const uint8_t *p) {
  return *reinterpret_cast<const uint16_t *>(p);
}

typedef __bf16 bf16x8_t __attribute__((ext_vector_type(8)));

template <bool kVec>
__device__ __forceinline__ void store8(float *dst, size_t base, size_t n,
                                       const float (&v)[8]) {
  if (kVec && base + 8 <= n) {
    float4 *p = reinterpret_cast<float4 *>(dst + base);
    p[0] = make_float4(v[0], v[1], v[2], v[3]);
    p[1] = make_float4(v[4], v[5], v[6], v[7]);
  } else {
#pragma unroll
    for (int j = 0; j < 8; j++)
      if (base + j < n) dst[base + j] = v[j];
  }
}

// bf16 output (the dequant-once GEMM route): each exact fp32 value rounded
// to nearest even, as the fused GEMM rounds its in-register weights.
template <bool kVec>
__device__ __forceinline__ void store8(__bf16 *dst, size_t base, size_t n,
                                       const float (&v)[8]) {
  if (kVec && base + 8 <= n) {
    bf16x8_t b;
#pragma unroll
    for (int j = 0; j < 8; j++) b[j] = __bf16(v[j]);
    *reinterpret_cast<bf16x8_t *>(dst + base) = b;
  } else {
#pragma unroll
    for (int j = 0; j < 8; j++)
      if (base + j < n) dst[base + j] = __bf16(v[j]);
  }
}

// q4_0::dequant (q4_0.rs:22-37): element i of a block is byte i/2, low
// nibble for even i; value (nib - 8) * f16(d).
template <bool kVec, class T = float>
__global__ void dequant_q4_0_kernel(const uint8_t *__restrict__ raw,
                                    T *__restrict__ dst, size_t n) {
  const size_t g = size_t(blockIdx.x) * blockDim.x + threadIdx.x;
  const size_t base = g * 8;
  if (base >= n) return;
  const size_t b = g >> 2;
  const int t = int(g & 3);
  const uint8_t *blk = raw + b * 18;
  const float d = f16_bits_to_f32_exact(ld_u16(blk));
  const uint32_t nib = ld_u16(blk + 2 + 4 * t) | (ld_u16(blk + 4 + 4 * t) << 16);
  float v[8];
#pragma unroll
  for (int j = 0; j < 8; j++) {
    const int q = int((nib >> (4 * j)) & 0xFu);  // byte j/2, low nibble first
    v[j] = float(q - 8) * d;
  }
  store8<kVec>(dst, base, n, v);
}

// q8_0::dequant scalar arm (q8_0.rs:127-139): value int8 * f16(d).
template <bool kVec, class T = float>
__global__ void dequant_q8_0_kernel(const uint8_t *__restrict__ raw,
                                    T *__restrict__ dst, size_t n) {
  const size_t g = size_t(blockIdx.x) * blockDim.x + threadIdx.x;
  const size_t base = g * 8;
  if (base >= n) return;
  const size_t b = g >> 2;
  const int t = int(g & 3);
  const uint8_t *blk = raw + b * 34;
  const float d = f16_bits_to_f32_exact(ld_u16(blk));
  const uint8_t *qs = blk + 2 + 8 * t;
  const uint32_t lo = ld_u16(qs) | (ld_u16(qs + 2) << 16);
  const uint32_t hi = ld_u16(qs + 4) | (ld_u16(qs + 6) << 16);
  float v[8];
#pragma unroll
  for (int j = 0; j < 4; j++) {
    v[j] = float(int8_t(uint8_t(lo >> (8 * j)))) * d;
    v[4 + j] = float(int8_t(uint8_t(hi >> (8 * j)))) * d;
  }
  store8<kVec>(dst, base, n, v);
}

// q4_k::dequant_scalar (q4_k.rs:278-321) with unpack_scales (:37-53),
// layout A: pair p = sub-blocks (2p, 2p+1) use qs[32p..32p+32], low nibble
// for the even sub-block, high nibble for the odd one.
template <bool kVec, class T = float>
__global__ void dequant_q4_k_kernel(const uint8_t *__restrict__ raw,
                                    T *__restrict__ dst, size_t n) {
  const size_t g = size_t(blockIdx.x) * blockDim.x + threadIdx.x;
  const size_t base = g * 8;
  if (base >= n) return;
  const size_t b = g >> 5;
  const int e0 = int(g & 31) * 8;  // first element within the super-block
  const int sb = e0 >> 5;          // sub-block 0..7
  const int i0 = e0 & 31;
  const int pair = sb >> 1;
  const bool high = sb & 1;
  const uint8_t *blk = raw + b * 144;
  const uint4 hdr = *reinterpret_cast<const uint4 *>(blk);
  const float d = f16_bits_to_f32_exact(hdr.x & 0xFFFFu);
  const float dmin = f16_bits_to_f32_exact(hdr.x >> 16);
  // 12 scale bytes: sc[0..3] = hdr.y, sc[4..7] = hdr.z, sc[8..11] = hdr.w
  const uint32_t s03 = hdr.y, s47 = hdr.z, s811 = hdr.w;
  uint32_t scale, mn;
  if (sb < 4) {
    scale = (s03 >> (8 * sb)) & 63u;
    mn = (s47 >> (8 * sb)) & 63u;
  } else {
    const int j = sb - 4;
    const uint32_t b8 = (s811 >> (8 * j)) & 0xFFu;        // sc[j+8]
    const uint32_t bj = (s03 >> (8 * j)) & 0xFFu;         // sc[j]
    const uint32_t bj4 = (s47 >> (8 * j)) & 0xFFu;        // sc[j+4]
    scale = (b8 & 0xFu) | ((bj >> 6) << 4);
    mn = (b8 >> 4) | ((bj4 >> 6) << 4);
  }
  const float sv = d * float(scale & 0x3Fu);
  const float mv = dmin * float(mn & 0x3Fu);
  const uint2 q = *reinterpret_cast<const uint2 *>(blk + 16 + 32 * pair + i0);
  float v[8];
#pragma unroll
  for (int j = 0; j < 8; j++) {
    const uint32_t byte = ((j < 4 ? q.x : q.y) >> (8 * (j & 3))) & 0xFFu;
    const uint32_t qi = high ? (byte >> 4) : (byte & 0xFu);
    const float t = sv * float(qi);
    v[j] = t - mv;
  }
  store8<kVec>(dst, base, n, v);
}

// q6_k::dequant_scalar (q6_k.rs:22-56): the 8 outputs of a thread are
// elements l0..l0+7 (l0 % 8 == 0) of group j of half h, i.e. outputs
// 128h + 32j + l.  Their low 4 bits are nibbles of ql[64h + 32(j&1) + l]
// (low for j < 2, high for j >= 2), bits 4-5 are bits 2j..2j+1 of
// qh[32h + l], and all 8 share the int8 scale sc[8h + l0/16 + 2j]; value
// (d * sc) * (q - 32).  Blocks are 210 bytes, so only 2-byte loads.
template <bool kVec, class T = float>
__global__ void dequant_q6_k_kernel(const uint8_t *__restrict__ raw,
                                    T *__restrict__ dst, size_t n) {
  const size_t g = size_t(blockIdx.x) * blockDim.x + threadIdx.x;
  const size_t base = g * 8;
  if (base >= n) return;
  const size_t b = g >> 5;
  const int e0 = int(g & 31) * 8;  // first element within the block
  const int h = e0 >> 7, j = (e0 >> 5) & 3, l0 = e0 & 31;
  const uint8_t *blk = raw + b * 210;
  const uint8_t *ql = blk + 64 * h + 32 * (j & 1) + l0;
  const uint8_t *qh = blk + 128 + 32 * h + l0;
  const uint32_t l_lo = ld_u16(ql) | (ld_u16(ql + 2) << 16);
  const uint32_t l_hi = ld_u16(ql + 4) | (ld_u16(ql + 6) << 16);
  const uint32_t h_lo = ld_u16(qh) | (ld_u16(qh + 2) << 16);
  const uint32_t h_hi = ld_u16(qh + 4) | (ld_u16(qh + 6) << 16);
  const int sc = int(int8_t(blk[192 + 8 * h + (l0 >> 4) + 2 * j]));
  const float d = f16_bits_to_f32_exact(ld_u16(blk + 208));
  const float ds = d * float(sc);
  const int nsh = j >= 2 ? 4 : 0;
  float v[8];
#pragma unroll
  for (int k = 0; k < 8; k++) {
    const uint32_t lb = ((k < 4 ? l_lo : l_hi) >> (8 * (k & 3))) & 0xFFu;
    const uint32_t hb = ((k < 4 ? h_lo : h_hi) >> (8 * (k & 3))) & 0xFFu;
    const int q = int(((lb >> nsh) & 0xFu) | (((hb >> (2 * j)) & 3u) << 4)) - 32;
    v[k] = ds * float(q);
  }
  store8<kVec>(dst, base, n, v);
}

__global__ void dequant_f16_kernel(const uint16_t *__restrict__ raw,
                                   float *__restrict__ dst, size_t n) {
  const size_t i = size_t(blockIdx.x) * blockDim.x + threadIdx.x;
  if (i < n) dst[i] = f16_bits_to_f32_exact(raw[i]);
}

__global__ void dequant_bf16_kernel(const uint16_t *__restrict__ raw,
                                    float *__restrict__ dst, size_t n) {
  const size_t i = size_t(blockIdx.x) * blockDim.x + threadIdx.x;
  if (i < n) dst[i] = __uint_as_float(uint32_t(raw[i]) << 16);
}

}  // namespace

int swamp_launch_dequant(uint32_t dtype, const void *d_raw, float *d_dst,
                         size_t n, hipStream_t s) {
  if (n == 0) return SWAMP_OK;
  const int threads = 256;
  const bool vec = (reinterpret_cast<uintptr_t>(d_dst) & 15u) == 0;
  const uint8_t *raw = static_cast<const uint8_t *>(d_raw);
  const size_t groups = (n + 7) / 8;
  const dim3 grid8(unsigned((groups + threads - 1) / threads));
  const dim3 grid1(unsigned((n + threads - 1) / threads));
  switch (dtype) {
  case SWAMP_Q4_0:
    if (vec) dequant_q4_0_kernel<true><<<grid8, threads, 0, s>>>(raw, d_dst, n);
    else dequant_q4_0_kernel<false><<<grid8, threads, 0, s>>>(raw, d_dst, n);
    break;
  case SWAMP_Q8_0:
    if (vec) dequant_q8_0_kernel<true><<<grid8, threads, 0, s>>>(raw, d_dst, n);
    else dequant_q8_0_kernel<false><<<grid8, threads, 0, s>>>(raw, d_dst, n);
    break;
  case SWAMP_Q4_K:
    if (vec) dequant_q4_k_kernel<true><<<grid8, threads, 0, s>>>(raw, d_dst, n);
    else dequant_q4_k_kernel<false><<<grid8, threads, 0, s>>>(raw, d_dst, n);
    break;
  case SWAMP_Q6_K:
    if (vec) dequant_q6_k_kernel<true><<<grid8, threads, 0, s>>>(raw, d_dst, n);
    else dequant_q6_k_kernel<false><<<grid8, threads, 0, s>>>(raw, d_dst, n);
    break;
  case SWAMP_F16:
    dequant_f16_kernel<<<grid1, threads, 0, s>>>(static_cast<const uint16_t *>(d_raw), d_dst, n);
    break;
  case SWAMP_BF16:
    dequant_bf16_kernel<<<grid1, threads, 0, s>>>(static_cast<const uint16_t *>(d_raw), d_dst, n);
    break;
  case SWAMP_F32:
    if (hipMemcpyAsync(d_dst, d_raw, n * 4, hipMemcpyDeviceToDevice, s) != hipSuccess)
      return SWAMP_ELAUNCH;
    return SWAMP_OK;
  default:
    return SWAMP_EDTYPE;
  }
  return hipGetLastError() == hipSuccess ? SWAMP_OK : SWAMP_ELAUNCH;
}

namespace {

// ---- whole blocks to bf16 (the dequantize-once GEMM route) ------------------
// One thread per 32-weight block (Q4_0, Q8_0) or per 32-weight sub-block
// (Q4_K), dword loads realigned in registers, 16-byte stores: the values
// are those of the kernels above, rounded to nearest even.

__device__ __forceinline__ uint32_t ld_u32(const uint8_t *p) {
  return *reinterpret_cast<const uint32_t *>(p);
}

// The 32 bf16 values of thread t of a 256-thread workgroup go to LDS, then
// the workgroup's 16 KB are stored as 16-byte pieces of consecutive threads
// (each store instruction writes 1 KB of consecutive bytes).  dst is the
// workgroup's first output; `valid` pieces (of 1024) are stored.
// Thread t writes pieces p = 4t + c, the store reads p = 256c + t.  Piece p
// sits in 16-byte slot p ^ h(p), with h's two bits (p3 ^ p5, p4) chosen so
// that any 8 consecutive lanes (and any 16) of either access hit distinct
// slots modulo 8 (and 16): no bank conflicts with 32 or 64 four-byte banks.
__device__ __forceinline__ int stage_slot(int p) {
  return p ^ (((p >> 3) ^ (p >> 5)) & 1) ^ (p >> 3 & 2);
}

__device__ __forceinline__ void store32_bf16_wg(__bf16 *dst, const float (&v)[32], uint4 *lds,
                                                size_t valid) {
  const int t = threadIdx.x;
#pragma unroll
  for (int c = 0; c < 4; c++) {
    bf16x8_t b;
#pragma unroll
    for (int j = 0; j < 8; j++) b[j] = __bf16(v[8 * c + j]);
    lds[stage_slot(4 * t + c)] = __builtin_bit_cast(uint4, b);
  }
  __syncthreads();
  uint4 *out = reinterpret_cast<uint4 *>(dst);
#pragma unroll
  for (int c = 0; c < 4; c++) {
    const int piece = 256 * c + t;
    if (size_t(piece) < valid) out[piece] = lds[stage_slot(piece)];
  }
}

// Q4_0 / Q8_0: block b (18 or 34 bytes) starts at a 2-byte boundary; its
// bytes are read as dwords from the 4-byte boundary at or below it.
template <int DT>
__global__ void __launch_bounds__(256) blocks_to_bf16_kernel(const uint8_t *__restrict__ raw,
                                                             __bf16 *__restrict__ dst,
                                                             size_t n_blocks) {
  __shared__ uint4 lds[1024];
  const size_t b0 = size_t(blockIdx.x) * 256;
  const size_t b = b0 + threadIdx.x;
  const bool live = b < n_blocks;
  constexpr int kBytes = DT == SWAMP_Q4_0 ? 18 : 34;
  constexpr int kWords = DT == SWAMP_Q4_0 ? 5 : 9;  // covers kBytes + 2
  const size_t off = (live ? b : b0) * kBytes;  // a dead thread re-reads the first block
  const uint8_t *p = raw + (off & ~size_t(3));
  const uint32_t sh = uint32_t(off & 2);
  // the last dword holds 2 bytes past the block when it starts 4-byte
  // aligned: read only the 2 that belong to it (stay inside the buffer)
  uint32_t w[kWords + 1];
#pragma unroll
  for (int i = 0; i < kWords - 1; i++) w[i] = ld_u32(p + 4 * i);
  w[kWords - 1] = sh ? ld_u32(p + 4 * (kWords - 1)) : ld_u16(p + 4 * (kWords - 1));
  w[kWords] = 0;
  uint32_t a[kWords];  // the block's bytes from offset 0, dword-aligned
#pragma unroll
  for (int i = 0; i < kWords; i++) a[i] = __builtin_amdgcn_alignbyte(w[i + 1], w[i], sh);
  const float d = f16_bits_to_f32_exact(a[0] & 0xFFFFu);
  float v[32];
  if constexpr (DT == SWAMP_Q4_0) {
    // element i: byte 2 + i/2, low nibble for even i (q4_0.rs:30-35)
#pragma unroll
    for (int i = 0; i < 32; i++) {
      const int byte = 2 + i / 2;
      const uint32_t bv = (a[byte >> 2] >> (8 * (byte & 3))) & 0xFFu;
      const int q = int((i & 1) ? (bv >> 4) : (bv & 0xFu));
      v[i] = float(q - 8) * d;
    }
  } else {
#pragma unroll
    for (int i = 0; i < 32; i++) {
      const int byte = 2 + i;
      v[i] = float(int8_t(uint8_t(a[byte >> 2] >> (8 * (byte & 3))))) * d;
    }
  }
  store32_bf16_wg(dst + b0 * 32, v, lds, (n_blocks - b0) * 4);
}

// Q4_K: sub-block j of super-block b (144 bytes, 16-byte aligned).
__global__ void __launch_bounds__(256) q4k_to_bf16_kernel(const uint8_t *__restrict__ raw,
                                                          __bf16 *__restrict__ dst,
                                                          size_t n_sub) {
  __shared__ uint4 lds[1024];
  const size_t u0 = size_t(blockIdx.x) * 256;
  const size_t u = threadIdx.x + u0 < n_sub ? u0 + threadIdx.x : u0;  // dead: re-read the first
  const size_t b = u >> 3;
  const int sb = int(u & 7);
  const uint8_t *blk = raw + b * 144;
  const uint4 hdr = *reinterpret_cast<const uint4 *>(blk);
  const float d = f16_bits_to_f32_exact(hdr.x & 0xFFFFu);
  const float dmin = f16_bits_to_f32_exact(hdr.x >> 16);
  const uint32_t s03 = hdr.y, s47 = hdr.z, s811 = hdr.w;
  uint32_t scale, mn;
  if (sb < 4) {
    scale = (s03 >> (8 * sb)) & 63u;
    mn = (s47 >> (8 * sb)) & 63u;
  } else {
    const int j = sb - 4;
    const uint32_t b8 = (s811 >> (8 * j)) & 0xFFu;
    scale = (b8 & 0xFu) | ((((s03 >> (8 * j)) & 0xFFu) >> 6) << 4);
    mn = (b8 >> 4) | ((((s47 >> (8 * j)) & 0xFFu) >> 6) << 4);
  }
  const float sv = d * float(scale);
  const float mv = dmin * float(mn);
  const uint4 *q = reinterpret_cast<const uint4 *>(blk + 16 + 32 * (sb >> 1));
  const uint4 q0 = q[0], q1 = q[1];
  const uint32_t qw[8] = {q0.x, q0.y, q0.z, q0.w, q1.x, q1.y, q1.z, q1.w};
  const uint32_t nsh = (sb & 1) ? 4u : 0u;
  float v[32];
#pragma unroll
  for (int i = 0; i < 32; i++) {
    const uint32_t qi = (qw[i >> 2] >> (8 * (i & 3) + nsh)) & 0xFu;
    const float t = sv * float(qi);
    v[i] = t - mv;
  }
  store32_bf16_wg(dst + u0 * 32, v, lds, (n_sub - u0) * 4);
}

}  // namespace

int swamp_launch_dequant_bf16(uint32_t dtype, const void *d_raw, void *d_dst, size_t n,
                              hipStream_t s) {
  if (n == 0) return SWAMP_OK;
  if (n % 32 != 0 || (reinterpret_cast<uintptr_t>(d_dst) & 15u) != 0) return SWAMP_EINVAL;
  const uint8_t *raw = static_cast<const uint8_t *>(d_raw);
  __bf16 *dst = static_cast<__bf16 *>(d_dst);
  const size_t units = n / 32;
  const unsigned grid = unsigned((units + 255) / 256);
  switch (dtype) {
  case SWAMP_Q4_0:
    blocks_to_bf16_kernel<SWAMP_Q4_0><<<grid, 256, 0, s>>>(raw, dst, units);
    break;
  case SWAMP_Q8_0:
    blocks_to_bf16_kernel<SWAMP_Q8_0><<<grid, 256, 0, s>>>(raw, dst, units);
    break;
  case SWAMP_Q4_K:
    if (n % 256 != 0) return SWAMP_EINVAL;
    q4k_to_bf16_kernel<<<grid, 256, 0, s>>>(raw, dst, units);
    break;
  case SWAMP_Q6_K: {
    // 210-byte blocks, 2-byte aligned: the 8-outputs-per-thread kernel
    if (n % 256 != 0) return SWAMP_EINVAL;
    const dim3 grid8(unsigned(((n + 7) / 8 + 255) / 256));
    dequant_q6_k_kernel<true, __bf16><<<grid8, 256, 0, s>>>(raw, dst, n);
    break;
  }
  default:
    return SWAMP_EDTYPE;
  }
  return hipGetLastError() == hipSuccess ? SWAMP_OK : SWAMP_ELAUNCH;
}
