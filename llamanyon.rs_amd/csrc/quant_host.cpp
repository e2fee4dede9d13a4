// quant_host.cpp -- host-side quantizers and seeded synthetic data.
//
// The reference has dequantizers only (swamp-gguf/src/quant/*.rs), so the
// quantizers here are this library's own.  Their output layouts are the
// ones the reference reads back (see swamp_quant.h).  Q4_0 and Q8_0 use the
// block formulas ggml publishes for its reference quantizers; Q4_K uses a
// simple max/min per-sub-block scheme packed with the scale/min bit layout
// of the reference's test packer (swamp-kernels/src/fused_gemv_q4k.rs:708-724);
// Q6_K uses a signed per-sub-block scheme like ggml's (quant_block_q6_k).
#include "swamp_quant.h"

#include <algorithm>
#include <cmath>
#include <cstring>
#include <thread>
#include <vector>

namespace {

uint32_t f32_bits(float f) {
  uint32_t b;
  std::memcpy(&b, &f, 4);
  return b;
}

float bits_f32(uint32_t b) {
  float f;
  std::memcpy(&f, &b, 4);
  return f;
}

float f16_to_f32(uint16_t h) {
  uint32_t sign = uint32_t(h & 0x8000u) << 16;
  uint32_t exp = (h >> 10) & 0x1Fu, man = h & 0x3FFu;
  if (exp == 0) {
    if (man == 0) return bits_f32(sign);
    int e = -1;
    do {
      e++;
      man <<= 1;
    } while (!(man & 0x400u));
    return bits_f32(sign | (uint32_t(127 - 15 - e) << 23) | ((man & 0x3FFu) << 13));
  }
  if (exp == 31) return bits_f32(sign | 0x7F800000u | (man ? 0x400000u | (man << 13) : 0u));
  return bits_f32(sign | ((exp + 112u) << 23) | (man << 13));
}

uint64_t splitmix64(uint64_t &s) {
  uint64_t z = (s += 0x9E3779B97F4A7C15ull);
  z = (z ^ (z >> 30)) * 0xBF58476D1CE4E5B9ull;
  z = (z ^ (z >> 27)) * 0x94D049BB133111EBull;
  return z ^ (z >> 31);
}

void normal_row(uint64_t seed, float sigma, size_t row, float *dst, size_t cols) {
  uint64_t s = seed ^ ((uint64_t(row) + 1) * 0xD1B54A32D192ED03ull);
  const double two_pi = 6.283185307179586476925286766559;
  for (size_t c = 0; c < cols; c += 2) {
    double u1 = double((splitmix64(s) >> 11) + 1) * (1.0 / 9007199254740992.0);
    double u2 = double(splitmix64(s) >> 11) * (1.0 / 9007199254740992.0);
    double r = std::sqrt(-2.0 * std::log(u1));
    double th = two_pi * u2;
    dst[c] = float(double(sigma) * r * std::cos(th));
    if (c + 1 < cols) dst[c + 1] = float(double(sigma) * r * std::sin(th));
  }
}

void put_f16(uint8_t *p, float v) {
  uint16_t h = swamp_f32_to_f16(v);
  p[0] = uint8_t(h & 0xFF);
  p[1] = uint8_t(h >> 8);
}

// Q4_0: ggml quantize_row_q4_0_ref block formula, interleaved packing.
void quant_block_q4_0(const float *x, uint8_t *out) {
  float amax = 0.0f, vmax = 0.0f;
  for (int j = 0; j < 32; j++) {
    float a = std::fabs(x[j]);
    if (amax < a) {
      amax = a;
      vmax = x[j];
    }
  }
  const float d = vmax / -8.0f;
  const float id = d != 0.0f ? 1.0f / d : 0.0f;
  put_f16(out, d);
  uint8_t q[32];
  for (int j = 0; j < 32; j++) {
    float v = x[j] * id + 8.5f;
    int t = int(int8_t(v));  // truncation toward zero, as the C cast does
    q[j] = uint8_t(std::min(15, std::max(0, t)));
  }
  for (int j = 0; j < 16; j++) out[2 + j] = uint8_t(q[2 * j] | (q[2 * j + 1] << 4));
}

// Q8_0: ggml quantize_row_q8_0_ref block formula.
void quant_block_q8_0(const float *x, uint8_t *out) {
  float amax = 0.0f;
  for (int j = 0; j < 32; j++) amax = std::max(amax, std::fabs(x[j]));
  const float d = amax / 127.0f;
  const float id = d != 0.0f ? 1.0f / d : 0.0f;
  put_f16(out, d);
  for (int j = 0; j < 32; j++) {
    float v = std::round(x[j] * id);
    v = std::min(127.0f, std::max(-127.0f, v));
    out[2 + j] = uint8_t(int8_t(v));
  }
}

// Q4_K: per sub-block j, step s_j = (max - min0) / 15 and offset
// m_j = -min0 with min0 = min(0, min x).  d = max s_j / 63 and
// dmin = max m_j / 63 are rounded to f16, the 6-bit codes are rounded up so
// the coded range covers the data, and q = round((x + dmin*mn) / (d*sc)).
void quant_block_q4_k(const float *x, uint8_t *out) {
  float s[8], m[8];
  float smax = 0.0f, mmax = 0.0f;
  for (int j = 0; j < 8; j++) {
    const float *v = x + 32 * j;
    float lo = 0.0f, hi = v[0];
    for (int i = 0; i < 32; i++) {
      lo = std::min(lo, v[i]);
      hi = std::max(hi, v[i]);
    }
    hi = std::max(hi, lo);
    s[j] = (hi - lo) / 15.0f;
    m[j] = -lo;
    smax = std::max(smax, s[j]);
    mmax = std::max(mmax, m[j]);
  }
  const uint16_t dh = swamp_f32_to_f16(smax / 63.0f);
  const uint16_t mh = swamp_f32_to_f16(mmax / 63.0f);
  const float d = f16_to_f32(dh), dmin = f16_to_f32(mh);
  uint8_t sc[8], mn[8];
  for (int j = 0; j < 8; j++) {
    float a = d > 0.0f ? std::ceil(s[j] / d) : 0.0f;
    float b = dmin > 0.0f ? std::ceil(m[j] / dmin) : 0.0f;
    sc[j] = uint8_t(std::min(63.0f, std::max(0.0f, a)));
    mn[j] = uint8_t(std::min(63.0f, std::max(0.0f, b)));
  }
  out[0] = uint8_t(dh & 0xFF);
  out[1] = uint8_t(dh >> 8);
  out[2] = uint8_t(mh & 0xFF);
  out[3] = uint8_t(mh >> 8);
  for (int j = 0; j < 4; j++) {
    out[4 + j] = uint8_t((sc[j] & 0x3F) | ((sc[4 + j] >> 4) << 6));
    out[8 + j] = uint8_t((mn[j] & 0x3F) | ((mn[4 + j] >> 4) << 6));
    out[12 + j] = uint8_t((sc[4 + j] & 0x0F) | ((mn[4 + j] & 0x0F) << 4));
  }
  uint8_t q[8][32];
  for (int j = 0; j < 8; j++) {
    const float step = d * float(sc[j]);
    const float off = dmin * float(mn[j]);
    for (int i = 0; i < 32; i++) {
      float t = step > 0.0f ? std::round((x[32 * j + i] + off) / step) : 0.0f;
      q[j][i] = uint8_t(std::min(15.0f, std::max(0.0f, t)));
    }
  }
  for (int p = 0; p < 4; p++)
    for (int i = 0; i < 32; i++)
      out[16 + 32 * p + i] = uint8_t(q[2 * p][i] | (q[2 * p + 1][i] << 4));
}

// Q6_K: each 16-weight sub-block j gets the signed step s_j = v_j / -32
// (v_j its value of largest magnitude, so v_j codes as q = 0); the block
// scale d = s_m / -128 for the s_m of largest magnitude is rounded to f16,
// sc_j = s_j / d rounded away from zero and clamped to [-128, 127]
// (negative codes occur), and
// q = round(x / (d * sc_j)) + 32 clamped to [0, 63].  Packed as the
// reference's dequantizer reads it (swamp-gguf/src/quant/q6_k.rs:36-44):
// output 128h + 32k + l (k = 0..3, l < 32) keeps its low 4 bits in byte
// 64h + l + 32(k & 1) of ql (low nibble for k < 2, high for k >= 2) and
// its bits 4-5 in bits 2k..2k+1 of qh[32h + l].
void quant_block_q6_k(const float *x, uint8_t *out) {
  float s[16];
  float smax = 0.0f;
  for (int j = 0; j < 16; j++) {
    float amax = 0.0f, vmax = 0.0f;
    for (int i = 0; i < 16; i++) {
      const float a = std::fabs(x[16 * j + i]);
      if (amax < a) {
        amax = a;
        vmax = x[16 * j + i];
      }
    }
    s[j] = vmax / -32.0f;
    if (std::fabs(s[j]) > std::fabs(smax)) smax = s[j];
  }
  std::memset(out, 0, 210);
  const uint16_t dh = swamp_f32_to_f16(smax / -128.0f);
  const float d = f16_to_f32(dh);
  if (d == 0.0f) return;  // all-zero block: every code 0 decodes to 0
  int8_t sc[16];
  for (int j = 0; j < 16; j++) {
    // magnitude rounded up, so the step covers the sub-block's range
    const float r = std::copysign(std::ceil(std::fabs(s[j] / d)), s[j] / d);
    sc[j] = int8_t(std::min(127.0f, std::max(-128.0f, r)));
  }
  uint8_t q[256];
  for (int e = 0; e < 256; e++) {
    const float step = d * float(sc[e / 16]);
    const float t = step != 0.0f ? std::round(x[e] / step) : 0.0f;
    q[e] = uint8_t(std::min(31.0f, std::max(-32.0f, t)) + 32.0f);
  }
  for (int h = 0; h < 2; h++)
    for (int l = 0; l < 32; l++) {
      const uint8_t *v = q + 128 * h + l;  // v[32k] is output 128h + 32k + l
      out[64 * h + l] = uint8_t((v[0] & 0xF) | ((v[64] & 0xF) << 4));
      out[64 * h + l + 32] = uint8_t((v[32] & 0xF) | ((v[96] & 0xF) << 4));
      out[128 + 32 * h + l] =
          uint8_t((v[0] >> 4) | ((v[32] >> 4) << 2) | ((v[64] >> 4) << 4) | ((v[96] >> 4) << 6));
    }
  for (int j = 0; j < 16; j++) out[192 + j] = uint8_t(sc[j]);
  out[208] = uint8_t(dh & 0xFF);
  out[209] = uint8_t(dh >> 8);
}

struct Fmt {
  size_t block, bytes;
  void (*fn)(const float *, uint8_t *);
};

bool fmt_for(uint32_t dtype, Fmt &f) {
  switch (dtype) {
  case 2: f = {32, 18, quant_block_q4_0}; return true;
  case 8: f = {32, 34, quant_block_q8_0}; return true;
  case 12: f = {256, 144, quant_block_q4_k}; return true;
  case 14: f = {256, 210, quant_block_q6_k}; return true;
  default: return false;
  }
}

int resolve_threads(int n_threads) {
  if (n_threads > 0) return n_threads;
  unsigned h = std::thread::hardware_concurrency();
  return int(std::min(16u, std::max(1u, h)));
}

template <class F>
void parallel_rows(size_t rows, int n_threads, F &&body) {
  int nt = resolve_threads(n_threads);
  if (size_t(nt) > rows) nt = int(rows ? rows : 1);
  size_t rpt = (rows + nt - 1) / nt;
  std::vector<std::thread> pool;
  for (int t = 1; t < nt; t++) {
    size_t rs = std::min(rows, t * rpt), re = std::min(rows, rs + rpt);
    pool.emplace_back([&body, rs, re] { body(rs, re); });
  }
  body(0, std::min(rows, rpt));
  for (auto &th : pool) th.join();
}

}  // namespace

extern "C" {

uint16_t swamp_f32_to_f16(float f) {
  const uint32_t x = f32_bits(f);
  const uint16_t sign = uint16_t((x >> 16) & 0x8000u);
  const uint32_t exp = (x >> 23) & 0xFFu;
  const uint32_t man = x & 0x7FFFFFu;
  if (exp == 0xFF) return uint16_t(sign | 0x7C00u | (man ? 0x200u | (man >> 13) : 0u));
  const int e = int(exp) - 112;  // f16 biased exponent
  if (e >= 31) return uint16_t(sign | 0x7C00u);
  if (e >= 1) {
    uint32_t h = (uint32_t(e) << 10) | (man >> 13);
    const uint32_t rem = man & 0x1FFFu;
    if (rem > 0x1000u || (rem == 0x1000u && (h & 1u))) h++;  // may carry into inf
    return uint16_t(sign | h);
  }
  // f16 subnormal range: value = full * 2^(exp-150); code = value * 2^24
  if (exp == 0) return sign;  // f32 zero/subnormal -> +-0
  const uint64_t full = 0x800000u | man;
  const int shift = 126 - int(exp);  // >= 14
  if (shift > 24) return sign;
  uint64_t h = full >> shift;
  const uint64_t rem = full & ((uint64_t(1) << shift) - 1);
  const uint64_t half = uint64_t(1) << (shift - 1);
  if (rem > half || (rem == half && (h & 1u))) h++;
  return uint16_t(sign | uint16_t(h));
}

uint16_t swamp_f32_to_bf16(float f) {
  uint32_t x = f32_bits(f);
  if ((x & 0x7F800000u) == 0x7F800000u && (x & 0x7FFFFFu)) return uint16_t((x >> 16) | 0x40u);
  x += 0x7FFFu + ((x >> 16) & 1u);
  return uint16_t(x >> 16);
}

void swamp_f32_to_bf16_array(const float *src, uint16_t *dst, size_t n) {
  for (size_t i = 0; i < n; i++) dst[i] = swamp_f32_to_bf16(src[i]);
}

int swamp_fill_normal(uint64_t seed, float sigma, float *dst, size_t rows,
                      size_t cols, int n_threads) {
  if (!dst && rows * cols) return -1;
  parallel_rows(rows, n_threads, [&](size_t rs, size_t re) {
    for (size_t r = rs; r < re; r++) normal_row(seed, sigma, r, dst + r * cols, cols);
  });
  return 0;
}

int swamp_quantize(uint32_t dtype, const float *src, uint8_t *dst, size_t rows,
                   size_t cols, int n_threads) {
  Fmt f;
  if (!fmt_for(dtype, f)) return -2;
  if (cols % f.block != 0) return -1;
  if ((!src || !dst) && rows * cols) return -1;
  const size_t nb = cols / f.block, row_bytes = nb * f.bytes;
  parallel_rows(rows, n_threads, [&](size_t rs, size_t re) {
    for (size_t r = rs; r < re; r++)
      for (size_t b = 0; b < nb; b++)
        f.fn(src + r * cols + b * f.block, dst + r * row_bytes + b * f.bytes);
  });
  return 0;
}

int swamp_synth_quantized(uint32_t dtype, uint64_t seed, float sigma,
                          uint8_t *dst, size_t rows, size_t cols,
                          int n_threads) {
  Fmt f;
  if (!fmt_for(dtype, f)) return -2;
  if (cols % f.block != 0) return -1;
  if (!dst && rows * cols) return -1;
  const size_t nb = cols / f.block, row_bytes = nb * f.bytes;
  parallel_rows(rows, n_threads, [&](size_t rs, size_t re) {
    std::vector<float> buf(cols);
    for (size_t r = rs; r < re; r++) {
      normal_row(seed, sigma, r, buf.data(), cols);
      for (size_t b = 0; b < nb; b++)
        f.fn(buf.data() + b * f.block, dst + r * row_bytes + b * f.bytes);
    }
  });
  return 0;
}

}  // extern "C"
