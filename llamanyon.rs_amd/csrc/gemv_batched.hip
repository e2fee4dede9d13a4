// gemv_batched.hip -- small-batch (2..16 tokens per pass) quantized GEMV on
// the matrix cores, for speculative verify and continuous batching.
//
// Replaces forward_linear_batch (swamp-engine/src/linear.rs:176-239) and
// fused_gemv_q4k_batched (swamp-kernels/src/fused_gemv_q4k.rs:527-554,
// scalar body :650-698).
//
// Still HBM-bound (at 16 tokens a Q4 weight byte feeds ~57 FLOP, the chip's
// balance is ~300), so the weights must stream exactly once per pass of 16
// tokens, with enough bytes in flight per CU to cover HBM latency.
//  * V_MFMA_F32_16X16X32_F16 with A = activations (16 tokens x 32 k) and
//    B = weights (32 k x 16 rows); C = 16 tokens x 16 rows, 4 VGPRs.
//  * Work unit = one 16-row tile x one K group (K_g columns).  Every wave
//    runs its own units from start to end: no reduction across waves, no
//    barrier in the main loop.  Lane (r = l%16, g = l/16) reads items
//    g, g+4, g+8, ... (64 weights each) of row r.
//  * The K group's activations sit in LDS for the whole kernel, rounded to
//    fp16 and stored in MFMA fragment order: one ds_read_b128 per lane and
//    step.  The k order inside each MFMA is permuted so that a lane's 8
//    weights come from ONE nibble dword (Q4) or two int8 dwords (Q8_0); the
//    activation fragments use the same permutation.
//  * Weight bytes stream through buffer loads (one descriptor per tile, the
//    chunk offset in an SGPR) into two register chunks: chunk s+1 is in
//    flight while chunk s is dequantized (nibble -> fp16 1024+q with one
//    and-or per pair, packed fp16 offset and scale) and multiplied.
//  * K groups of one tile combine through a workspace: each writes its
//    16x16 partial, bumps the tile's counter, and the group that arrives
//    last sums the partials in K order (deterministic: 0 + p0 + p1 + ...),
//    writes y and resets the counter for the next launch.  With one K group
//    y is written directly.
#include <cstdlib>
#include <mutex>
#include <vector>

#include "swamp_common.hpp"
#include "swamp_items.hpp"

namespace {

using swamp::Raw;
using swamp::shr16;

typedef _Float16 half8_t __attribute__((ext_vector_type(8)));
typedef _Float16 half2_t __attribute__((ext_vector_type(2)));
typedef float float4_t __attribute__((ext_vector_type(4)));

constexpr int kWaves = 8;       // waves per workgroup
constexpr int kThreads = kWaves * 64;
constexpr int kTok = 16;        // tokens per pass (MFMA M)
constexpr int kRowsTile = 16;   // rows per tile (MFMA N)
constexpr int kLdsBytes = 65536;  // activation bytes per workgroup: 2 workgroups per CU
constexpr uint32_t kF16Magic = 0x64006400u;  // fp16 pair (1024, 1024)
constexpr uint32_t kOob = 0x80000000u;       // buffer offset past any descriptor: reads 0

__device__ __forceinline__ half2_t as_h2(uint32_t u) { return __builtin_bit_cast(half2_t, u); }
__device__ __forceinline__ uint32_t as_u(half2_t h) { return __builtin_bit_cast(uint32_t, h); }

// Element (0..63 of the item) that operand slot i (0..7) of MFMA step st
// (0..7) multiplies.  Slot i = pair i/2, half i%2; pair p of a nibble dword
// holds the nibbles at bit offsets 4p and 4p+16 (P0..P3 = w>>0,4,8,12).
template <int DT>
__host__ __device__ constexpr int slot_elem(int st, int i) {
  const int p = i / 2, h = i % 2;
  if (DT == SWAMP_Q8_0) {
    // two int8 dwords per step; pair 0/1 of dword 0 -> bytes (0,2), (1,3)
    const int dw = p / 2, pb = p % 2;
    const int byte = pb + 2 * h;
    return 32 * (st / 4) + 8 * (st % 4) + 4 * dw + byte;
  }
  const int n = p + 4 * h;  // nibble index in the dword (bit 4n)
  if (DT == SWAMP_Q4_0) return 32 * (st / 4) + 8 * (st % 4) + n;  // interleaved: nibble n = element n
  // Q4_K quarter: dword st = bytes 4st..4st+3; low nibble -> sub-block A
  // element 4st + byte, high nibble -> sub-block B (item elements 32..63)
  return 32 * (n % 2) + 4 * st + n / 2;
}

// The 8 elements of step st, as loaded by the activation staging: Q4_0 and
// Q8_0 read elements base(st)+0..7; Q4_K reads 4st+0..3 and 32+4st+0..3.
// slot_local gives the index (0..7) of slot i in that 8-float group.
template <int DT>
__host__ __device__ constexpr int stage_elem(int st, int v) {
  if (DT == SWAMP_Q4_K) return (v < 4 ? 0 : 32) + 4 * st + (v & 3);
  return 32 * (st / 4) + 8 * (st % 4) + v;
}
template <int DT>
__host__ __device__ constexpr int slot_local(int i) {
  const int p = i / 2, h = i % 2;
  if (DT == SWAMP_Q8_0) return 4 * (p / 2) + (p % 2) + 2 * h;
  const int n = p + 4 * h;
  if (DT == SWAMP_Q4_0) return n;
  return 4 * (n % 2) + n / 2;
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

// 8 fp16 weights (4 packed dwords) of MFMA step st from one item (for
// Q4_K with its scales from q4k_item_scales).
template <int DT>
__device__ __forceinline__ half8_t weights_step(const Raw<DT> &r, int st, const Q4kScales &ks) {
  uint32_t o[4];
  if constexpr (DT == SWAMP_Q4_0) {
    const int blk = st / 4, t = st % 4;
    const uint32_t w = blk == 0 ? shr16(r.d[t + 1], r.d[t]) : r.d[5 + t];
    const uint32_t dbits = blk == 0 ? (r.d[0] & 0xFFFFu) : (r.d[4] >> 16);
    const half2_t d2 = as_h2(dbits | (dbits << 16));
    const half2_t off = {_Float16(-1032.0f), _Float16(-1032.0f)};
#pragma unroll
    for (int p = 0; p < 4; p++) {
      const uint32_t P = ((w >> (4 * p)) & 0x000F000Fu) | kF16Magic;
      o[p] = as_u((as_h2(P) + off) * d2);  // (q - 8) exact, then one rounding
    }
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
    o[0] = as_u((as_h2((u0 & 0x00FF00FFu) | kF16Magic) + off) * d2);
    o[1] = as_u((as_h2(((u0 >> 8) & 0x00FF00FFu) | kF16Magic) + off) * d2);
    o[2] = as_u((as_h2((u1 & 0x00FF00FFu) | kF16Magic) + off) * d2);
    o[3] = as_u((as_h2(((u1 >> 8) & 0x00FF00FFu) | kF16Magic) + off) * d2);
  } else {
    const half2_t off = {_Float16(-1024.0f), _Float16(-1024.0f)};
    const uint32_t w = r.q[st];
#pragma unroll
    for (int p = 0; p < 4; p++) {
      // pair p: nibbles at bits 4p and 4p+16; p even -> low nibbles (A)
      const uint32_t P = ((w >> (4 * p)) & 0x000F000Fu) | kF16Magic;
      const half2_t q = as_h2(P) + off;
      const bool a = (p % 2) == 0;
      o[p] = as_u(q * (a ? ks.sa : ks.sb) - (a ? ks.ma : ks.mb));
    }
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
  return DT == SWAMP_Q4_0 ? 144u : DT == SWAMP_Q8_0 ? 272u : 144u;
}
template <int DT>
__device__ __forceinline__ uint32_t lane_item_offset(int g) {
  if constexpr (DT == SWAMP_Q4_K) return 16u + 32u * uint32_t(g);  // quarter g after the header
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
  float *part;     // [n_tiles][kgroups][256] partial tiles (kgroups > 1)
  int *cnt;        // [n_tiles] arrival counters, zero between launches
  int n_tok, n_rows, n_cols;
  uint32_t row_bytes;
  int ipr;         // items (64 weights) per row
  int ipg;         // items per K group (multiple of 4 * kChunk)
  int kgroups;     // K groups per tile
  int wpg;         // workgroups per K group
  int accumulate;  // y += W x instead of y = W x
};

// y[4g+i][row0 + r16] for the tokens and rows that exist.
__device__ __forceinline__ void write_y(const Args &a, int row0, int r16, int g, float4_t v) {
  const int row = row0 + r16;
  if (row >= a.n_rows) return;
#pragma unroll
  for (int i = 0; i < 4; i++) {
    const int t = 4 * g + i;
    if (t < a.n_tok) {
      float *d = a.y + size_t(t) * a.n_rows + row;
      *d = a.accumulate ? *d + v[i] : v[i];
    }
  }
}

// Finish a unit: store (one K group) or partial + counter + fix-up.
//
// The partials and counters are shared across XCDs, whose L2 caches are not
// coherent with each other.  Agent-scope fences would write back and
// invalidate the whole L2 once per unit; instead every access to shared
// data is an agent-scope atomic (partials: relaxed stores and loads that
// are coherent device-wide), and the order "partials complete, then the
// counter moves" comes from waiting for the stores to complete before the
// counter's read-modify-write is issued.  The group whose increment returns
// kgroups-1 therefore finds every other partial already written.
__device__ __forceinline__ void finish_unit(const Args &a, int tile, int kg, int lane, float4_t acc) {
  const int r16 = lane & 15, g = lane >> 4;
  if (a.kgroups == 1) {
    write_y(a, tile * kRowsTile, r16, g, acc);
    return;
  }
  float *tile_part = a.part + size_t(tile) * a.kgroups * 256;
  float *mine = tile_part + kg * 256 + lane * 4;
#pragma unroll
  for (int i = 0; i < 4; i++)
    __hip_atomic_store(mine + i, acc[i], __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  __builtin_amdgcn_s_waitcnt(0);  // the partial stores have completed
  int old = 0;
  if (lane == 0)
    old = __hip_atomic_fetch_add(a.cnt + tile, 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  old = __builtin_amdgcn_readfirstlane(old);
  if (old != a.kgroups - 1) return;
  // sum in K order, 8 partials' loads in flight at a time
  float4_t s = {0.f, 0.f, 0.f, 0.f};
  for (int k0 = 0; k0 < a.kgroups; k0 += 8) {
    float v[8][4];
#pragma unroll
    for (int kk = 0; kk < 8; kk++) {
      const float *p = tile_part + (k0 + kk) * 256 + lane * 4;
#pragma unroll
      for (int i = 0; i < 4; i++)
        v[kk][i] = k0 + kk < a.kgroups
                       ? __hip_atomic_load(p + i, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT)
                       : 0.f;
    }
#pragma unroll
    for (int kk = 0; kk < 8; kk++)
#pragma unroll
      for (int i = 0; i < 4; i++) s[i] += v[kk][i];
  }
  write_y(a, tile * kRowsTile, r16, g, s);
  if (lane == 0) __hip_atomic_store(a.cnt + tile, 0, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

// Workgroup b serves K group b % kgroups; its waves take that group's tiles
// round-robin.  TOK = tokens held in LDS (4, 8 or 16; lanes of larger token
// index read a duplicate, their C rows are discarded).  kChunk = items per
// lane in one register chunk.
template <int DT, int TOK, int kChunk>
__global__ void __launch_bounds__(kThreads, 2) gemv_batched_kernel(Args a) {
  extern __shared__ half8_t xl[];  // [ipg][8 steps][TOK] fragments
  const int tid = threadIdx.x;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6), lane = tid & 63;
  const int r16 = lane & 15, g = lane >> 4;
  const int kg = blockIdx.x % a.kgroups;
  const int wig = (blockIdx.x / a.kgroups) * kWaves + wave;  // wave index in the group
  const int wstride = a.wpg * kWaves;
  const int n_tiles = (a.n_rows + kRowsTile - 1) / kRowsTile;
  const int my_tiles = wig < n_tiles ? (n_tiles - 1 - wig) / wstride + 1 : 0;
  const int cpu = a.ipg / (4 * kChunk);  // chunks per unit
  const int n_chunks = my_tiles * cpu;
  const uint32_t rb = a.row_bytes;
  // items of this lane in chunk c: item0 + g + 4*(c*kChunk + i); valid while
  // 4*(c*kChunk + i) < lim
  const int item0 = kg * a.ipg;
  const int lim = a.ipr - item0 - g;
  const uint32_t lane_off = uint32_t(r16) * rb + lane_item_offset<DT>(g) +
                            uint32_t(item0 / 4) * quad_bytes<DT>();
  const uint32_t chunk_bytes = kChunk * quad_bytes<DT>();

  auto issue = [&](Raw<DT> (&r)[kChunk], int s) {
    // chunk s of this wave: unit s / cpu, chunk s % cpu (s < n_chunks)
    const int u = s / cpu, c = s - u * cpu;
    const int row0 = (wig + u * wstride) * kRowsTile;
    const int nr = min(kRowsTile, a.n_rows - row0);
    const __amdgpu_buffer_rsrc_t rs = swamp::make_rsrc(a.w + size_t(row0) * rb, uint32_t(nr) * rb);
    const uint32_t soff = uint32_t(c) * chunk_bytes;
#pragma unroll
    for (int i = 0; i < kChunk; i++) {
      const bool ok = 4 * (c * kChunk + i) < lim;
      const uint32_t voff = ok ? lane_off + uint32_t(i) * quad_bytes<DT>() : kOob;
      load_item<DT>(r[i], rs, voff, soff, g);
    }
  };

  Raw<DT> ra[kChunk], rbuf[kChunk];
  if (n_chunks > 0) issue(ra, 0);
  __builtin_amdgcn_sched_barrier(0);

  // Stage this K group's activations: entry e = (item, step, token) with
  // the token fastest, so the LDS writes are linear.
  {
    const int n_ent = a.ipg * 8 * TOK;
    for (int e = tid; e < n_ent; e += kThreads) {
      const int tok = e % TOK, st = (e / TOK) & 7, il = e / (8 * TOK);
      const int item = item0 + il;
      half8_t h;
      if (tok < a.n_tok && item < a.ipr) {
        const float *xp = a.x + size_t(tok) * a.n_cols + size_t(item) * 64;
        const float4 v0 = *reinterpret_cast<const float4 *>(xp + stage_elem<DT>(st, 0));
        const float4 v1 = *reinterpret_cast<const float4 *>(xp + stage_elem<DT>(st, 4));
        const float v[8] = {v0.x, v0.y, v0.z, v0.w, v1.x, v1.y, v1.z, v1.w};
#pragma unroll
        for (int i = 0; i < 8; i++) h[i] = _Float16(v[slot_local<DT>(i)]);
      } else {
#pragma unroll
        for (int i = 0; i < 8; i++) h[i] = _Float16(0.0f);
      }
      xl[e] = h;
    }
  }
  __syncthreads();
  if (n_chunks == 0) return;

  // LDS fragment of this lane: item g + 4*(c*kChunk + i), step st, token r16
  const half8_t *xlane = xl + g * 8 * TOK + (r16 % TOK);
  float4_t acc = {0.f, 0.f, 0.f, 0.f};
  int u = 0, c = 0;

  auto consume = [&](const Raw<DT> (&r)[kChunk]) {
    const half8_t *xc = xlane + c * kChunk * 32 * TOK;
#pragma unroll
    for (int i = 0; i < kChunk; i++) {
      Q4kScales ks{};
      if constexpr (DT == SWAMP_Q4_K) ks = q4k_item_scales(r[i], g);
#pragma unroll
      for (int st = 0; st < 8; st++) {
        const half8_t xa = xc[i * 32 * TOK + st * TOK];
        const half8_t wb = weights_step<DT>(r[i], st, ks);
        acc = __builtin_amdgcn_mfma_f32_16x16x32_f16(xa, wb, acc, 0, 0, 0);
      }
    }
    if (++c == cpu) {
      finish_unit(a, wig + u * wstride, kg, lane, acc);
      acc = float4_t{0.f, 0.f, 0.f, 0.f};
      c = 0;
      u++;
    }
  };

  for (int s = 0;;) {
    issue(rbuf, s + 1 < n_chunks ? s + 1 : s);
    __builtin_amdgcn_sched_barrier(0);
    consume(ra);
    if (++s >= n_chunks) break;
    issue(ra, s + 1 < n_chunks ? s + 1 : s);
    __builtin_amdgcn_sched_barrier(0);
    consume(rbuf);
    if (++s >= n_chunks) break;
  }
}

__global__ void zero_i32_kernel(int *__restrict__ p, size_t n) {
  const size_t i = size_t(blockIdx.x) * blockDim.x + threadIdx.x;
  if (i < n) p[i] = 0;
}

// Per (device, stream) workspace for the K-group partials and counters.
// Grown on demand (after draining the stream that used the old one); the
// counters are zeroed once at allocation and by the kernels afterwards.
struct Workspace {
  int device;
  hipStream_t stream;
  float *part = nullptr;
  int *cnt = nullptr;
  size_t part_floats = 0, n_cnt = 0;
};
std::mutex g_ws_mu;
std::vector<Workspace> g_ws;

int get_workspace(hipStream_t s, size_t part_floats, size_t n_cnt, float **part, int **cnt) {
  const int dev = swamp::device_info().device;
  std::lock_guard<std::mutex> lock(g_ws_mu);
  Workspace *w = nullptr;
  for (auto &e : g_ws)
    if (e.device == dev && e.stream == s) w = &e;
  if (!w) {
    g_ws.push_back(Workspace{dev, s});
    w = &g_ws.back();
  }
  if (w->part_floats < part_floats || w->n_cnt < n_cnt) {
    if (w->part || w->cnt) {
      if (hipStreamSynchronize(s) != hipSuccess) return SWAMP_ELAUNCH;
      (void)hipFree(w->part);
      (void)hipFree(w->cnt);
      w->part = nullptr;
      w->cnt = nullptr;
      w->part_floats = w->n_cnt = 0;
    }
    const size_t pf = std::max(part_floats, size_t(1) << 16);
    const size_t nc = std::max(n_cnt, size_t(1) << 12);
    if (hipMalloc(reinterpret_cast<void **>(&w->part), pf * sizeof(float)) != hipSuccess)
      return SWAMP_ELAUNCH;
    if (hipMalloc(reinterpret_cast<void **>(&w->cnt), nc * sizeof(int)) != hipSuccess) {
      (void)hipFree(w->part);
      w->part = nullptr;
      return SWAMP_ELAUNCH;
    }
    zero_i32_kernel<<<unsigned((nc + 255) / 256), 256, 0, s>>>(w->cnt, nc);
    if (hipGetLastError() != hipSuccess) return SWAMP_ELAUNCH;
    w->part_floats = pf;
    w->n_cnt = nc;
  }
  *part = w->part;
  *cnt = w->cnt;
  return SWAMP_OK;
}

template <int DT>
constexpr int chunk_items() {
  return DT == SWAMP_Q4_0 ? 4 : 2;  // 144, 136 and 96 bytes per lane and chunk
}

template <int DT, int TOK>
int launch_pass_tok(Args a, hipStream_t s) {
  constexpr int kC = chunk_items<DT>();
  auto kern = gemv_batched_kernel<DT, TOK, kC>;
  static std::once_flag once;
  std::call_once(once, [&] {
    (void)hipFuncSetAttribute(reinterpret_cast<const void *>(kern),
                              hipFuncAttributeMaxDynamicSharedMemorySize, kLdsBytes);
  });
  const int cus = swamp::device_info().num_cus;
  const int n_tiles = (a.n_rows + kRowsTile - 1) / kRowsTile;
  const int q = 4 * kC;                        // item granule of a K group
  const int ipg_max = kLdsBytes / (TOK * 16 * 8) / q * q;  // LDS: 128*TOK bytes per item
  const int granules = (a.ipr + q - 1) / q;
  // Fewest K groups that fit LDS, then more until the units cover the
  // wave slots (2 workgroups x 8 waves per CU) or a group is one granule.
  const int slots = cus * 2 * kWaves;
  int kgroups = (a.ipr + ipg_max - 1) / ipg_max;
  while (kgroups < granules && size_t(n_tiles) * kgroups < size_t(slots) * 3 / 4) kgroups++;
  static const int forced = [] {  // tuning override: SWAMP_BATCHED_KGROUPS
    const char *e = std::getenv("SWAMP_BATCHED_KGROUPS");
    return e ? std::atoi(e) : 0;
  }();
  if (forced > 0) kgroups = std::max((a.ipr + ipg_max - 1) / ipg_max, std::min(forced, granules));
  int ipg = ((granules + kgroups - 1) / kgroups) * q;
  kgroups = (a.ipr + ipg - 1) / ipg;
  a.ipg = ipg;
  a.kgroups = kgroups;
  a.wpg = std::max(1, std::min((n_tiles + kWaves - 1) / kWaves, (2 * cus) / kgroups));
  if (kgroups > 1) {
    if (int rc = get_workspace(s, size_t(n_tiles) * kgroups * 256, size_t(n_tiles), &a.part, &a.cnt))
      return rc;
  }
  const size_t lds = size_t(ipg) * 8 * TOK * 16;
  kern<<<unsigned(kgroups * a.wpg), kThreads, lds, s>>>(a);
  return hipGetLastError() == hipSuccess ? SWAMP_OK : SWAMP_ELAUNCH;
}

template <int DT>
int launch_pass(Args a, hipStream_t s) {
  if (a.n_tok <= 4) return launch_pass_tok<DT, 4>(a, s);
  if (a.n_tok <= 8) return launch_pass_tok<DT, 8>(a, s);
  return launch_pass_tok<DT, 16>(a, s);
}

}  // namespace

int swamp_launch_gemv_batched(uint32_t dtype, const void *d_w, const float *d_x, float *d_y,
                              int n_tok, int n_rows, int n_cols, int accumulate,
                              hipStream_t s) {
  if (n_rows == 0 || n_tok == 0) return SWAMP_OK;
  Args a{};
  a.w = static_cast<const uint8_t *>(d_w);
  a.n_rows = n_rows;
  a.n_cols = n_cols;
  a.row_bytes = uint32_t(swamp::row_bytes(int(dtype), size_t(n_cols)));
  a.ipr = n_cols / 64;
  a.accumulate = accumulate;
  for (int t0 = 0; t0 < n_tok; t0 += kTok) {
    a.n_tok = std::min(kTok, n_tok - t0);
    a.x = d_x + size_t(t0) * n_cols;
    a.y = d_y + size_t(t0) * n_rows;
    int rc;
    switch (dtype) {
    case SWAMP_Q4_0: rc = launch_pass<SWAMP_Q4_0>(a, s); break;
    case SWAMP_Q8_0: rc = launch_pass<SWAMP_Q8_0>(a, s); break;
    case SWAMP_Q4_K: rc = launch_pass<SWAMP_Q4_K>(a, s); break;
    default: return SWAMP_EDTYPE;
    }
    if (rc) return rc;
  }
  return SWAMP_OK;
}
