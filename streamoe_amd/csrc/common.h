// common.h — device helpers shared by the libsmoe kernels (gfx950, wave64).
//
// Quantized-weight chunk model used by every decode kernel: one lane owns
// a "chunk" of 32 consecutive inputs of one weight row. A 4-bit chunk is
// 16 bytes (4 little-endian u32 words, 8 nibbles each, low nibble first);
// a packed 3-bit chunk is 12 bytes (four little-endian 24-bit packs, code
// i at bits 3i..3i+3; MLX's layout). Groups are multiples of 32, so a
// chunk never straddles a group: it has exactly one (scale, bias).
//
// The chunk dot product is computed group-factored:
//     sum_j (q_j * s + b) * x_j  =  s * sum_j q_j x_j  +  b * sum_j x_j
// which is one FMA per weight instead of two. The 3-bit and 4-bit paths
// share every floating-point operation after the codes are unpacked into
// exact small-integer floats, so a packed 3-bit row gives bit-identical
// results to the same codes stored as 4-bit nibbles.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include <atomic>

namespace smoe {

constexpr int kWave = 64;
constexpr int kChunk = 32;  // inputs per lane-chunk
constexpr int kMaxK = 16;
constexpr int kMaxSlots = kMaxK + 1;  // routed slots + shared expert

__device__ __forceinline__ float bf16f(uint16_t b) { return __uint_as_float((uint32_t)b << 16); }

template <int BITS>
struct Raw;
template <>
struct Raw<4> {
  uint32_t d[4];
};
template <>
struct Raw<3> {
  uint32_t d[3];
};

template <int BITS>
constexpr int chunk_bytes() {
  return BITS * kChunk / 8;
}

// Weights are streamed once per decode step: load them non-temporally so
// they do not evict the activations and routing data from L2
// (SMOE_NT_LOADS=0 builds plain loads, for cache experiments).
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
typedef float f32x4 __attribute__((ext_vector_type(4)));

#ifndef SMOE_NT_LOADS
#define SMOE_NT_LOADS 1
#endif
template <typename T>
__device__ __forceinline__ T ld_stream(const T* p) {
#if SMOE_NT_LOADS
  return __builtin_nontemporal_load(p);
#else
  return *p;
#endif
}

// Weight load: non-temporal (NT, the routed experts: streamed once per
// token) or temporal (data reused every token, e.g. router rows and the
// shared expert, which then stay resident in the memory-side cache).
template <bool NT, typename T>
__device__ __forceinline__ T ld_w(const T* p) {
  if constexpr (NT)
    return ld_stream(p);
  else
    return *p;
}

// A 32-bit lane offset made opaque at its use, so that the compiler adds it
// to a scalar base inside the load (scalar address + 32-bit vector offset)
// instead of widening it to 64 bits and adding with a vector instruction.
__device__ __forceinline__ uint32_t lane_off(uint32_t o) {
  asm volatile("" : "+v"(o));
  return o;
}

template <bool NT = true>
__device__ __forceinline__ Raw<4> load_raw4(const uint8_t* p) {
  const u32x4 v = ld_w<NT>(reinterpret_cast<const u32x4*>(p));
  Raw<4> r;
  r.d[0] = v.x;
  r.d[1] = v.y;
  r.d[2] = v.z;
  r.d[3] = v.w;
  return r;
}
template <bool NT = true>
__device__ __forceinline__ Raw<3> load_raw3(const uint8_t* p) {
  const uint32_t* q = reinterpret_cast<const uint32_t*>(p);
  Raw<3> r;
  r.d[0] = ld_w<NT>(q + 0);
  r.d[1] = ld_w<NT>(q + 1);
  r.d[2] = ld_w<NT>(q + 2);
  return r;
}
// LDS DMA (global_load_lds): each lane's 16 (or 4) bytes at g go to LDS at
// l + lane * 16 (or 4), without passing through registers. l must be the
// same for every lane of the wave; completion is counted by vmcnt.
#define SMOE_GPTR(p) ((const __attribute__((address_space(1))) void*)(p))
#define SMOE_LPTR(p) ((__attribute__((address_space(3))) void*)(p))
__device__ __forceinline__ void dma16(const void* g, void* l) {
  __builtin_amdgcn_global_load_lds(SMOE_GPTR(g), SMOE_LPTR(l), 16, 0, 0);
}
__device__ __forceinline__ void dma4(const void* g, void* l) {
  __builtin_amdgcn_global_load_lds(SMOE_GPTR(g), SMOE_LPTR(l), 4, 0, 0);
}

// Loads through an explicitly global pointer: a pointer that was itself
// loaded from memory (an expert blob from a route table) is generic to the
// compiler, which then emits flat loads, and a pending flat load makes every
// later wait a full vmcnt(0) (flat operations are not counted in order).
typedef const __attribute__((address_space(1))) uint8_t* gbytes;
__device__ __forceinline__ gbytes as_global(const void* p) { return (gbytes)p; }

template <bool NT, typename T>
__device__ __forceinline__ T gld(gbytes p) {
  typedef const __attribute__((address_space(1))) T* GT;
  if constexpr (NT)
    return __builtin_nontemporal_load((GT)p);
  else
    return *(GT)p;
}

template <int BITS, bool NT = true>
__device__ __forceinline__ Raw<BITS> load_raw_g(gbytes p) {
  Raw<BITS> r;
  if constexpr (BITS == 4) {
    const u32x4 v = gld<NT, u32x4>(p);
    r.d[0] = v.x;
    r.d[1] = v.y;
    r.d[2] = v.z;
    r.d[3] = v.w;
  } else {
    r.d[0] = gld<NT, uint32_t>(p);
    r.d[1] = gld<NT, uint32_t>(p + 4);
    r.d[2] = gld<NT, uint32_t>(p + 8);
  }
  return r;
}

template <int BITS, bool NT = true>
__device__ __forceinline__ Raw<BITS> load_raw(const uint8_t* p) {
  if constexpr (BITS == 4)
    return load_raw4<NT>(p);
  else
    return load_raw3<NT>(p);
}

// Codes of a chunk as exact floats, in input order j = 0..31.
__device__ __forceinline__ void unpack(const Raw<4>& r, float (&q)[kChunk]) {
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const uint32_t lo = r.d[i] & 0x0F0F0F0Fu;         // nibbles 0,2,4,6 in bytes 0..3
    const uint32_t hi = (r.d[i] >> 4) & 0x0F0F0F0Fu;  // nibbles 1,3,5,7
    q[8 * i + 0] = (float)(lo & 0xFFu);
    q[8 * i + 2] = (float)((lo >> 8) & 0xFFu);
    q[8 * i + 4] = (float)((lo >> 16) & 0xFFu);
    q[8 * i + 6] = (float)(lo >> 24);
    q[8 * i + 1] = (float)(hi & 0xFFu);
    q[8 * i + 3] = (float)((hi >> 8) & 0xFFu);
    q[8 * i + 5] = (float)((hi >> 16) & 0xFFu);
    q[8 * i + 7] = (float)(hi >> 24);
  }
}

__device__ __forceinline__ void unpack(const Raw<3>& r, float (&q)[kChunk]) {
#pragma unroll
  for (int j = 0; j < kChunk; ++j) {
    const int bit = 3 * j, w = bit >> 5, o = bit & 31;
    uint32_t v;
    if (o <= 29)
      v = __builtin_amdgcn_ubfe(r.d[w], o, 3);
    else
      v = __builtin_amdgcn_alignbit(r.d[w + 1], r.d[w], o) & 7u;
    q[j] = (float)v;
  }
}

// Integer code of input j of a chunk (used by the dequant probe).
__device__ __forceinline__ uint32_t code_at(const Raw<4>& r, int j) {
  return (r.d[j >> 3] >> ((j & 7) * 4)) & 0xFu;
}
__device__ __forceinline__ uint32_t code_at(const Raw<3>& r, int j) {
  const int bit = 3 * j, w = bit >> 5, o = bit & 31;
  if (o <= 29) return (r.d[w] >> o) & 7u;
  return ((r.d[w] >> o) | (r.d[w + 1] << (32 - o))) & 7u;
}

// sum_j q_j x_j over one chunk: four interleaved FMA chains.
__device__ __forceinline__ float qdot(const float (&q)[kChunk], const float (&x)[kChunk]) {
  float a0 = 0.f, a1 = 0.f, a2 = 0.f, a3 = 0.f;
#pragma unroll
  for (int j = 0; j < kChunk; j += 4) {
    a0 = __builtin_fmaf(q[j + 0], x[j + 0], a0);
    a1 = __builtin_fmaf(q[j + 1], x[j + 1], a1);
    a2 = __builtin_fmaf(q[j + 2], x[j + 2], a2);
    a3 = __builtin_fmaf(q[j + 3], x[j + 3], a3);
  }
  return (a0 + a1) + (a2 + a3);
}

__device__ __forceinline__ float xsum(const float (&x)[kChunk]) {
  float a0 = 0.f, a1 = 0.f, a2 = 0.f, a3 = 0.f;
#pragma unroll
  for (int j = 0; j < kChunk; j += 4) {
    a0 += x[j + 0];
    a1 += x[j + 1];
    a2 += x[j + 2];
    a3 += x[j + 3];
  }
  return (a0 + a1) + (a2 + a3);
}

// Contribution of one chunk: s * sum(q x) + b * sum(x).
template <int BITS>
__device__ __forceinline__ float chunk_dot(const Raw<BITS>& raw, const float (&x)[kChunk],
                                           float xs, float s, float b) {
  float q[kChunk];
  unpack(raw, q);
  return __builtin_fmaf(s, qdot(q, x), b * xs);
}

// DPP data movement within a wave (gfx9 encodings): row_shr:n = 0x110+n,
// row_bcast:15 = 0x142, row_bcast:31 = 0x143. Lanes whose source is out of
// range keep `identity`.
template <int CTRL, int ROW_MASK = 0xF>
__device__ __forceinline__ float dpp_f(float v, float identity) {
  return __int_as_float(__builtin_amdgcn_update_dpp(__float_as_int(identity), __float_as_int(v), CTRL,
                                                    ROW_MASK, 0xF, false));
}

// Sum over aligned groups of W lanes (W a power of two <= 64), on DPP and
// permlane swaps (a shuffle compiles to an LDS permute per step): quad
// lane ^ 1, quad lane ^ 2, the 8-lane half-row mirror, the 16-lane row
// mirror, then the row and half exchanges. Each step adds two partial sums
// over disjoint lane sets of equal size, and both partners form the same
// sum, so every lane of a group ends with the same value.
template <int W>
__device__ __forceinline__ float group_sum(float v) {
  static_assert(W >= 1 && W <= 64 && (W & (W - 1)) == 0, "W is a power of two <= 64");
  if constexpr (W >= 2) v += dpp_f<0xB1>(v, 0.f);
  if constexpr (W >= 4) v += dpp_f<0x4E>(v, 0.f);
  if constexpr (W >= 8) v += dpp_f<0x141>(v, 0.f);
  if constexpr (W >= 16) v += dpp_f<0x140>(v, 0.f);
  if constexpr (W >= 32) {
    const auto r = __builtin_amdgcn_permlane16_swap(__float_as_uint(v), __float_as_uint(v), false, false);
    v = __uint_as_float(r[0]) + __uint_as_float(r[1]);
  }
  if constexpr (W == 64) {
    const auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(v), __float_as_uint(v), false, false);
    v = __uint_as_float(r[0]) + __uint_as_float(r[1]);
  }
  return v;
}

// Sum over aligned groups of W lanes (16, 32 or 64) with DPP prefix steps.
// The group's total is exact-order deterministic and valid in the group's
// LAST lane (lane % W == W - 1); other lanes hold partial prefixes.
template <int W>
__device__ __forceinline__ float group_sum_last(float v) {
  static_assert(W == 16 || W == 32 || W == 64, "DPP groups are 16, 32 or 64 lanes");
  v += dpp_f<0x111>(v, 0.f);
  v += dpp_f<0x112>(v, 0.f);
  v += dpp_f<0x114>(v, 0.f);
  v += dpp_f<0x118>(v, 0.f);
  if (W >= 32) v += dpp_f<0x142, 0xA>(v, 0.f);
  if (W == 64) v += dpp_f<0x143, 0xC>(v, 0.f);
  return v;
}

// Transposed reductions: several per-lane partial sums reduced at once, each
// exchange halving the values per lane while every lane stays busy.
// swap32_add(a, b): lanes 0-31 hold a's partial over lanes {l, l + 32},
// lanes 32-63 hold b's (v_permlane32_swap exchanges a's upper half with b's
// lower half).
__device__ __forceinline__ float swap32_add(float a, float b) {
  const auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(a), __float_as_uint(b), false, false);
  return __uint_as_float(r[0]) + __uint_as_float(r[1]);
}

// swap16_add(a, b): 16-lane rows 0..3 hold a (rows 0+1), b (rows 0+1),
// a (rows 2+3), b (rows 2+3) (v_permlane16_swap exchanges a's odd rows with
// b's even rows).
__device__ __forceinline__ float swap16_add(float a, float b) {
  const auto r = __builtin_amdgcn_permlane16_swap(__float_as_uint(a), __float_as_uint(b), false, false);
  return __uint_as_float(r[0]) + __uint_as_float(r[1]);
}

// Sum over each 16-lane row, in every lane of the row (row rotations by
// 8, 4, 2, 1).
__device__ __forceinline__ float row_sum16_all(float v) {
  v += dpp_f<0x128>(v, 0.f);
  v += dpp_f<0x124>(v, 0.f);
  v += dpp_f<0x122>(v, 0.f);
  v += dpp_f<0x121>(v, 0.f);
  return v;
}

// Max over the wave, valid in lane 63.
__device__ __forceinline__ float wave_max_last(float v) {
  v = fmaxf(v, dpp_f<0x111>(v, -INFINITY));
  v = fmaxf(v, dpp_f<0x112>(v, -INFINITY));
  v = fmaxf(v, dpp_f<0x114>(v, -INFINITY));
  v = fmaxf(v, dpp_f<0x118>(v, -INFINITY));
  v = fmaxf(v, dpp_f<0x142, 0xA>(v, -INFINITY));
  v = fmaxf(v, dpp_f<0x143, 0xC>(v, -INFINITY));
  return v;
}

__device__ __forceinline__ float readlane_f(float v, int lane) {
  return __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), lane));
}

__device__ __forceinline__ float wave_max(float v) {
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) v = fmaxf(v, __shfl_xor(v, o, kWave));
  return v;
}

__device__ __forceinline__ void load_x32(const float* p, float (&x)[kChunk]) {
  const float4* p4 = reinterpret_cast<const float4*>(p);
#pragma unroll
  for (int i = 0; i < kChunk / 4; ++i) {
    const float4 v = p4[i];
    x[4 * i + 0] = v.x;
    x[4 * i + 1] = v.y;
    x[4 * i + 2] = v.z;
    x[4 * i + 3] = v.w;
  }
}

__device__ __forceinline__ float silu_mul(float g, float u) {
  // moe_cpu.rs:213-217: silu = g / (1 + exp(-g)); act = silu * up.
  const float silu = g / (1.0f + expf(-g));
  return silu * u;
}

__device__ __forceinline__ float sigmoidf_ref(float x) { return 1.0f / (1.0f + expf(-x)); }

// ---------------------------------------------------------------------------
// Integer chunk dot product.
//
// A chunk of activations x[0..32) is written as 24-bit block floating
// point, x_j ~= m_j * 2^-f with one exponent per chunk (|m_j| <= 2^22, i.e.
// relative rounding 2^-23 of the chunk's largest |x|), and m_j is split
// into three signed 8-bit limbs, m = d0 + 2^8 d1 + 2^16 d2. The codes are
// unpacked to bytes, and v_dot4c_i32_i8 accumulates sum_j q_j d_Lj exactly
// in int32 (|sum| <= 32 * 15 * 128). The dot product is then
//     sum_j q_j x_j = 2^-f * (S0 + 2^8 S1 + 2^16 S2)
// rounded once or twice at f32 precision: 1.1 VALU ops per 4-bit weight
// instead of 2.4 for convert-and-FMA. A chunk whose largest |x| is below
// 2^-128 gets a scale 2^-f that underflows to 0 and contributes 0 (an
// absolute error below 480 * 2^-128).
//
// Byte order: code word i (inputs 8i .. 8i+7) unpacks to lo = bytes
// [q(8i), q(8i+2), q(8i+4), q(8i+6)] and hi = [q(8i+1), q(8i+3), q(8i+5),
// q(8i+7)] (4-bit: nibble masks; 3-bit pack i: 6-bit fields spread to
// bytes). Limb word 2i holds the lo order, word 2i+1 the hi order.
// ---------------------------------------------------------------------------
struct XLimbs {
  uint32_t w[3][8];  // limb L, word 2i (lo order) / 2i+1 (hi order)
  float scale;       // 2^-f
  float xs;          // sum_j x_j (f32, for the bias term)
};
constexpr int kXLimbWords = 32;  // dwords per chunk in memory: 24 limbs, scale, xs, pad

__device__ __forceinline__ uint32_t pack_bytes(int32_t a, int32_t b, int32_t c, int32_t d) {
  return (uint32_t)(a & 0xFF) | ((uint32_t)(b & 0xFF) << 8) | ((uint32_t)(c & 0xFF) << 16) |
         ((uint32_t)d << 24);
}

__device__ __forceinline__ void make_limbs(const float (&x)[kChunk], XLimbs& o) {
  float amax = 0.f;
#pragma unroll
  for (int j = 0; j < kChunk; ++j) amax = fmaxf(amax, fabsf(x[j]));
  // |x| < 2^E with E the frexp exponent of amax; scale to |m| < 2^22.
  const int f = amax > 0.f ? 22 - __builtin_amdgcn_frexp_expf(amax) : 0;
  int32_t d[3][kChunk];
#pragma unroll
  for (int j = 0; j < kChunk; ++j) {
    const int32_t m = (int32_t)__builtin_rintf(__builtin_ldexpf(x[j], f));
    const int32_t d0 = (m << 24) >> 24;
    const int32_t m1 = (m - d0) >> 8;
    const int32_t d1 = (m1 << 24) >> 24;
    d[0][j] = d0;
    d[1][j] = d1;
    d[2][j] = (m1 - d1) >> 8;
  }
#pragma unroll
  for (int L = 0; L < 3; ++L)
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      o.w[L][2 * i] = pack_bytes(d[L][8 * i], d[L][8 * i + 2], d[L][8 * i + 4], d[L][8 * i + 6]);
      o.w[L][2 * i + 1] = pack_bytes(d[L][8 * i + 1], d[L][8 * i + 3], d[L][8 * i + 5], d[L][8 * i + 7]);
    }
  o.scale = __builtin_ldexpf(1.0f, -f);
  o.xs = xsum(x);
}

// Codes of a chunk as bytes in the order above.
__device__ __forceinline__ void unpack_bytes(const Raw<4>& r, uint32_t (&b)[8]) {
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    b[2 * i] = r.d[i] & 0x0F0F0F0Fu;
    b[2 * i + 1] = (r.d[i] >> 4) & 0x0F0F0F0Fu;
  }
}

__device__ __forceinline__ void unpack_bytes(const Raw<3>& r, uint32_t (&b)[8]) {
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    // 24-bit pack i of the 96-bit chunk.
    uint32_t p;
    if (i == 0)
      p = r.d[0];
    else if (i == 1)
      p = __builtin_amdgcn_alignbit(r.d[1], r.d[0], 24);
    else if (i == 2)
      p = __builtin_amdgcn_alignbit(r.d[2], r.d[1], 16);
    else
      p = r.d[2] >> 8;
    // 6-bit field k (codes 2k, 2k+1) to byte k in two bitfield inserts
    // (v_bfi_b32): fields 2, 3 move up by 4 bits, then fields 1, 3 by 2.
    // Bits outside the fields (p's upper byte, copies left between the
    // fields) end up only in bits 6-7 of each byte, which the masks drop.
    // (The empty asm keeps the compiler from distributing the final masks
    // back into the inserts, which costs more instructions than it saves.)
    uint32_t u = (p & 0x00000FFFu) | ((p << 4) & ~0x00000FFFu);
    asm volatile("" : "+v"(u));
    uint32_t t = (u & 0x003F003Fu) | ((u << 2) & ~0x003F003Fu);
    asm volatile("" : "+v"(t));
    b[2 * i] = t & 0x07070707u;
    b[2 * i + 1] = (t >> 3) & 0x07070707u;
  }
}

// s * sum_j q_j x_j + b * sum_j x_j for one chunk.
template <int BITS>
__device__ __forceinline__ float chunk_dot_i(const Raw<BITS>& raw, const XLimbs& xl, float s, float b) {
  uint32_t q[8];
  unpack_bytes(raw, q);
  int32_t S0 = 0, S1 = 0, S2 = 0;
#pragma unroll
  for (int w = 0; w < 8; ++w) {
    S0 = __builtin_amdgcn_sdot4((int)q[w], (int)xl.w[0][w], S0, false);
    S1 = __builtin_amdgcn_sdot4((int)q[w], (int)xl.w[1][w], S1, false);
    S2 = __builtin_amdgcn_sdot4((int)q[w], (int)xl.w[2][w], S2, false);
  }
  const float t = __builtin_fmaf((float)S2, 65536.0f, __builtin_fmaf((float)S1, 256.0f, (float)S0));
  return __builtin_fmaf(s, t * xl.scale, b * xl.xs);
}

__device__ __forceinline__ void load_limbs(const uint32_t* p, XLimbs& o) {
  const u32x4* p4 = reinterpret_cast<const u32x4*>(p);
  u32x4 v[7];
#pragma unroll
  for (int i = 0; i < 7; ++i) v[i] = p4[i];
#pragma unroll
  for (int i = 0; i < 6; ++i) {
    const uint32_t e[4] = {v[i].x, v[i].y, v[i].z, v[i].w};
#pragma unroll
    for (int c = 0; c < 4; ++c) o.w[(4 * i + c) / 8][(4 * i + c) % 8] = e[c];
  }
  o.scale = __uint_as_float(v[6].x);
  o.xs = __uint_as_float(v[6].y);
}

__device__ __forceinline__ void store_limbs(uint32_t* p, const XLimbs& o) {
  u32x4* p4 = reinterpret_cast<u32x4*>(p);
#pragma unroll
  for (int i = 0; i < 6; ++i) {
    u32x4 v;
    v.x = o.w[(4 * i) / 8][(4 * i) % 8];
    v.y = o.w[(4 * i + 1) / 8][(4 * i + 1) % 8];
    v.z = o.w[(4 * i + 2) / 8][(4 * i + 2) % 8];
    v.w = o.w[(4 * i + 3) / 8][(4 * i + 3) % 8];
    p4[i] = v;
  }
  u32x4 t;
  t.x = __float_as_uint(o.scale);
  t.y = __float_as_uint(o.xs);
  t.z = 0;
  t.w = 0;
  p4[6] = t;
}

// Raises kernel fn's dynamic LDS limit to `bytes` on the current device,
// once per device (`done` holds one bit per device index); function
// attributes belong to a device, so a process that launches on several
// devices sets them on each.
inline hipError_t raise_lds_limit(const void* fn, int bytes, std::atomic<uint64_t>& done) {
  int dev = 0;
  hipError_t e = hipGetDevice(&dev);
  if (e != hipSuccess) return e;
  const uint64_t bit = 1ull << (dev & 63);
  if (done.load(std::memory_order_acquire) & bit) return hipSuccess;
  e = hipFuncSetAttribute(fn, hipFuncAttributeMaxDynamicSharedMemorySize, bytes);
  if (e == hipSuccess) done.fetch_or(bit, std::memory_order_acq_rel);
  return e;
}

}  // namespace smoe
