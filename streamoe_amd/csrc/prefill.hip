// prefill.hip — many tokens through one layer's routed experts (gfx950).
//
// Replaces the reference's gather-by-expert prefill (encode_moe_gather_id_fuse,
// expert_forward.rs:1874-2042: map0 bucketing, per-expert quantized GEMMs,
// combine), whose CPU statement is build_expert_buckets (moe_router.rs:
// 374-436) + moe_permute_fuse_cpu (moe_cpu.rs:282-339).
//
//   k_pf_route    one block: bucket the n*k assignments by expert (stable in
//                 token order), per-token entry positions in ascending
//                 expert order, and a work list of (expert, <= kPfMC
//                 entries) items, so a hot expert is spread over many waves.
//   k_pf_rowsum   group sums of x rows (and later of the activations), the
//                 per-group terms of the dequant epilogue.
//   k_pf_gemm     one block per (item, 256 output columns), bf16 MFMA
//                 (v_mfma_f32_16x16x32_bf16): mode 0 gate and up rows of the
//                 item's expert -> act = silu(gate) * up; mode 1 down rows
//                 over the activations split into bf16 hi + lo halves.
//   k_pf_combine  out[t] = sum over t's entries in ascending expert order of
//                 fma(down[entry], w[entry], out) (moe_cpu.rs:330-337), no
//                 atomics.
//
// Exact dequant semantics on MFMA: a code q enters the MFMA as the bf16
// number 128 + q (bits 0x4300 | q, exact), each group of G inputs
// accumulates into its own fp32 accumulator acc = sum (128 + q_k) x_k, and
// the epilogue adds s * (acc - 128 * sum x) + b * sum x = s * acc + (b -
// 128 s) * sum x, which is sum_k (q_k s + b) x_k up to fp32 rounding. x is
// bf16 (exact in the MFMA) or an fp32 vector split into bf16 hi + lo (two
// MFMAs into the same accumulator, ~2^-17 relative).
//
// K order inside one MFMA (16x16x32: lane l holds row/column l % 16 and 8
// values at k-block l / 16): within a group, lane block q covers the 8*NU
// consecutive inputs G*g + 8*NU*q + [0, 8*NU), NU = G / 32 MFMAs per group,
// and the 8 values of one MFMA step are in the order of the code unpack,
// [v0, v4, v1, v5, v2, v6, v3, v7]; activations are permuted to match.
#include "common.h"
#include "kernels.h"

namespace smoe {

typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef __bf16 bf16x2 __attribute__((ext_vector_type(2)));
typedef float f32x2 __attribute__((ext_vector_type(2)));

constexpr uint32_t kPfMC = 32;  // entries per work item (two 16-row MFMA tiles)

// ---------------------------------------------------------------------------
// Bucketing (one block of 1024 threads).
// ---------------------------------------------------------------------------
__device__ __forceinline__ uint32_t popc_below(const uint32_t* row, uint32_t e) {
  uint32_t c = 0;
  for (uint32_t w = 0; w < (e >> 5); ++w) c += __popc(row[w]);
  return c + __popc(row[e >> 5] & ((1u << (e & 31)) - 1u));
}

// Exclusive scan of v over threads [0, n) (n <= 1024) through LDS.
__device__ uint32_t block_exscan(uint32_t v, uint32_t n, uint32_t* tmp, uint32_t* total) {
  const uint32_t t = threadIdx.x;
  if (t < n) tmp[t] = v;
  __syncthreads();
  for (uint32_t o = 1; o < n; o <<= 1) {
    uint32_t add = 0;
    if (t < n && t >= o) add = tmp[t - o];
    __syncthreads();
    if (t < n) tmp[t] += add;
    __syncthreads();
  }
  const uint32_t incl = t < n ? tmp[t] : 0;
  *total = tmp[n - 1];
  __syncthreads();
  return incl - (t < n ? v : 0);
}

__global__ __launch_bounds__(1024) void k_pf_route(PfArgs a) {
  __shared__ uint32_t bits[kPfMaxTokens * (kPfMaxExperts / 32)];
  __shared__ uint8_t slot_of[kPfMaxTokens * kPfMaxK];
  __shared__ uint32_t tmp[1024];
  const uint32_t tid = threadIdx.x, n = a.n_tokens, k = a.k, E = a.E;
  const uint32_t words = (E + 31) / 32, total = n * k;
  for (uint32_t i = tid; i < n * words; i += blockDim.x) bits[i] = 0;
  __syncthreads();
  for (uint32_t i = tid; i < total; i += blockDim.x) {
    const int32_t e = a.idx[i];
    if (e < 0 || (uint32_t)e >= E) {
      *a.err = 2u;
      continue;
    }
    const uint32_t old = atomicOr(&bits[(i / k) * words + (e >> 5)], 1u << (e & 31));
    if (old & (1u << (e & 31))) *a.err = 2u;  // an expert twice in one token
  }
  __syncthreads();
  // Entry rank of (t, s) among t's experts in ascending order -> slot s.
  for (uint32_t i = tid; i < total; i += blockDim.x) {
    const int32_t e = a.idx[i];
    if (e < 0 || (uint32_t)e >= E) continue;
    const uint32_t t = i / k;
    slot_of[t * k + popc_below(&bits[t * words], (uint32_t)e)] = (uint8_t)(i - t * k);
  }
  uint32_t cnt = 0;
  if (tid < E)
    for (uint32_t t = 0; t < n; ++t) cnt += (bits[t * words + (tid >> 5)] >> (tid & 31)) & 1u;
  uint32_t n_entries;
  const uint32_t off = block_exscan(cnt, E, tmp, &n_entries);
  const uint32_t nch = (cnt + kPfMC - 1) / kPfMC;
  uint32_t n_items;
  const uint32_t ibase = block_exscan(nch, E, tmp, &n_items);
  if (tid == 0) *a.n_items = n_items;
  if (tid < E) {
    for (uint32_t c = 0; c < nch; ++c) {
      const uint32_t start = off + c * kPfMC;
      const uint32_t m = min(kPfMC, cnt - c * kPfMC);
      a.items[2 * (ibase + c)] = tid;
      a.items[2 * (ibase + c) + 1] = start | (m << 16);
    }
    uint32_t pos = off;
    for (uint32_t t = 0; t < n && pos < off + cnt; ++t) {
      const uint32_t* row = &bits[t * words];
      if (!((row[tid >> 5] >> (tid & 31)) & 1u)) continue;
      const uint32_t r = popc_below(row, tid);
      const uint32_t s = slot_of[t * k + r];
      a.ent_token[pos] = (int32_t)t;
      a.ent_weight[pos] = a.w[t * k + s];
      a.tok_pos[t * k + r] = (int32_t)pos;
      ++pos;
    }
  }
}

// ---------------------------------------------------------------------------
// Group sums: out[r, g] = sum of src[r, G*g .. G*g + G) (bf16 or f32 rows).
// ---------------------------------------------------------------------------
__global__ __launch_bounds__(256) void k_pf_rowsum(const void* src, int is_bf16, uint32_t cols,
                                                   uint32_t G, const uint32_t* n_rows_dev,
                                                   uint32_t n_rows, float* out) {
  const uint32_t r = blockIdx.x;
  if (n_rows_dev && r >= *n_rows_dev) return;
  if (r >= n_rows) return;
  const uint32_t ng = cols / G;
  for (uint32_t g = threadIdx.x; g < ng; g += blockDim.x) {
    float s = 0.f;
    if (is_bf16) {
      const uint16_t* p = reinterpret_cast<const uint16_t*>(src) + (size_t)r * cols + (size_t)g * G;
      for (uint32_t j = 0; j < G; ++j) s += bf16f(p[j]);
    } else {
      const float* p = reinterpret_cast<const float*>(src) + (size_t)r * cols + (size_t)g * G;
      for (uint32_t j = 0; j < G; ++j) s += p[j];
    }
    out[(size_t)r * ng + g] = s;
  }
}

// ---------------------------------------------------------------------------
// MFMA operand helpers.
// ---------------------------------------------------------------------------
// 8 codes (one 4-bit u32) as bf16 (128 + q) in the order [q0,q4,q1,q5,q2,q6,q3,q7].
__device__ __forceinline__ u32x4 codes_bf16_4(uint32_t d) {
  u32x4 r;
  r.x = (d & 0x000F000Fu) | 0x43004300u;
  r.y = ((d >> 4) & 0x000F000Fu) | 0x43004300u;
  r.z = ((d >> 8) & 0x000F000Fu) | 0x43004300u;
  r.w = ((d >> 12) & 0x000F000Fu) | 0x43004300u;
  return r;
}

// 8 codes of one 24-bit 3-bit pack as bf16 (128 + q), same order.
__device__ __forceinline__ u32x4 codes_bf16_3(uint32_t p) {
  const uint32_t t = (p & 0x3Fu) | ((p & 0xFC0u) << 2) | ((p & 0x3F000u) << 4) | ((p & 0xFC0000u) << 6);
  const uint32_t lo = t & 0x07070707u;         // [c0, c2, c4, c6]
  const uint32_t hi = (t >> 3) & 0x07070707u;  // [c1, c3, c5, c7]
  u32x4 r;
  r.x = (lo & 0x00FF00FFu) | 0x43004300u;         // (c0, c4)
  r.y = (hi & 0x00FF00FFu) | 0x43004300u;         // (c1, c5)
  r.z = ((lo >> 8) & 0x00FF00FFu) | 0x43004300u;  // (c2, c6)
  r.w = ((hi >> 8) & 0x00FF00FFu) | 0x43004300u;  // (c3, c7)
  return r;
}

// 8 bf16 values (4 dwords, natural order) -> [v0,v4,v1,v5,v2,v6,v3,v7].
__device__ __forceinline__ u32x4 perm_bf16(u32x4 v) {
  u32x4 r;
  r.x = __builtin_amdgcn_perm(v.z, v.x, 0x05040100u);
  r.y = __builtin_amdgcn_perm(v.z, v.x, 0x07060302u);
  r.z = __builtin_amdgcn_perm(v.w, v.y, 0x05040100u);
  r.w = __builtin_amdgcn_perm(v.w, v.y, 0x07060302u);
  return r;
}

__device__ __forceinline__ uint32_t pk_bf16(float a, float b) {
  const f32x2 v = {a, b};
  return __builtin_bit_cast(uint32_t, __builtin_convertvector(v, bf16x2));
}

// 8 floats -> hi and lo bf16 halves in the permuted order.
__device__ __forceinline__ void split_f32(const float (&f)[8], u32x4& hi, u32x4& lo) {
  hi.x = pk_bf16(f[0], f[4]);
  hi.y = pk_bf16(f[1], f[5]);
  hi.z = pk_bf16(f[2], f[6]);
  hi.w = pk_bf16(f[3], f[7]);
  const uint32_t h[4] = {hi.x, hi.y, hi.z, hi.w};
  float r[8];
#pragma unroll
  for (int j = 0; j < 4; ++j) {
    r[j] = f[j] - __uint_as_float(h[j] << 16);
    r[j + 4] = f[j + 4] - __uint_as_float(h[j] & 0xFFFF0000u);
  }
  lo.x = pk_bf16(r[0], r[4]);
  lo.y = pk_bf16(r[1], r[5]);
  lo.z = pk_bf16(r[2], r[6]);
  lo.w = pk_bf16(r[3], r[7]);
}

__device__ __forceinline__ f32x4 mfma(u32x4 a, u32x4 b, f32x4 c) {
  return __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(bf16x8, a),
                                                 __builtin_bit_cast(bf16x8, b), c, 0, 0, 0);
}

// Codes of `row` for lane block q of group g: NU u32 words of 8 codes each
// (4-bit), or NU 24-bit packs (3-bit), for inputs G*g + 8*NU*q + [0, 8*NU).
template <int BITS, int NU>
__device__ __forceinline__ void load_codes(const uint8_t* base, uint32_t row_bytes, uint32_t row,
                                           uint32_t g, uint32_t q, uint32_t (&w)[NU]) {
  const uint8_t* r = base + (size_t)row * row_bytes;
  if (BITS == 4) {
    // byte offset (32*NU*g + 8*NU*q) / 2
    const uint32_t* p = reinterpret_cast<const uint32_t*>(r + (size_t)(4 * g + q) * NU * 4);
#pragma unroll
    for (int u = 0; u < NU; ++u) w[u] = ld_stream(p + u);
  } else {
    // 3*NU bytes at byte offset 3*(32*NU*g + 8*NU*q)/8 = 3*NU*(4g + q); load
    // the dword-aligned window around them (within the blob: the scales
    // follow the codes of every block).
    const uint32_t o = (4 * g + q) * NU * 3;
    const uint32_t* p = reinterpret_cast<const uint32_t*>(r + (o & ~3u));
    constexpr int ND = (3 * NU + 6) / 4;
    uint32_t d[ND];
#pragma unroll
    for (int i = 0; i < ND; ++i) d[i] = ld_stream(p + i);
    const uint32_t sh = (o & 3u) * 8;
#pragma unroll
    for (int u = 0; u < NU; ++u) {
      const uint32_t bit = sh + 24 * u;
      uint32_t lo = 0, hi = 0;
#pragma unroll
      for (int i = 0; i < ND; ++i) {
        if ((uint32_t)i == (bit >> 5)) lo = d[i];
        if ((uint32_t)i == (bit >> 5) + 1) hi = d[i];
      }
      w[u] = __builtin_amdgcn_alignbit(hi, lo, bit & 31) & 0xFFFFFFu;
    }
  }
}

template <int BITS>
__device__ __forceinline__ u32x4 codes_bf16(uint32_t w) {
  return BITS == 4 ? codes_bf16_4(w) : codes_bf16_3(w);
}

// ---------------------------------------------------------------------------
// Grouped GEMM over the work list. One block (16 waves) per (item, 256
// output columns); wave w owns columns 16w .. 16w + 15 of the block, lane
// (n = l % 16, q = l / 16) column n and k-block q. The item's <= 32 entry
// rows are staged in LDS chunk by chunk (kPfKC inputs, permuted to the code
// order, split into bf16 hi + lo when they are fp32); the next chunk's codes
// and scales are loaded into registers while the current chunk computes.
// MODE 0: gate and up (K = hidden, A = x rows of the entries' tokens),
// act = silu(gate) * up. MODE 1: down (K = inter, A = act rows).
// ---------------------------------------------------------------------------
// Inputs per LDS chunk: 128 for gate/up (two weight matrices in flight per
// lane), 256 for down; both dimensions of the layer are multiples of 256.
template <int MODE>
constexpr int pf_kc() {
  return MODE == 0 ? 128 : 256;
}
constexpr int kPfKC = 256;

template <int BITS, int G, int NMAT, int KC>
struct PfChunk {
  static constexpr int NU = G / 32, CG = KC / G;
  uint32_t w[NMAT][CG][NU];
  uint32_t sb[NMAT][CG];  // bf16 scale | bf16 bias << 16
};

template <int BITS, int G, int MODE, bool SPLIT>
__global__ __launch_bounds__(1024) void k_pf_gemm(PfArgs a) {
  constexpr int KC = pf_kc<MODE>();
  constexpr int AROW = KC + 8;  // LDS row stride in bf16 (16-byte pad)
  constexpr int NU = G / 32, CG = KC / G, NMAT = MODE == 0 ? 2 : 1;
  static_assert(CG >= 1, "chunk must hold a whole group");
  __shared__ __attribute__((aligned(16))) uint16_t ahi[kPfMC * AROW];
  __shared__ __attribute__((aligned(16))) uint16_t alo[(SPLIT ? kPfMC : 1) * AROW];
  __shared__ float sxs[kPfMC * kPfMaxGroupsK];
  const uint32_t item = blockIdx.x;
  if (item >= *a.n_items) return;
  const uint32_t e = a.items[2 * item];
  const uint32_t start = a.items[2 * item + 1] & 0xFFFFu, cnt = a.items[2 * item + 1] >> 16;
  const uint32_t tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const uint32_t n = lane & 15, q = lane >> 4;
  const BlobGeom& gm = a.g;
  const uint32_t K = MODE == 0 ? gm.hidden : gm.inter;
  const uint32_t N = MODE == 0 ? gm.inter : gm.hidden;
  const uint32_t ng = K / G, nch = K / KC, rowb = K * BITS / 8;
  const uint32_t col = blockIdx.y * 256 + wave * 16 + n;
  const uint8_t* blob = a.experts + (size_t)e * a.stride;
  const uint32_t ntiles = (cnt + 15) / 16;

  // Group sums of the entries' A rows.
  for (uint32_t i = tid; i < kPfMC * ng; i += blockDim.x) {
    const uint32_t m = i / ng, g = i % ng, mm = min(m, cnt - 1);
    sxs[i] = MODE == 0 ? a.xsum[(size_t)a.ent_token[start + mm] * ng + g]
                       : a.asum[(size_t)(start + mm) * ng + g];
  }

  // A staging: thread -> (row m, 8 inputs at 8 * sp of the chunk); the first
  // kPfMC * KC / 8 threads take part.
  constexpr uint32_t SPR = KC / 8;  // staging threads per row
  const bool stager = tid < kPfMC * SPR;
  const uint32_t sm = stager ? tid / SPR : 0, sp = tid % SPR;
  const uint32_t srow = MODE == 0 ? (uint32_t)a.ent_token[start + min(sm, cnt - 1)] : start + min(sm, cnt - 1);
  float sf[8];
  u32x4 sv;
  auto a_load = [&](uint32_t c) {
    if (!stager) return;
    const size_t k0 = (size_t)c * KC + 8 * sp;
    if (MODE == 0 && !SPLIT) {
      sv = *reinterpret_cast<const u32x4*>(reinterpret_cast<const uint16_t*>(a.x) + (size_t)srow * K + k0);
    } else {
      const float* p = (MODE == 0 ? reinterpret_cast<const float*>(a.x) : a.act) + (size_t)srow * K + k0;
      const float4 v0 = *reinterpret_cast<const float4*>(p);
      const float4 v1 = *reinterpret_cast<const float4*>(p + 4);
      sf[0] = v0.x; sf[1] = v0.y; sf[2] = v0.z; sf[3] = v0.w;
      sf[4] = v1.x; sf[5] = v1.y; sf[6] = v1.z; sf[7] = v1.w;
    }
  };
  auto a_store = [&]() {
    if (!stager) return;
    u32x4* dh = reinterpret_cast<u32x4*>(ahi + sm * AROW + 8 * sp);
    if (MODE == 0 && !SPLIT) {
      *dh = perm_bf16(sv);
    } else {
      u32x4 hi, lo;
      split_f32(sf, hi, lo);
      *dh = hi;
      if (SPLIT) *reinterpret_cast<u32x4*>(alo + sm * AROW + 8 * sp) = lo;
    }
  };
  auto b_load = [&](uint32_t c, PfChunk<BITS, G, NMAT, KC>& ch) {
#pragma unroll
    for (int mat = 0; mat < NMAT; ++mat) {
      const int blk = MODE == 0 ? mat : 2;
#pragma unroll
      for (int gl = 0; gl < CG; ++gl) {
        const uint32_t g = c * CG + gl;
        load_codes<BITS, NU>(blob + gm.w[blk], rowb, col, g, q, ch.w[mat][gl]);
        const size_t gi = ((size_t)col * ng + g) * 2;
        const uint32_t sv16 = *reinterpret_cast<const uint16_t*>(blob + gm.s[blk] + gi);
        const uint32_t bv16 = *reinterpret_cast<const uint16_t*>(blob + gm.b[blk] + gi);
        ch.sb[mat][gl] = sv16 | (bv16 << 16);
      }
    }
  };
  f32x4 tot[NMAT][2];
#pragma unroll
  for (int mat = 0; mat < NMAT; ++mat)
#pragma unroll
    for (int t = 0; t < 2; ++t) tot[mat][t] = f32x4{0.f, 0.f, 0.f, 0.f};

  auto compute = [&](uint32_t c, const PfChunk<BITS, G, NMAT, KC>& ch) {
#pragma unroll
    for (int gl = 0; gl < CG; ++gl) {
      const uint32_t g = c * CG + gl;
      float s[NMAT], cb[NMAT];
#pragma unroll
      for (int mat = 0; mat < NMAT; ++mat) {
        s[mat] = __uint_as_float(ch.sb[mat][gl] << 16);
        cb[mat] = __builtin_fmaf(-128.0f, s[mat], __uint_as_float(ch.sb[mat][gl] & 0xFFFF0000u));
      }
#pragma unroll
      for (int t = 0; t < 2; ++t) {
        if ((uint32_t)t >= ntiles) continue;
        const uint32_t arow = (16 * t + n) * AROW + gl * G + 8 * NU * q;
        f32x4 acc[NMAT];
#pragma unroll
        for (int mat = 0; mat < NMAT; ++mat) acc[mat] = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
        for (int u = 0; u < NU; ++u) {
          const u32x4 ah = *reinterpret_cast<const u32x4*>(ahi + arow + 8 * u);
          u32x4 al;
          if (SPLIT) al = *reinterpret_cast<const u32x4*>(alo + arow + 8 * u);
#pragma unroll
          for (int mat = 0; mat < NMAT; ++mat) {
            const u32x4 bq = codes_bf16<BITS>(ch.w[mat][gl][u]);
            acc[mat] = mfma(ah, bq, acc[mat]);
            if (SPLIT) acc[mat] = mfma(al, bq, acc[mat]);
          }
        }
#pragma unroll
        for (int r = 0; r < 4; ++r) {
          const float xs = sxs[(16 * t + 4 * q + r) * ng + g];
#pragma unroll
          for (int mat = 0; mat < NMAT; ++mat)
            tot[mat][t][r] = __builtin_fmaf(s[mat], acc[mat][r], __builtin_fmaf(cb[mat], xs, tot[mat][t][r]));
        }
      }
    }
  };

  PfChunk<BITS, G, NMAT, KC> b0, b1;
  a_load(0);
  b_load(0, b0);
  a_store();
  __syncthreads();
  for (uint32_t c = 0; c < nch; c += 2) {
    if (c + 1 < nch) {
      a_load(c + 1);
      b_load(c + 1, b1);
    }
    compute(c, b0);
    if (c + 1 >= nch) break;
    __syncthreads();
    a_store();
    __syncthreads();
    if (c + 2 < nch) {
      a_load(c + 2);
      b_load(c + 2, b0);
    }
    compute(c + 1, b1);
    if (c + 2 >= nch) break;
    __syncthreads();
    a_store();
    __syncthreads();
  }

#pragma unroll
  for (int t = 0; t < 2; ++t) {
    if ((uint32_t)t >= ntiles) continue;
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      const uint32_t m = 16 * t + 4 * q + r;
      if (m >= cnt) continue;
      if (MODE == 0)
        a.act[(size_t)(start + m) * N + col] = silu_mul(tot[0][t][r], tot[1][t][r]);
      else
        a.down[(size_t)(start + m) * N + col] = tot[0][t][r];
    }
  }
}

// ---------------------------------------------------------------------------
// Combine: out[t, :] = fold over t's entries in ascending expert order.
// ---------------------------------------------------------------------------
__global__ __launch_bounds__(256) void k_pf_combine(PfArgs a) {
  const uint32_t t = blockIdx.x;
  const uint32_t H = a.g.hidden, k = a.k;
  int32_t pos[kPfMaxK];
  float wt[kPfMaxK];
  const uint32_t nk = a.n_tokens * k;
  for (uint32_t r = 0; r < k; ++r) {
    // In range even when bucketing rejected the input (then *err is set).
    pos[r] = (int32_t)min((uint32_t)a.tok_pos[t * k + r], nk - 1);
    wt[r] = a.ent_weight[pos[r]];
  }
  for (uint32_t h = threadIdx.x * 4; h < H; h += blockDim.x * 4) {
    float4 o = make_float4(0.f, 0.f, 0.f, 0.f);
    for (uint32_t r = 0; r < k; ++r) {
      const float4 d = *reinterpret_cast<const float4*>(a.down + (size_t)pos[r] * H + h);
      o.x = __builtin_fmaf(d.x, wt[r], o.x);
      o.y = __builtin_fmaf(d.y, wt[r], o.y);
      o.z = __builtin_fmaf(d.z, wt[r], o.z);
      o.w = __builtin_fmaf(d.w, wt[r], o.w);
    }
    *reinterpret_cast<float4*>(a.out + (size_t)t * H + h) = o;
  }
}

// ---------------------------------------------------------------------------
// Host side.
// ---------------------------------------------------------------------------
static uint64_t al256(uint64_t n) { return (n + 255) & ~255ull; }

uint64_t prefill_workspace(uint32_t hidden, uint32_t inter, uint32_t group, uint32_t n_tokens,
                           uint32_t n_experts, uint32_t k, PfArgs* a, uint8_t* base) {
  const uint64_t nk = (uint64_t)n_tokens * k;
  const uint64_t max_items = n_experts + nk / kPfMC + 1;
  uint64_t off = 0;
  auto take = [&](uint64_t bytes) {
    const uint64_t o = off;
    off += al256(bytes);
    return base ? base + o : nullptr;
  };
  uint8_t* p_items = take(max_items * 2 * 4);
  uint8_t* p_nitems = take(4);
  uint8_t* p_tok = take(nk * 4);
  uint8_t* p_w = take(nk * 4);
  uint8_t* p_pos = take(nk * 4);
  uint8_t* p_xsum = take((uint64_t)n_tokens * (hidden / group) * 4);
  uint8_t* p_asum = take(nk * (inter / group) * 4);
  uint8_t* p_act = take(nk * inter * 4);
  uint8_t* p_down = take(nk * hidden * 4);
  if (a) {
    a->items = reinterpret_cast<uint32_t*>(p_items);
    a->n_items = reinterpret_cast<uint32_t*>(p_nitems);
    a->ent_token = reinterpret_cast<int32_t*>(p_tok);
    a->ent_weight = reinterpret_cast<float*>(p_w);
    a->tok_pos = reinterpret_cast<int32_t*>(p_pos);
    a->xsum = reinterpret_cast<float*>(p_xsum);
    a->asum = reinterpret_cast<float*>(p_asum);
    a->act = reinterpret_cast<float*>(p_act);
    a->down = reinterpret_cast<float*>(p_down);
    a->max_items = (uint32_t)max_items;
  }
  return off;
}

bool prefill_supported(uint32_t hidden, uint32_t inter, uint32_t group, uint32_t bits,
                       uint32_t n_tokens, uint32_t n_experts, uint32_t k) {
  if (bits != 4 && bits != 3) return false;
  if (group != 32 && group != 64 && group != 128) return false;
  if (hidden % kPfKC || inter % kPfKC) return false;
  if (hidden / group > kPfMaxGroupsK || inter / group > kPfMaxGroupsK) return false;
  if (n_tokens < 1 || n_tokens > kPfMaxTokens || n_experts < 1 || n_experts > kPfMaxExperts) return false;
  if (k < 1 || k > kPfMaxK || k > n_experts) return false;
  if ((uint64_t)n_tokens * k > 0xFFFFu) return false;
  return true;
}

template <int BITS, int G>
static void launch_gemms(const PfArgs& a, hipStream_t st) {
  const dim3 gu(a.max_items, a.g.inter / 256), dn(a.max_items, a.g.hidden / 256);
  if (a.x_bf16)
    hipLaunchKernelGGL((k_pf_gemm<BITS, G, 0, false>), gu, dim3(1024), 0, st, a);
  else
    hipLaunchKernelGGL((k_pf_gemm<BITS, G, 0, true>), gu, dim3(1024), 0, st, a);
  const uint32_t nk = a.n_tokens * a.k;
  hipLaunchKernelGGL(k_pf_rowsum, dim3(nk), dim3(64), 0, st, (const void*)a.act, 0, a.g.inter,
                     (uint32_t)G, (const uint32_t*)nullptr, nk, a.asum);
  hipLaunchKernelGGL((k_pf_gemm<BITS, G, 1, true>), dn, dim3(1024), 0, st, a);
}

hipError_t launch_prefill(const PfArgs& a, hipStream_t st) {
  hipLaunchKernelGGL(k_pf_route, dim3(1), dim3(1024), 0, st, a);
  hipLaunchKernelGGL(k_pf_rowsum, dim3(a.n_tokens), dim3(64), 0, st, a.x, a.x_bf16, a.g.hidden,
                     a.g.group, (const uint32_t*)nullptr, a.n_tokens, a.xsum);
  const uint32_t G = a.g.group;
  if (a.g.bits == 4) {
    if (G == 32) launch_gemms<4, 32>(a, st);
    else if (G == 64) launch_gemms<4, 64>(a, st);
    else launch_gemms<4, 128>(a, st);
  } else {
    if (G == 32) launch_gemms<3, 32>(a, st);
    else if (G == 64) launch_gemms<3, 64>(a, st);
    else launch_gemms<3, 128>(a, st);
  }
  hipLaunchKernelGGL(k_pf_combine, dim3(a.n_tokens), dim3(256), 0, st, a);
  return hipGetLastError();
}

}  // namespace smoe
