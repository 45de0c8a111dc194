// prefill.hip — many tokens through one layer's routed experts (gfx950).
//
// Replaces the reference's gather-by-expert prefill (encode_moe_gather_id_fuse,
// expert_forward.rs:1874-2042: map0 bucketing, per-expert quantized GEMMs,
// combine), whose CPU statement is build_expert_buckets (moe_router.rs:
// 374-436) + moe_permute_fuse_cpu (moe_cpu.rs:282-339).
//
//   k_pf_route    blocks 0..nb-1 (nb <= 8), one thread per token: bucket
//                 the n*k assignments by expert (stable in token order),
//                 per-token entry positions in ascending expert order, a work
//                 list of (expert, <= kPfMC entries) items, so a hot expert
//                 is spread over many waves, and the token of each item row
//                 (every block buckets, each stores a share). Blocks
//                 nb..: each token's x row in the MFMA k-order (bf16, or f32
//                 split into bf16 hi + lo) and its group sums (the per-group
//                 terms of the dequant epilogue), once per token.
//   k_pf_mm       persistent pipelined grouped GEMM on MFMA
//                 (v_mfma_f32_16x16x32_bf16 / _f16) over (item, column
//                 block) units: mode 0 gate and up rows of the item's expert
//                 over its tokens' x rows (copied by token id) ->
//                 act = silu(gate) * up as fp16, with the down GEMM's
//                 activation group sums for G <= 64; mode 2 down rows over
//                 the fp16 activations -> f32 per entry (mode 1: the same
//                 over bf16 hi + lo rows, the dense qmm).
//   k_pf_gu64     the gate/up GEMM for 4-bit group-64 experts over bf16 x
//                 (the reference models' format): the same pipeline on
//                 v_mfma_f32_32x32x16_bf16 tiles over (item, 128 column)
//                 units, so a chunk's token rows are a third of its copies.
//   k_pf_act_sum  activation group sums for G > 64 (a group spans more than
//                 one gate/up unit).
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
// MFMAs into the same accumulator, ~2^-17 relative). The down GEMM's
// activations are fp16 (one rounding, 2^-11 relative, as the reference's
// gather GEMM casts them, gather_mm_id.metal:397-402; magnitudes beyond
// 65504 become inf there as here); its codes enter as the fp16 number
// 1 + q / 64 (bits 0x3C00 | q << 4, exact) and the epilogue adds
// 64 s * acc + (b - 64 s) * sum a.
//
// K order inside one MFMA (16x16x32: lane l holds row/column l % 16 and 8
// values at k-block l / 16): within a group, lane block q covers the 8*NU
// consecutive inputs G*g + 8*NU*q + [0, 8*NU), NU = G / 32 MFMAs per group,
// and the 8 values of one MFMA step are in the order of the code unpack,
// [v0, v4, v1, v5, v2, v6, v3, v7]; activations are permuted to match.
#include "common.h"
#include "expf_ref.h"
#include "kernels.h"

namespace smoe {

typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef _Float16 f16x8 __attribute__((ext_vector_type(8)));
typedef _Float16 f16x2 __attribute__((ext_vector_type(2)));
typedef __bf16 bf16x2 __attribute__((ext_vector_type(2)));
typedef float f32x2 __attribute__((ext_vector_type(2)));

constexpr uint32_t kPfMC = 32;   // entries per work item (two 16-row MFMA tiles)
constexpr uint32_t kPfKC = 256;  // inputs per pipelined K chunk

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

__device__ __forceinline__ f32x4 mfma_f16(u32x4 a, u32x4 b, f32x4 c) {
  return __builtin_amdgcn_mfma_f32_16x16x32_f16(__builtin_bit_cast(f16x8, a),
                                                __builtin_bit_cast(f16x8, b), c, 0, 0, 0);
}

// Codes as fp16 for the down GEMM over fp16 activations: a code q enters as
// 1 + q / 64 (bits 0x3C00 | q << 4, exact), same order as the bf16 forms.
// The epilogue then adds 64 s * acc + (b - 64 s) * sum a.
__device__ __forceinline__ u32x4 codes_f16_4p(uint32_t d) {
  const uint32_t c3c = 0x3C3C3C3Cu;
  const uint32_t lo = (d << 4) & 0xF0F0F0F0u;  // q0, q2, q4, q6 in bits 4-7
  const uint32_t hi = d & 0xF0F0F0F0u;         // q1, q3, q5, q7 in bits 4-7
  u32x4 r;
  r.x = __builtin_amdgcn_perm(c3c, lo, 0x04020400u);  // (q0, q4)
  r.y = __builtin_amdgcn_perm(c3c, hi, 0x04020400u);  // (q1, q5)
  r.z = __builtin_amdgcn_perm(c3c, lo, 0x04030401u);  // (q2, q6)
  r.w = __builtin_amdgcn_perm(c3c, hi, 0x04030401u);  // (q3, q7)
  return r;
}

__device__ __forceinline__ u32x4 codes_f16_3(uint32_t p) {
  const uint32_t t = (p & 0x3Fu) | ((p & 0xFC0u) << 2) | ((p & 0x3F000u) << 4) | ((p & 0xFC0000u) << 6);
  const uint32_t lo = (t << 4) & 0x70707070u;  // [c0, c2, c4, c6] in bits 4-6
  const uint32_t hi = (t << 1) & 0x70707070u;  // [c1, c3, c5, c7] in bits 4-6
  u32x4 r;
  r.x = (lo & 0x00FF00FFu) | 0x3C003C00u;         // (c0, c4)
  r.y = (hi & 0x00FF00FFu) | 0x3C003C00u;         // (c1, c5)
  r.z = ((lo >> 8) & 0x00FF00FFu) | 0x3C003C00u;  // (c2, c6)
  r.w = ((hi >> 8) & 0x00FF00FFu) | 0x3C003C00u;  // (c3, c7)
  return r;
}

template <int BITS>
__device__ __forceinline__ u32x4 codes_bf16(uint32_t w) {
  return BITS == 4 ? codes_bf16_4(w) : codes_bf16_3(w);
}

// ---------------------------------------------------------------------------
// Bucketing (blocks 0..nb-1 of k_pf_route, 1024 threads) and the per-token
// x preparation (blocks nb.., four tokens each), in one launch: the
// preparation runs on other CUs while the bucketing blocks work.
// ---------------------------------------------------------------------------
#define PF_STAMP(i)                                                         \
  do {                                                                      \
    if (a.trace && threadIdx.x == 0 && blockIdx.x == 0) a.trace[i] = __builtin_amdgcn_s_memrealtime(); \
  } while (0)

constexpr uint32_t kPfPrepTokens = 4;                    // tokens per preparation block (256 threads each)

// Bucketing blocks: each computes the whole bucketing (bitmaps, counts,
// scans) from the routing input and stores one share of its results (a
// wave of tokens' entries, every nb-th expert's items), so the scattered
// stores spread over nb CUs instead of queueing on one.
__host__ __device__ constexpr uint32_t pf_bucket_blocks(uint32_t n) {
  return (n + 63) / 64 < 8 ? (n + 63) / 64 : 8;
}
constexpr uint32_t kPfPart8 = kPfMaxGroupsK * 128 / 8;   // 8-input partial sums of one row (H <= 16384)

// Token t's x row -> MFMA-ready bf16 hi (and lo for fp32 input) and its
// group sums over what the MFMAs see (hi + lo), in row t of x_hi / x_lo /
// xsum. 256 threads (tid); part8: kPfPart8 floats of LDS. Every thread of
// the block reaches the barrier (live = false: no work).
__device__ __forceinline__ void pf_prep_token(const PfArgs& a, uint32_t t, bool live, uint32_t tid, float* part8) {
  const uint32_t H = a.g.hidden, G = a.g.group;
  const bool x_bf16 = a.x_bf16;
  const float* const gate = a.gate;
  float gdot = 0.f;  // this thread's share of the shared-expert gate score gate . x_t
  if (live) {
    for (uint32_t k0 = tid * 8; k0 < H; k0 += 256 * 8) {
      float f[8];
      if (x_bf16) {
        const u32x4 v = *reinterpret_cast<const u32x4*>(reinterpret_cast<const uint16_t*>(a.x) + (size_t)t * H + k0);
        const uint32_t w4[4] = {v.x, v.y, v.z, v.w};
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          f[2 * i] = __uint_as_float(w4[i] << 16);
          f[2 * i + 1] = __uint_as_float(w4[i] & 0xFFFF0000u);
        }
      } else {
        const f32x4* p = reinterpret_cast<const f32x4*>(reinterpret_cast<const float*>(a.x) + (size_t)t * H + k0);
        const f32x4 u = p[0], v = p[1];
        f[0] = u.x, f[1] = u.y, f[2] = u.z, f[3] = u.w, f[4] = v.x, f[5] = v.y, f[6] = v.z, f[7] = v.w;
      }
      if (gate) {
        const f32x4* gp = reinterpret_cast<const f32x4*>(gate + k0);
        const f32x4 g0 = gp[0], g1 = gp[1];
        const float gv[8] = {g0.x, g0.y, g0.z, g0.w, g1.x, g1.y, g1.z, g1.w};
#pragma unroll
        for (int i = 0; i < 8; ++i) gdot = __builtin_fmaf(gv[i], f[i], gdot);
      }
      u32x4 hi, lo;
      split_f32(f, hi, lo);
      *reinterpret_cast<u32x4*>(a.x_hi + (size_t)t * H + k0) = hi;
      if (!x_bf16) *reinterpret_cast<u32x4*>(a.x_lo + (size_t)t * H + k0) = lo;
      // Partial sum of these 8 inputs as the MFMA sees them.
      const uint32_t hv[4] = {hi.x, hi.y, hi.z, hi.w}, lv[4] = {lo.x, lo.y, lo.z, lo.w};
      float p = 0.f;
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        p += __uint_as_float(hv[i] << 16) + __uint_as_float(hv[i] & 0xFFFF0000u);
        if (!x_bf16) p += __uint_as_float(lv[i] << 16) + __uint_as_float(lv[i] & 0xFFFF0000u);
      }
      part8[k0 / 8] = p;
    }
  }
  __syncthreads();
  if (live) {
    const uint32_t ng = H / G, per = G / 8;
    for (uint32_t g = tid; g < ng; g += 256) {
      float sum = 0.f;
      for (uint32_t j = 0; j < per; ++j) sum += part8[g * per + j];
      a.xsum[(size_t)t * ng + g] = sum;
    }
  }
  if (gate) {
    // The 256 thread shares, summed in thread order.
    __syncthreads();
    part8[tid] = gdot;
    __syncthreads();
    if (live && tid == 0) {
      float sum = 0.f;
      for (uint32_t j = 0; j < 256; ++j) sum += part8[j];
      a.gscore[t] = sum;
    }
  }
}

// LDS of a bucketing block: col [E, cws] u32 (row stride cws = cw | 1,
// odd, so that the words of different experts spread over the LDS banks)
// then pre [E, cw] u16 (cw = ceil(n / 32)); the preparation blocks use the
// same memory as kPfPrepTokens rows of part sums.
__host__ __device__ constexpr uint32_t pf_route_bucket_lds(uint32_t E, uint32_t n) {
  return (E * (((n + 31) / 32) | 1u) * 4 + E * ((n + 31) / 32) * 2 + 15) / 16 * 16;
}
__host__ __device__ constexpr uint32_t pf_route_lds(uint32_t E, uint32_t n) {
  return pf_route_bucket_lds(E, n) > kPfPrepTokens * kPfPart8 * 4 ? pf_route_bucket_lds(E, n)
                                                                  : kPfPrepTokens * kPfPart8 * 4;
}

// Lane l - d's value (DPP row shift right; row_shr:d = 0x110 + d), 0 where
// the source lies before the 16-lane row or outside ROW_MASK.
template <int CTRL, int ROW_MASK = 0xF>
__device__ __forceinline__ uint32_t dpp_shr_u(uint32_t v) {
  return (uint32_t)__builtin_amdgcn_update_dpp(0, (int)v, CTRL, ROW_MASK, 0xF, false);
}

// Inclusive prefix sum over the wave: shifts by 1, 2, 4, 8 within each
// 16-lane row, then row 0's total into row 1 and row 2's into row 3
// (row_bcast:15), then rows 0-1's total into rows 2-3 (row_bcast:31).
__device__ __forceinline__ uint32_t wave_scan_incl(uint32_t v) {
  v += dpp_shr_u<0x111>(v);
  v += dpp_shr_u<0x112>(v);
  v += dpp_shr_u<0x114>(v);
  v += dpp_shr_u<0x118>(v);
  v += dpp_shr_u<0x142, 0xA>(v);
  v += dpp_shr_u<0x143, 0xC>(v);
  return v;
}

// Per-expert counts from the column bitmaps: tpe threads per expert
// (adjacent lanes), each over PER >= ceil(cw / tpe) words. Every word read
// is issued unconditionally (addresses clamped into the bitmap, values
// masked), so the reads overlap instead of one LDS round trip each.
template <uint32_t PER>
__device__ __forceinline__ void pf_count_words(const uint32_t* col, uint16_t* pre, uint32_t* scnt, uint32_t* snch,
                                               uint32_t E, uint32_t cw, uint32_t cws, uint32_t tpe, uint32_t tid) {
  const uint32_t e = tid / tpe, j = tid % tpe, per = (cw + tpe - 1) / tpe;
  const uint32_t ec = e < E ? e : E - 1u;
  uint32_t pc[PER], loc = 0;
#pragma unroll
  for (uint32_t i = 0; i < PER; ++i) {
    const uint32_t c = j * per + i;
    const uint32_t v = col[ec * cws + (c < cw ? c : cw - 1u)];
    pc[i] = (e < E && i < per && c < cw) ? __popc(v) : 0u;
    loc += pc[i];
  }
  // Inclusive scan over the tpe lanes of the expert (aligned groups of 2
  // or 4 within a 16-lane row): DPP shifts by 1 and 2.
  uint32_t incl = loc;
  const uint32_t t1 = dpp_shr_u<0x111>(incl);
  if (j >= 1) incl += t1;
  if (tpe == 4) {
    const uint32_t t2 = dpp_shr_u<0x112>(incl);
    if (j >= 2) incl += t2;
  }
  if (e < E) {
    uint32_t run = incl - loc;
#pragma unroll
    for (uint32_t i = 0; i < PER; ++i) {
      const uint32_t c = j * per + i;
      if (i < per && c < cw) pre[e * cw + c] = (uint16_t)run;
      run += pc[i];
    }
    if (j == tpe - 1) {
      scnt[e] = incl;
      snch[e] = (incl + kPfMC - 1) / kPfMC;
    }
  }
}

// Work-list index of routed item i: the routed items in expert order, cut
// into 8 XCD ranges [nr x / 8, nr (x + 1) / 8); with ns shared-expert
// items in the list, range x's shared items follow its routed ones.
__device__ __forceinline__ uint32_t pf_fidx(uint32_t i, uint32_t nr, uint32_t ns) {
  return i + ns * ((8u * (i + 1u) - 1u) / nr) / 8u;
}

struct PfPlace {
  const uint32_t* col;
  const uint16_t* pre;
  const uint32_t* offs;
  const uint32_t* sibase;
  uint32_t E, cw, cws, k, nr, ns;
};

// Token tid's entries (slots s < KM, ids past k are INT32_MAX): position =
// the expert's offset + the tokens before tid that chose the same expert
// (its row in the expert's items); rank among the token's experts in
// ascending expert order = how many of its ids are smaller. Stores the
// (position, weight) pair at the rank and the token id into its item row.
template <uint32_t KM, bool SHARED>
__device__ __forceinline__ void pf_place(const PfArgs& a, const PfPlace& p, const int32_t (&ex)[kPfMaxK],
                                         const float (&wt)[kPfMaxK], uint32_t tid) {
  // Every slot's LDS reads first (an invalid slot reads expert 0's words
  // and stores nothing), so they take one round trip, not one per slot.
  bool ok[KM];
  uint32_t pv[KM], cv[KM], ov[KM], sv[KM];
#pragma unroll
  for (uint32_t s = 0; s < KM; ++s) {
    ok[s] = s < p.k && ex[s] >= 0 && (uint32_t)ex[s] < p.E;
    const uint32_t e = ok[s] ? (uint32_t)ex[s] : 0u;
    pv[s] = p.pre[e * p.cw + (tid >> 5)];
    cv[s] = p.col[e * p.cws + (tid >> 5)];
    ov[s] = p.offs[e];
    sv[s] = p.sibase[e];
  }
#pragma unroll
  for (uint32_t s = 0; s < KM; ++s) {
    const uint32_t row = pv[s] + __popc(cv[s] & ((1u << (tid & 31)) - 1u));
    uint32_t r = 0;
#pragma unroll
    for (uint32_t q = 0; q < KM; ++q) r += ex[q] < ex[s] ? 1u : 0u;
    r = min(r, p.k - 1);  // a duplicated expert (already reported) stays in range
    const uint32_t it = sv[s] + row / kPfMC;
    if (ok[s]) {
      a.tok_pw[tid * p.k + r] = make_uint2(ov[s] + row, __float_as_uint(wt[s]));
      a.item_tok[(SHARED ? pf_fidx(it, p.nr, p.ns) : it) * kPfMC + row % kPfMC] = tid;
    }
  }
}

__global__ __launch_bounds__(1024) void k_pf_route(PfArgs a) {
  extern __shared__ __attribute__((aligned(16))) uint8_t pf_dyn[];
  // Every argument either role reads, in scalar registers in one batch
  // before the role branch (the compiler would otherwise load them lazily,
  // a dependent round trip per branch level; the argument block is not in
  // the cache when the kernel starts).
  asm volatile("" ::"s"(a.n_tokens), "s"(a.k), "s"(a.E), "s"(a.idx), "s"(a.w), "s"(a.err), "s"(a.trace),
               "s"(a.items), "s"(a.n_items), "s"(a.item_tok), "s"(a.tok_pw), "s"(a.xr), "s"(a.shared),
               "s"(a.shared_in_list));
  asm volatile("" ::"s"(a.g.hidden), "s"(a.g.group), "s"(a.x_bf16), "s"(a.x), "s"(a.gate), "s"(a.x_hi),
               "s"(a.x_lo), "s"(a.xsum), "s"(a.gscore));
  const uint32_t tid = threadIdx.x;
  const uint32_t nb = pf_bucket_blocks(a.n_tokens), bb = blockIdx.x;
  if (bb >= nb) {
    const uint32_t sub = tid >> 8, t = (bb - nb) * kPfPrepTokens + sub;
    pf_prep_token(a, t, t < a.n_tokens, tid & 255u, reinterpret_cast<float*>(pf_dyn) + sub * kPfPart8);
    return;
  }
  PF_STAMP(0);
  const uint32_t n = a.n_tokens, k = a.k, E = a.E;
  const uint32_t cw = (n + 31) / 32, cws = cw | 1u;
  // col[e][c]: bit (t & 31) set when token 32c + (t & 31) chose expert e;
  // pre[e][c]: tokens before 32c that chose e.
  uint32_t* const col = reinterpret_cast<uint32_t*>(pf_dyn);
  uint16_t* const pre = reinterpret_cast<uint16_t*>(pf_dyn + E * cws * 4);
  __shared__ uint32_t offs[kPfMaxExperts];
  __shared__ uint32_t s_nr;  // routed work items
  // Thread t owns token t: its k experts and weights stay in registers
  // (one read of the routing input), validated here.
  int32_t ex[kPfMaxK];
  float wt[kPfMaxK];
  const bool tok = tid < n;
  bool bad = false;
#pragma unroll
  for (uint32_t s = 0; s < kPfMaxK; ++s) {
    ex[s] = INT32_MAX;  // past k: above every expert id (out of range, never smaller)
    wt[s] = 0.f;
  }
  const bool per_entry = k <= 8;  // entries placed one lane each (below); else per token
  const bool vec = (k & 3) == 0 && ((reinterpret_cast<uintptr_t>(a.idx) | reinterpret_cast<uintptr_t>(a.w)) & 15) == 0;
  if (tok && vec) {
    // A token's k ids / weights are contiguous and 16-byte aligned: read
    // them four at a time.
    const int4* ip = reinterpret_cast<const int4*>(a.idx + tid * k);
    const float4* wp = reinterpret_cast<const float4*>(a.w + tid * k);
#pragma unroll
    for (uint32_t q = 0; q < kPfMaxK / 4; ++q)
      if (4 * q < k) {
        const int4 iv = ip[q];
        ex[4 * q] = iv.x, ex[4 * q + 1] = iv.y, ex[4 * q + 2] = iv.z, ex[4 * q + 3] = iv.w;
        if (!per_entry) {  // the per-token placement's weights
          const float4 wv = wp[q];
          wt[4 * q] = wv.x, wt[4 * q + 1] = wv.y, wt[4 * q + 2] = wv.z, wt[4 * q + 3] = wv.w;
        }
      }
  } else if (tok) {
#pragma unroll
    for (uint32_t s = 0; s < kPfMaxK; ++s)
      if (s < k) {
        ex[s] = a.idx[tid * k + s];
        if (!per_entry) wt[s] = a.w[tid * k + s];
      }
  }
  // Entry placement for k <= 8, one lane per (token, slot): thread tid
  // places slot pslot of token ptok (token wave bb + nb (tid / 512), eight
  // lanes per token); its id and weight and its token's ids (for the rank)
  // are loaded here with the rest of the routing input.
  const uint32_t ptok = 64u * (bb + nb * (tid >> 9)) + ((tid & 511u) >> 3), pslot = tid & 7u;
  const bool plive = per_entry && ptok < n && pslot < k;
  int32_t pid[8];
  int32_t pex = INT32_MAX;
  float pwt = 0.f;
#pragma unroll
  for (uint32_t q = 0; q < 8; ++q) pid[q] = INT32_MAX;
  if (plive) {
    pex = a.idx[ptok * k + pslot];
    pwt = a.w[ptok * k + pslot];
    if (vec) {
      const int4* ip = reinterpret_cast<const int4*>(a.idx + ptok * k);
#pragma unroll
      for (uint32_t q = 0; q < 2; ++q)
        if (4 * q < k) {
          const int4 iv = ip[q];
          pid[4 * q] = iv.x, pid[4 * q + 1] = iv.y, pid[4 * q + 2] = iv.z, pid[4 * q + 3] = iv.w;
        }
    } else {
#pragma unroll
      for (uint32_t q = 0; q < 8; ++q)
        if (q < k) pid[q] = a.idx[ptok * k + q];
    }
  }
  // The bitmaps cleared while the routing input is in flight (the block
  // size is the launch bound: no kernel-argument load for blockDim).
  for (uint32_t i = tid; i < E * cws; i += 1024u) col[i] = 0;
#pragma unroll
  for (uint32_t s = 0; s < kPfMaxK; ++s)
    if (tok && s < k) bad |= ex[s] < 0 || (uint32_t)ex[s] >= E;
  __syncthreads();
  PF_STAMP(1);
  // No returned value: an expert twice in one token shows as a bitmap
  // total below n k (checked with the scans).
  if (tok && k <= 8) {
    // Lane l starts at slot l mod 8 (slots past k hold INT32_MAX), so the
    // lanes that hit one word together (the same expert in the same slot,
    // such as a hot expert in slot 0) are spread over the 8 instructions.
    int32_t rx[8];
#pragma unroll
    for (uint32_t s = 0; s < 8; ++s) rx[s] = ex[s];
#pragma unroll
    for (uint32_t b = 1; b < 8; b <<= 1) {
      const bool sh = (tid & b) != 0;
      int32_t t[8];
#pragma unroll
      for (uint32_t s = 0; s < 8; ++s) t[s] = sh ? rx[(s + b) & 7] : rx[s];
#pragma unroll
      for (uint32_t s = 0; s < 8; ++s) rx[s] = t[s];
    }
#pragma unroll
    for (uint32_t s = 0; s < 8; ++s)
      if (rx[s] >= 0 && (uint32_t)rx[s] < E) atomicOr(&col[rx[s] * cws + (tid >> 5)], 1u << (tid & 31));
  } else if (tok) {
#pragma unroll
    for (uint32_t s = 0; s < kPfMaxK; ++s) {
      if (s >= k || ex[s] < 0 || (uint32_t)ex[s] >= E) continue;
      atomicOr(&col[ex[s] * cws + (tid >> 5)], 1u << (tid & 31));
    }
    if (bad) *a.err = 2u;
  }
  __syncthreads();
  PF_STAMP(2);
  __shared__ uint32_t scnt[kPfMaxExperts], snch[kPfMaxExperts], sibase[kPfMaxExperts];
  {
    // TPE = 4 threads per expert (2 above 256 experts), adjacent lanes of
    // one wave, each over a share of the expert's bitmap words: popcounts,
    // an exclusive scan across the TPE, then the running counts before
    // each word.
    static_assert(kPfMaxTokens / 32 <= 2 * 16 && 2 * kPfMaxExperts <= 1024 && 4 * 256 <= 1024, "count split");
    const uint32_t tpe = E <= 256 ? 4u : 2u;
    const uint32_t per = (cw + tpe - 1) / tpe;
    if (per <= 4)
      pf_count_words<4>(col, pre, scnt, snch, E, cw, cws, tpe, tid);
    else if (per <= 8)
      pf_count_words<8>(col, pre, scnt, snch, E, cw, cws, tpe, tid);
    else
      pf_count_words<16>(col, pre, scnt, snch, E, cw, cws, tpe, tid);
  }
  __syncthreads();
  PF_STAMP(3);
  // Wave 0: exclusive scans of the counts (entry offsets) and of the items
  // per expert (work-list bases), 8 experts per lane and a DPP scan.
  if (tid < 64) {
    constexpr int EPL = kPfMaxExperts / 64;
    uint32_t c8[EPL], n8[EPL], ca = 0, na = 0;
#pragma unroll
    for (int q = 0; q < EPL; ++q) {
      const uint32_t e = tid * EPL + q;
      c8[q] = e < E ? scnt[e] : 0u;
      n8[q] = e < E ? snch[e] : 0u;
      ca += c8[q];
      na += n8[q];
    }
    const uint32_t ci = wave_scan_incl(ca), ni = wave_scan_incl(na);  // inclusive scans over lanes
    uint32_t co = ci - ca, no = ni - na;
#pragma unroll
    for (int q = 0; q < EPL; ++q) {
      const uint32_t e = tid * EPL + q;
      if (e < E) {
        offs[e] = co;
        sibase[e] = no;
      }
      co += c8[q];
      no += n8[q];
    }
    if (tid == 63) {
      s_nr = ni;
      if (bb == 0 && ci != n * k) *a.err = 2u;  // a duplicated (or invalid) expert id
    }
  }
  __syncthreads();
  PF_STAMP(4);
  // Work-list order: the routed items in expert order, cut into 8 XCD
  // ranges [nr x / 8, nr (x + 1) / 8) (the GEMMs give range x to XCD x);
  // a shared expert's items (all n tokens, entries n k + t, expert id E)
  // are spread over the ranges, ns x / 8 .. ns (x + 1) / 8 after range x's
  // routed items, so that no XCD takes all of them.
  const uint32_t nr = s_nr;
  const uint32_t ns = a.shared && a.shared_in_list ? (n + kPfMC - 1) / kPfMC : 0u;
  auto fidx = [=](uint32_t i) { return pf_fidx(i, nr, ns); };
  // Shared-expert items on wave wi + 1 and routed items on wave wi (threads
  // rotated so that the wave holds the block's first 64 of them): when
  // nb > 1 neither places tokens (the waves bb, bb + nb, ... do).
  const uint32_t wi = (bb + nb / 2) & 15u, it = (tid + 1024u - 64u * wi) & 1023u;
  const uint32_t is = (tid + 1024u - 64u * ((wi + 1u) & 15u)) & 1023u;
  if (bb == 0 && tid < 9) a.xr[tid] = nr * tid / 8u + ns * tid / 8u;
  if (bb == 0 && tid == 0) *a.n_items = nr + ns;
  for (uint32_t j = bb + nb * is; j < ns; j += nb * 1024u) {
    const uint32_t x = (8u * (j + 1u) - 1u) / ns, f = nr * (x + 1u) / 8u + j;
    const uint32_t cnt = min(kPfMC, n - j * kPfMC);
    a.items[2 * f] = E;
    a.items[2 * f + 1] = (n * k + j * kPfMC) | (cnt << 16);
    for (uint32_t r = 0; r < cnt; ++r) a.item_tok[f * kPfMC + r] = j * kPfMC + r;
  }
  if (a.shared && !a.shared_in_list) {
    // A list of its own for 4-bit GEMM launches (routed bits 3).
    const uint32_t ms = (n + kPfMC - 1) / kPfMC;
    for (uint32_t j = bb + nb * is; j < ms; j += nb * 1024u) {
      const uint32_t cnt = min(kPfMC, n - j * kPfMC);
      a.sitems[2 * j] = 0;
      a.sitems[2 * j + 1] = (n * k + j * kPfMC) | (cnt << 16);
      for (uint32_t r = 0; r < cnt; ++r) a.sitem_tok[j * kPfMC + r] = j * kPfMC + r;
    }
    if (bb == 0 && tid < 9) a.sxr[tid] = ms * tid / 8u;
    if (bb == 0 && tid == 0) *a.sn_items = ms;
  }
  if (bb + nb * it < E) {
    const uint32_t e = bb + nb * it;
    const uint32_t cnt = scnt[e], nch = snch[e], off = offs[e], ibase = sibase[e];
    for (uint32_t c = 0; c < nch; ++c) {
      const uint32_t f = fidx(ibase + c);
      a.items[2 * f] = e;
      a.items[2 * f + 1] = (off + c * kPfMC) | (min(kPfMC, cnt - c * kPfMC) << 16);
    }
    // Rows past the count of the expert's last item are not written: the
    // GEMM clamps whatever they hold to a token id (their results are
    // dropped).
  }
  // Every entry places itself: position = the expert's offset + the tokens
  // before t that chose the same expert (its row in the expert's items);
  // rank r among t's experts in ascending expert order = how many of t's
  // experts are smaller. The token writes its entry positions and weights
  // in that order (token-major), and its id into its items' row slots.
  // Block bb places the tokens of waves bb, bb + nb, ...: for k <= 8 one
  // lane per entry, else one thread per token.
  if (per_entry) {
    if (plive && pex >= 0 && (uint32_t)pex < E) {
      const uint32_t e = (uint32_t)pex, wv = ptok >> 5;
      const uint32_t row = pre[e * cw + wv] + __popc(col[e * cws + wv] & ((1u << (ptok & 31)) - 1u));
      uint32_t r = 0;
#pragma unroll
      for (uint32_t q = 0; q < 8; ++q) r += pid[q] < pex ? 1u : 0u;
      r = min(r, k - 1);  // a duplicated expert (already reported) stays in range
      a.tok_pw[ptok * k + r] = make_uint2(offs[e] + row, __float_as_uint(pwt));
      const uint32_t it = sibase[e] + row / kPfMC;
      a.item_tok[(ns ? fidx(it) : it) * kPfMC + row % kPfMC] = ptok;
    }
  } else if (tok && (tid >> 6) % nb == bb) {
    const PfPlace p{col, pre, offs, sibase, E, cw, cws, k, nr, ns};
    if (ns) pf_place<kPfMaxK, true>(a, p, ex, wt, tid);
    else pf_place<kPfMaxK, false>(a, p, ex, wt, tid);
  }
  PF_STAMP(5);
  __syncthreads();
  __builtin_amdgcn_s_waitcnt(0);
  PF_STAMP(6);
}

// ---------------------------------------------------------------------------
// Persistent pipelined GEMM (k_pf_mm). One block of 8 waves per CU loops
// over work units (item, NCOL output columns); a unit is K / 256 chunks,
// and the block's chunk sequence streams through an S-stage LDS ring:
// global_load_lds copies each chunk's weight codes, bf16 scales/biases,
// A rows (MFMA-ready bf16, already permuted) and A group sums straight
// into LDS (no registers), S - 1 chunks ahead of the MFMAs. Each wave
// waits only for its own copies of the chunk it is about to use
// (s_waitcnt vmcnt), then one barrier makes all waves' copies visible.
// Waves 0-3 and 4-7 take the lower and upper K half of each chunk for the
// same columns (two waves per SIMD, so one's VALU work overlaps the other's
// MFMAs) and add their sums through LDS when a unit ends. Swizzles: weight rows XOR (4-bit) or rotate (3-bit) their 16-byte parts
// by the row, A rows XOR their parts by the row, so the 16 lanes of an
// MFMA operand read different banks.
// ---------------------------------------------------------------------------

// A loop-invariant 32-bit lane offset, made opaque at its use so that the
// compiler adds it to the scalar base in the copy instruction itself
// (global_load_lds with a scalar address and a 32-bit vector offset)
// instead of keeping it widened to 64 bits and adding it with a vector
// instruction before every copy.
__device__ __forceinline__ uint32_t pf_voff(uint32_t o) {
  asm volatile("" : "+v"(o));
  return o;
}

// Position of natural index i (0..7) of an 8-block in the MFMA order
// [v0, v4, v1, v5, v2, v6, v3, v7].
__device__ __forceinline__ uint32_t perm8_pos(uint32_t i) { return i < 4 ? 2 * i : 2 * (i - 4) + 1; }

template <int BITS, int G, int MODE, bool SPLIT, int KU = 0, int NWD = 0>
struct PfMM {
  // Compute waves: 4 column waves x 2 K halves. With NWD > 0, NWD more
  // waves only copy (their issue stalls on the memory pipeline never delay
  // the MFMA work); else the compute waves copy too.
  static constexpr int NWC = 8;
  static constexpr int NWT = NWC + NWD;               // waves per block
  static constexpr int NW = NWD > 0 ? NWD : NWC;      // copying waves
  static constexpr int KC = kPfKC;                    // inputs per chunk
  static constexpr int CG = KC / G;                   // groups per chunk
  static constexpr int CGW = CG / 2;                  // groups per wave (its K half of the chunk)
  static constexpr int NU = G / 32;                   // MFMA steps per group
  // MODE 0: gate/up (bf16 x, or hi + lo); MODE 1: down over bf16 hi + lo
  // A rows (the dense qmm); MODE 2: down over fp16 activations (SPLIT false).
  static constexpr bool F16 = MODE == 2;
  static constexpr int NMAT = MODE == 0 ? 2 : 1;      // weight matrices per column
  static constexpr int CT = MODE == 0 ? 1 : 4;        // 16-column tiles per wave
  static constexpr int NCOL = 64 * CT;                // output columns per unit
  static constexpr int ROWS = NMAT * NCOL;            // weight rows per unit
  static constexpr int RB = KC * BITS / 8;            // code bytes per row and chunk
  static constexpr int PPR = RB / 16;                 // 16-byte parts per row
  // Scales and biases: per chunk in each stage ([row][array][CG] bf16), or,
  // with KU = K > 0, for a whole unit in one of two unit buffers ([row][array]
  // [K / G], rows padded by 16 bytes against bank conflicts), copied once per
  // unit in 16-byte pieces instead of 8 small pieces per chunk.
  static constexpr bool USB = KU > 0;
  static constexpr int NGU = USB ? KU / G : CG;       // groups per scale row in LDS
  static constexpr int SB_BYTES = 2 * CG;             // scale (or bias) bytes per row and chunk
  static constexpr int SB_SZ = SB_BYTES >= 16 ? 16 : 4;
  static constexpr int SB_PIECES = SB_BYTES / SB_SZ;  // per row and array
  static constexpr int SB_ROW = USB ? 4 * NGU + 16 : 2 * SB_BYTES;  // LDS bytes per scale row
  static constexpr int S = MODE == 0 ? (SPLIT || USB ? 3 : 4) : 2;
  // Copy pieces per chunk and category; every wave copies an equal,
  // contiguous share (so every wave issues the same number of copies).
  static constexpr int P_BQ = ROWS * PPR;             // 16-byte code parts
  static constexpr int P_BS = USB ? 0 : ROWS * 2 * SB_PIECES;  // scale / bias pieces
  static constexpr int P_A = kPfMC * KC * 2 / 16;     // 16-byte A parts (per half)
  static constexpr int P_XS = USB ? 0 : kPfMC * CG;  // group sums ([group][row] per chunk)
  static constexpr int P_US = USB ? ROWS * (2 * (2 * NGU / 16) + 1) : 0;  // unit scale slots (16 B, one pad per row)
  static constexpr int N_BQ = (P_BQ / NW + 63) / 64;  // copy instructions per wave
  static constexpr int N_BS = (P_BS / NW + 63) / 64;
  static constexpr int N_A = P_A / NW / 64;           // one row pair (m, m + 16) each
  static constexpr int N_XS = (P_XS / NW + 63) / 64;
  static constexpr int N_US = (P_US / NW + 63) / 64;
  // With USB the A group sums also come once per unit: [row][NGU] f32.
  static constexpr int P_UXS = USB ? kPfMC * NGU / 4 : 0;  // 16-byte pieces
  static constexpr int N_UXS = (P_UXS / NW + 63) / 64;
  static constexpr int D = N_BQ + N_BS + N_A * (SPLIT ? 2 : 1) + N_XS;  // per chunk
  static constexpr int DU = N_US + N_UXS;                                 // per unit
  // LDS layout of one stage (bytes). A rows sit in pairs: row m at slot
  // 2 (m % 16) + m / 16, so one copy instruction moves rows m and m + 16.
  static constexpr int OFF_BQ = 0;
  static constexpr int OFF_BS = OFF_BQ + P_BQ * 16;
  static constexpr int OFF_AH = OFF_BS + P_BS * SB_SZ;
  static constexpr int OFF_AL = OFF_AH + P_A * 16;
  static constexpr int OFF_XS = OFF_AL + (SPLIT ? P_A * 16 : 0);
  static constexpr int STAGE = OFF_XS + P_XS * 4;
  static constexpr int OFF_UXS = ROWS * SB_ROW;           // group sums in a unit buffer
  static constexpr int UBUF = USB ? OFF_UXS + P_UXS * 16 : 0;  // one unit buffer, after the stages
  // Gate/up with G <= 64: the column waves' activation row sums of the
  // last finished unit ([column wave][32 rows] f32), after the unit buffers.
  static constexpr bool ASUM = MODE == 0 && G <= 64;
  static constexpr int OFF_PS = S * STAGE + 2 * UBUF;
  // Gate/up: the token ids of two units' rows (A rows and group sums are
  // gathered from the per-token arrays), one buffer per unit parity.
  static constexpr bool GATHER = MODE == 0;
  static constexpr int OFF_TOK = OFF_PS + (ASUM ? 4 * kPfMC * 4 : 0);
  // Accumulators per lane, exchanged between the K halves at a unit's end:
  // each half finishes rows r = 2 kh, 2 kh + 1 of every 4-row group and
  // parks the other half's NT / 2 partial sums, in an area of its own when
  // the LDS has room for it (then a unit end takes one block barrier), else
  // in the stage just read (one more barrier, so that no wave still reads
  // it).
  static constexpr int NT = NMAT * CT * 2 * 4;
  static constexpr int EX_BYTES = 4 * NT * 64 * 4;
  static constexpr int OFF_EX = OFF_TOK + (GATHER ? 2 * kPfMC * 4 : 0);
  static constexpr bool EXD = OFF_EX + EX_BYTES <= 160 * 1024;
  static constexpr int LDS = OFF_EX + (EXD ? EX_BYTES : 0);
  // Per-lane row offsets of one unit's group-sum copies.
  static constexpr int NXR = USB ? N_UXS : N_XS;
  static_assert(CG % 2 == 0, "K halves");
  static_assert(P_BQ % NW == 0 && P_BS % NW == 0 && P_XS % NW == 0 && P_US % NW == 0 && P_UXS % NW == 0,
                "equal shares");
  static_assert(!USB || NGU % 4 == 0, "unit group sums in 16-byte pieces");
  static_assert(!USB || ((NGU / 4) & (NGU / 4 - 1)) == 0, "unit group-sum rows: a power-of-two piece count (XOR swizzle)");
  static_assert(N_A * NW * 64 == P_A && P_A == 16 * 64, "one row pair per A copy");
  static_assert((S - 2) * D + DU <= 63, "vmcnt range");
  static_assert(NWD == 0 || (MODE == 0 && USB), "copy waves: unit-staged gate/up only");
  static_assert(!F16 || !SPLIT, "fp16 activations are one half");
  static_assert(LDS <= 160 * 1024, "LDS per CU");
  static_assert(EXD || EX_BYTES <= STAGE, "accumulator exchange fits a stage");

  static_assert(!USB || (2 * NGU) % 16 == 0, "unit scale rows in 16-byte pieces");
};

// 8 codes of one 4-bit u32 as bf16 (128 + q), order [q0,q4,q1,q5,q2,q6,q3,q7],
// in 7 instructions: the low and high nibbles of each byte, then one byte
// permute per output word pairing them with 0x43 bytes (c43 = 0x43434343).
// Builtins only: inline asm feeding an MFMA hides the VALU-to-MFMA
// dependency from the compiler's hazard checks.
__device__ __forceinline__ u32x4 codes_bf16_4p(uint32_t d, uint32_t c43) {
  const uint32_t lo = d & 0x0F0F0F0Fu;         // q0, q2, q4, q6
  const uint32_t hi = (d >> 4) & 0x0F0F0F0Fu;  // q1, q3, q5, q7
  u32x4 r;
  r.x = __builtin_amdgcn_perm(c43, lo, 0x04020400u);  // (q0, q4)
  r.y = __builtin_amdgcn_perm(c43, hi, 0x04020400u);  // (q1, q5)
  r.z = __builtin_amdgcn_perm(c43, lo, 0x04030401u);  // (q2, q6)
  r.w = __builtin_amdgcn_perm(c43, hi, 0x04030401u);  // (q3, q7)
  return r;
}

// The MFMA work of one chunk for one wave: groups gl0 .. gl0 + CGW - 1 of
// the stage at st, NTL 16-row tiles, into tot. Straight-line code (no
// branches), so the scheduler can overlap LDS reads with MFMAs.
template <int BITS, int G, int MODE, bool SPLIT, int KU, int NTL>
__device__ __forceinline__ void pf_chunk_seq(const uint8_t* st, const uint8_t* sbb, const float* uxs, uint32_t gofs, uint32_t gl0,
                                         uint32_t cw, uint32_t n, uint32_t q, uint32_t c43,
                                         f32x4 (&tot)[PfMM<BITS, G, MODE, SPLIT, KU>::NMAT][PfMM<BITS, G, MODE, SPLIT, KU>::CT][2]) {
  using C = PfMM<BITS, G, MODE, SPLIT, KU>;
#pragma unroll
  for (int gi = 0; gi < C::CGW; ++gi) {
    const uint32_t gl = gl0 + gi;
    uint32_t bw[C::NMAT][C::CT][C::NU];
    float s[C::NMAT][C::CT], cbias[C::NMAT][C::CT];
#pragma unroll
    for (int mt = 0; mt < C::NMAT; ++mt)
#pragma unroll
      for (int ct = 0; ct < C::CT; ++ct) {
        const uint32_t row = mt * C::NCOL + cw * 16 * C::CT + ct * 16 + n;
        const uint8_t* rb = st + C::OFF_BQ + row * C::RB;
        if (BITS == 4) {
          const uint32_t off = gl * (G / 2) + 4 * C::NU * q;  // byte offset in the chunk row
          const uint32_t slot = (off / 16) ^ (row & 7);
          const uint32_t* w = reinterpret_cast<const uint32_t*>(rb + slot * 16 + off % 16);
#pragma unroll
          for (int uu = 0; uu < C::NU; ++uu) bw[mt][ct][uu] = w[uu];
        } else {
          const uint32_t off = (gl * G + 8 * C::NU * q) * 3 / 8;  // 3*NU bytes
          constexpr int ND = (3 * C::NU + 6) / 4;
          uint32_t d[ND];
#pragma unroll
          for (int i = 0; i < ND; ++i) {
            const uint32_t dw = (off & ~3u) / 4 + i;  // dword index in the row (0 .. RB/4)
            const uint32_t part = min(dw / 4, (uint32_t)C::PPR - 1);
            const uint32_t slot = (part + C::PPR - row % C::PPR) % C::PPR;
            d[i] = *reinterpret_cast<const uint32_t*>(rb + slot * 16 + (dw % 4) * 4);
          }
          const uint32_t sh = (off & 3u) * 8;
#pragma unroll
          for (int uu = 0; uu < C::NU; ++uu) {
            const uint32_t bit = sh + 24 * uu;
            uint32_t lo = 0, hi = 0;
#pragma unroll
            for (int i = 0; i < ND; ++i) {
              if ((uint32_t)i == (bit >> 5)) lo = d[i];
              if ((uint32_t)i == (bit >> 5) + 1) hi = d[i];
            }
            bw[mt][ct][uu] = __builtin_amdgcn_alignbit(hi, lo, bit & 31) & 0xFFFFFFu;
          }
        }
        // Scales of the row, then biases: [row][array][NGU] at sbb; this chunk's
        // groups start at gofs.
        const uint16_t* sb = reinterpret_cast<const uint16_t*>(sbb + row * C::SB_ROW) + gofs;
        s[mt][ct] = bf16f(sb[gl]);
        cbias[mt][ct] = __builtin_fmaf(C::F16 ? -64.0f : -128.0f, s[mt][ct], bf16f(sb[C::NGU + gl]));
        if (C::F16) s[mt][ct] *= 64.0f;
      }
    u32x4 bq[C::NMAT][C::CT][C::NU];
#pragma unroll
    for (int mt = 0; mt < C::NMAT; ++mt)
#pragma unroll
      for (int ct = 0; ct < C::CT; ++ct)
#pragma unroll
        for (int uu = 0; uu < C::NU; ++uu) {
          if constexpr (C::F16)
            bq[mt][ct][uu] = BITS == 4 ? codes_f16_4p(bw[mt][ct][uu]) : codes_f16_3(bw[mt][ct][uu]);
          else
            bq[mt][ct][uu] = BITS == 4 ? codes_bf16_4p(bw[mt][ct][uu], c43) : codes_bf16_3(bw[mt][ct][uu]);
        }
#pragma unroll
    for (int t = 0; t < NTL; ++t) {
      f32x4 acc[C::NMAT][C::CT];
#pragma unroll
      for (int mt = 0; mt < C::NMAT; ++mt)
#pragma unroll
        for (int ct = 0; ct < C::CT; ++ct) acc[mt][ct] = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
      for (int uu = 0; uu < C::NU; ++uu) {
        const uint32_t part = (gl * G + 8 * C::NU * q + 8 * uu) / 8;
        const uint32_t aoff = (2 * n + t) * C::KC * 2 + ((part ^ n) * 16);
        const u32x4 ah = *reinterpret_cast<const u32x4*>(st + C::OFF_AH + aoff);
        u32x4 al;
        if (SPLIT) al = *reinterpret_cast<const u32x4*>(st + C::OFF_AL + aoff);
#pragma unroll
        for (int mt = 0; mt < C::NMAT; ++mt)
#pragma unroll
          for (int ct = 0; ct < C::CT; ++ct) {
            if constexpr (C::F16) {
              acc[mt][ct] = mfma_f16(ah, bq[mt][ct][uu], acc[mt][ct]);
            } else {
              acc[mt][ct] = mfma(ah, bq[mt][ct][uu], acc[mt][ct]);
              if (SPLIT) acc[mt][ct] = mfma(al, bq[mt][ct][uu], acc[mt][ct]);
            }
          }
      }
      // Group sums of rows 16t + 4q .. + 3: one read from the stage
      // ([group][row]), or four from the unit buffer ([row][NGU]).
      f32x4 xs;
      if constexpr (C::USB) {
        const float* xr = uxs + (16 * t + 4 * q) * C::NGU + gofs + gl;
        xs = f32x4{xr[0], xr[C::NGU], xr[2 * C::NGU], xr[3 * C::NGU]};
      } else {
        xs = *reinterpret_cast<const f32x4*>(st + C::OFF_XS + (gl * kPfMC + 16 * t + 4 * q) * 4);
      }
#pragma unroll
      for (int r = 0; r < 4; ++r)
#pragma unroll
        for (int mt = 0; mt < C::NMAT; ++mt)
#pragma unroll
          for (int ct = 0; ct < C::CT; ++ct)
            tot[mt][ct][t][r] =
                __builtin_fmaf(s[mt][ct], acc[mt][ct][r], __builtin_fmaf(cbias[mt][ct], xs[r], tot[mt][ct][t][r]));
    }
  }
}

// Codes of group gl, matrix row `row`, lane block q (NU words) from a stage.
template <int BITS, int G, int MODE, bool SPLIT, int KU>
__device__ __forceinline__ void pf_codes(const uint8_t* st, uint32_t row, uint32_t gl, uint32_t q,
                                         uint32_t (&bw)[PfMM<BITS, G, MODE, SPLIT, KU>::NU]) {
  using C = PfMM<BITS, G, MODE, SPLIT, KU>;
  const uint8_t* rb = st + C::OFF_BQ + row * C::RB;
  if (BITS == 4) {
    const uint32_t off = gl * (G / 2) + 4 * C::NU * q;  // byte offset in the chunk row
    const uint32_t slot = (off / 16) ^ (row & 7);
    const uint32_t* w = reinterpret_cast<const uint32_t*>(rb + slot * 16 + off % 16);
#pragma unroll
    for (int uu = 0; uu < C::NU; ++uu) bw[uu] = w[uu];
  } else {
    const uint32_t off = (gl * G + 8 * C::NU * q) * 3 / 8;  // 3*NU bytes
    constexpr int ND = (3 * C::NU + 6) / 4;
    uint32_t d[ND];
#pragma unroll
    for (int i = 0; i < ND; ++i) {
      const uint32_t dw = (off & ~3u) / 4 + i;  // dword index in the row (0 .. RB/4)
      const uint32_t part = min(dw / 4, (uint32_t)C::PPR - 1);
      const uint32_t slot = (part + C::PPR - row % C::PPR) % C::PPR;
      d[i] = *reinterpret_cast<const uint32_t*>(rb + slot * 16 + (dw % 4) * 4);
    }
    const uint32_t sh = (off & 3u) * 8;
#pragma unroll
    for (int uu = 0; uu < C::NU; ++uu) {
      const uint32_t bit = sh + 24 * uu;
      uint32_t lo = 0, hi = 0;
#pragma unroll
      for (int i = 0; i < ND; ++i) {
        if ((uint32_t)i == (bit >> 5)) lo = d[i];
        if ((uint32_t)i == (bit >> 5) + 1) hi = d[i];
      }
      bw[uu] = __builtin_amdgcn_alignbit(hi, lo, bit & 31) & 0xFFFFFFu;
    }
  }
}

// The MFMA work of one chunk for one wave, in phases: every LDS read of the
// chunk (codes, scales, A rows, group sums of all CGW groups and NTL tiles)
// is issued first, so the wave waits for LDS once per chunk instead of once
// per group; then the code conversions and MFMAs of all groups, then the
// dequant epilogue. Straight-line code (no branches).
template <int BITS, int G, int MODE, bool SPLIT, int KU, int NTL>
__device__ __forceinline__ void pf_chunk(const uint8_t* st, const uint8_t* sbb, const float* uxs, uint32_t gofs,
                                         uint32_t gl0, uint32_t cw, uint32_t n, uint32_t q, uint32_t c43,
                                         f32x4 (&tot)[PfMM<BITS, G, MODE, SPLIT, KU>::NMAT][PfMM<BITS, G, MODE, SPLIT, KU>::CT][2]) {
  using C = PfMM<BITS, G, MODE, SPLIT, KU>;
  if constexpr (MODE != 0) {
    pf_chunk_seq<BITS, G, MODE, SPLIT, KU, NTL>(st, sbb, uxs, gofs, gl0, cw, n, q, c43, tot);
  } else {
    constexpr int NG = C::CGW;
    uint32_t bw[NG][C::NMAT][C::CT][C::NU];
    uint16_t sr[NG][C::NMAT][C::CT], br[NG][C::NMAT][C::CT];
    u32x4 ah[NG][NTL][C::NU], al[NG][NTL][C::NU];
    f32x4 xs[NG][NTL];
#pragma unroll
    for (int gi = 0; gi < NG; ++gi) {
      const uint32_t gl = gl0 + gi;
#pragma unroll
      for (int mt = 0; mt < C::NMAT; ++mt)
#pragma unroll
        for (int ct = 0; ct < C::CT; ++ct) {
          const uint32_t row = mt * C::NCOL + cw * 16 * C::CT + ct * 16 + n;
          pf_codes<BITS, G, MODE, SPLIT, KU>(st, row, gl, q, bw[gi][mt][ct]);
          const uint16_t* sb = reinterpret_cast<const uint16_t*>(sbb + row * C::SB_ROW) + gofs;
          sr[gi][mt][ct] = sb[gl];
          br[gi][mt][ct] = sb[C::NGU + gl];
        }
#pragma unroll
      for (int t = 0; t < NTL; ++t) {
#pragma unroll
        for (int uu = 0; uu < C::NU; ++uu) {
          const uint32_t part = (gl * G + 8 * C::NU * q + 8 * uu) / 8;
          const uint32_t aoff = (2 * n + t) * C::KC * 2 + ((part ^ n) * 16);
          ah[gi][t][uu] = *reinterpret_cast<const u32x4*>(st + C::OFF_AH + aoff);
          if (SPLIT) al[gi][t][uu] = *reinterpret_cast<const u32x4*>(st + C::OFF_AL + aoff);
        }
        if constexpr (C::USB) {
          const float* xr = uxs + (16 * t + 4 * q) * C::NGU + gofs + gl;
          xs[gi][t] = f32x4{xr[0], xr[C::NGU], xr[2 * C::NGU], xr[3 * C::NGU]};
        } else {
          xs[gi][t] = *reinterpret_cast<const f32x4*>(st + C::OFF_XS + (gl * kPfMC + 16 * t + 4 * q) * 4);
        }
      }
    }
#pragma unroll
    for (int gi = 0; gi < NG; ++gi) {
      float s[C::NMAT][C::CT], cbias[C::NMAT][C::CT];
      u32x4 bq[C::NMAT][C::CT][C::NU];
#pragma unroll
      for (int mt = 0; mt < C::NMAT; ++mt)
#pragma unroll
        for (int ct = 0; ct < C::CT; ++ct) {
          s[mt][ct] = bf16f(sr[gi][mt][ct]);
          cbias[mt][ct] = __builtin_fmaf(-128.0f, s[mt][ct], bf16f(br[gi][mt][ct]));
#pragma unroll
          for (int uu = 0; uu < C::NU; ++uu)
            bq[mt][ct][uu] = BITS == 4 ? codes_bf16_4p(bw[gi][mt][ct][uu], c43) : codes_bf16_3(bw[gi][mt][ct][uu]);
        }
#pragma unroll
      for (int t = 0; t < NTL; ++t) {
        f32x4 acc[C::NMAT][C::CT];
#pragma unroll
        for (int mt = 0; mt < C::NMAT; ++mt)
#pragma unroll
          for (int ct = 0; ct < C::CT; ++ct) acc[mt][ct] = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
        for (int uu = 0; uu < C::NU; ++uu)
#pragma unroll
          for (int mt = 0; mt < C::NMAT; ++mt)
#pragma unroll
            for (int ct = 0; ct < C::CT; ++ct) {
              acc[mt][ct] = mfma(ah[gi][t][uu], bq[mt][ct][uu], acc[mt][ct]);
              if (SPLIT) acc[mt][ct] = mfma(al[gi][t][uu], bq[mt][ct][uu], acc[mt][ct]);
            }
#pragma unroll
        for (int r = 0; r < 4; ++r)
#pragma unroll
          for (int mt = 0; mt < C::NMAT; ++mt)
#pragma unroll
            for (int ct = 0; ct < C::CT; ++ct) {
              // With unit buffers the bias term sum_g cbias_g * xs_g is added
              // once per unit by fp32 MFMAs (pf_unit_bias).
              if constexpr (C::USB)
                tot[mt][ct][t][r] = __builtin_fmaf(s[mt][ct], acc[mt][ct][r], tot[mt][ct][t][r]);
              else
                tot[mt][ct][t][r] = __builtin_fmaf(s[mt][ct], acc[mt][ct][r],
                                                   __builtin_fmaf(cbias[mt][ct], xs[gi][t][r], tot[mt][ct][t][r]));
            }
      }
    }
  }
}

// The bias part of the dequant epilogue for a whole unit (gate/up with unit
// buffers): tot[m][c] += sum over this wave's groups g of (b - 128 s)[c][g] *
// xs[m][g], as v_mfma_f32_16x16x4_f32 (A = group sums [16 rows x 4 groups],
// B = column biases [4 groups x 16 columns]); the output layout is the
// 16x16 layout of the bf16 MFMAs. Wave K half kh owns groups
// c * CG + kh * CGW + gi of every chunk c.
template <int BITS, int G, int MODE, bool SPLIT, int KU>
__device__ __forceinline__ void pf_unit_bias(const uint8_t* ub, uint32_t nch, uint32_t kh, uint32_t cw,
                                             uint32_t lane, uint32_t ntiles,
                                             f32x4 (&tot)[PfMM<BITS, G, MODE, SPLIT, KU>::NMAT][PfMM<BITS, G, MODE, SPLIT, KU>::CT][2]) {
  using C = PfMM<BITS, G, MODE, SPLIT, KU>;
  static_assert(C::USB && C::CT == 1, "gate/up with unit buffers");
  const float* uxs = reinterpret_cast<const float*>(ub + C::OFF_UXS);
  const uint32_t r16 = lane & 15, kq = lane >> 4;
  const uint32_t nk = nch * C::CGW;  // groups of this K half
  for (uint32_t j = 0; j * 4 < nk; ++j) {
    const uint32_t e = 4 * j + kq;  // this lane's group slot
    const uint32_t g = (e / C::CGW) * C::CG + kh * C::CGW + e % C::CGW;
    float bb[C::NMAT];
#pragma unroll
    for (int mt = 0; mt < C::NMAT; ++mt) {
      const uint32_t row = mt * C::NCOL + cw * 16 + r16;
      const uint16_t* sb = reinterpret_cast<const uint16_t*>(ub + row * C::SB_ROW);
      bb[mt] = __builtin_fmaf(-128.0f, bf16f(sb[g]), bf16f(sb[C::NGU + g]));
    }
#pragma unroll
    for (int t = 0; t < 2; ++t) {
      if ((uint32_t)t >= ntiles) break;
      // Group g of row m sits in 16-byte slot (g / 4) ^ (m % XPR) of the row.
      constexpr uint32_t XPR = C::NGU / 4;
      const uint32_t m = 16 * t + r16;
      const float xa = uxs[m * C::NGU + ((((g >> 2) ^ (m & (XPR - 1))) << 2) | (g & 3u))];
#pragma unroll
      for (int mt = 0; mt < C::NMAT; ++mt)
        tot[mt][0][t] = __builtin_amdgcn_mfma_f32_16x16x4f32(xa, bb[mt], tot[mt][0][t], 0, 0, 0);
    }
  }
}

template <int BITS, int G, int MODE, bool SPLIT, int KU, int NWD>
__global__ __launch_bounds__(64 * (8 + NWD)) void k_pf_mm(PfArgs a, const uint32_t* __restrict__ items,
                                                          const uint32_t* __restrict__ n_items_p,
                                                          const uint32_t* __restrict__ xr) {
  using C = PfMM<BITS, G, MODE, SPLIT, KU, NWD>;
  extern __shared__ __attribute__((aligned(16))) uint8_t lds[];
  // The wave index is uniform: in a scalar register, the role branches
  // below are scalar branches and every LDS destination (M0) of a copy is
  // scalar arithmetic, with no vector-to-scalar move per copy.
  const uint32_t tid = threadIdx.x, lane = tid & 63, wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const uint32_t cw = wave & 3, kh = (wave >> 2) & 1;  // column wave, K half (compute waves)
  const bool copier = NWD == 0 || wave >= (uint32_t)C::NWC;   // issues copies
  const bool computer = NWD == 0 || wave < (uint32_t)C::NWC;  // runs MFMAs
  const uint32_t dw = NWD > 0 ? wave - C::NWC : wave;          // copy share index
  const uint32_t n = lane & 15, q = lane >> 4;
  // Every kernel argument used below is copied into a scalar local first,
  // so that nothing takes the argument block's address (that would move it
  // to scratch memory, and a wait on those loads would drain the copy
  // pipeline).
  const uint32_t K = MODE == 0 ? a.g.hidden : a.g.inter;
  const uint32_t N = MODE == 0 ? a.g.inter : a.g.hidden;
  const uint32_t ng = K / G, nch = K / C::KC, rowb = K * BITS / 8;
  const uint32_t ncb = N / C::NCOL;
  // XCD-aware schedule: block b runs on XCD b % 8. XCD group x takes the
  // contiguous item range [n x / 8, n (x + 1) / 8): items are in expert
  // order, so a hot expert's items (and an item's ncb column blocks) run
  // side by side on one XCD, and its weights and A rows are fetched into
  // that XCD's L2 once instead of once per item.
  const uint32_t nx = gridDim.x % 8 == 0 ? 8 : 1, per = gridDim.x / nx;
  const uint32_t xg = blockIdx.x % nx, lb = blockIdx.x / nx;
  // The ranges come from the bucketing launch (xr), or split evenly.
  const uint32_t n_items = *n_items_p;
  const uint32_t item_lo = xr && nx == 8 ? xr[xg] : n_items * xg / nx;
  const uint32_t item_hi = xr && nx == 8 ? xr[xg + 1] : n_items * (xg + 1) / nx;
  const uint32_t group_units = (item_hi - item_lo) * ncb;
  const uint32_t my_units = group_units > lb ? (group_units - lb + per - 1) / per : 0;
  const uint32_t total = my_units * nch;
  if (total == 0) return;
  // Gate/up: A rows are token rows of x_hi / x_lo / xsum, looked up by the
  // unit's token ids; down: entry rows of the activations, in place.
  const uint16_t* const ahi_src = MODE == 0 ? a.x_hi : a.act_hi;
  const uint16_t* const alo_src = MODE == 0 ? a.x_lo : a.act_lo;
  const float* const gsum = MODE == 0 ? a.xsum : a.asum;
  const uint8_t* const experts = a.experts;
  // Items of expert id E are the shared expert's (same geometry).
  const uint8_t* const shared = a.shared_in_list ? a.shared : nullptr;
  const uint32_t e_shared = a.E;
  const uint32_t* const item_tok = a.item_tok;
  const uint32_t last_tok = a.n_tokens - 1;
  const uint64_t stride = a.stride;
  uint16_t* const act_hi = a.act_hi;
  float* const down = a.down;
  float* const asum_out = a.asum;
  const uint64_t wo0 = a.g.w[MODE == 0 ? 0 : 2], wo1 = a.g.w[MODE == 0 ? 1 : 2];
  const uint64_t so0 = a.g.s[MODE == 0 ? 0 : 2], so1 = a.g.s[MODE == 0 ? 1 : 2];
  const uint64_t bo0 = a.g.b[MODE == 0 ? 0 : 2];
  // Lane offsets of the weight copies (fixed for the whole kernel; the
  // per-chunk part of the address is scalar).
  uint32_t off_bq[C::N_BQ], off_bs[C::N_BS > 0 ? C::N_BS : 1], off_us[C::N_US > 0 ? C::N_US : 1];
#pragma unroll
  for (int i = 0; i < C::N_BQ; ++i) {
    const uint32_t p = dw * (C::P_BQ / C::NW) + i * 64 + lane;
    const uint32_t row = p / C::PPR, sp = p % C::PPR;
    const uint32_t part = BITS == 4 ? (sp ^ (row & 7)) : (sp + row) % C::PPR;
    const uint32_t mat = row / C::NCOL;
    off_bq[i] = (uint32_t)(mat * (wo1 - wo0)) + (row % C::NCOL) * rowb + part * 16;
  }
#pragma unroll
  for (int i = 0; i < C::N_BS; ++i) {
    const uint32_t p = dw * (C::P_BS / C::NW) + i * 64 + lane;
    const uint32_t row = p / (2 * C::SB_PIECES), arr = (p / C::SB_PIECES) % 2, pc = p % C::SB_PIECES;
    const uint32_t mat = row / C::NCOL;
    // Biases follow scales at the same distance in both matrices.
    off_bs[i] = (uint32_t)(mat * (so1 - so0) + arr * (bo0 - so0)) + (row % C::NCOL) * ng * 2 + pc * C::SB_SZ;
  }
  // Unit scale slots: LDS slot p = (row, slot r of 2 UPC + 1) holds piece
  // r % UPC of the row's scales (r < UPC) or biases (r < 2 UPC); the last
  // slot pads the row and repeats piece 0. off_us = global offset from the
  // unit's scale base.
  constexpr uint32_t UPC = 2 * C::NGU / 16;  // pieces per row and array
#pragma unroll
  for (int i = 0; i < C::N_US; ++i) {
    const uint32_t p = dw * (C::P_US / C::NW) + i * 64 + lane;
    const uint32_t row = p / (2 * UPC + 1), r = p % (2 * UPC + 1);
    const uint32_t arr = r < 2 * UPC ? r / UPC : 0u, pc = r < 2 * UPC ? r % UPC : 0u;
    const uint32_t mat = row / C::NCOL;
    off_us[i] = (uint32_t)(mat * (so1 - so0) + arr * (bo0 - so0)) + (row % C::NCOL) * ng * 2 + pc * 16;
  }
  const uint32_t c43 = 0x43434343u;

  // Copy sources of one unit at its chunk 0 (the chunk offsets are added
  // per chunk). Computed once per unit; the unit's item is decoded with one
  // division.
  struct UnitSrc {
    const uint8_t* bq;
    const uint8_t* bs;
    const uint8_t* ah;
    const uint8_t* al;
    const uint8_t* xs;
    uint32_t cnt;
  };
  // Work-list words (expert, start | count << 16) of unit v's item, a
  // scalar load; each unit's words are loaded one unit ahead of their use,
  // so no wave waits on this load when a unit starts.
  auto item_words = [=](uint32_t v) {
    return *reinterpret_cast<const uint2*>(items + 2 * (size_t)(item_lo + v / ncb));
  };
  auto unit_src = [=](uint32_t v, uint2 iw) {
    const uint32_t cb = v % ncb;
    const uint32_t e = iw.x;
    const uint32_t start = iw.y & 0xFFFFu, cnt = iw.y >> 16;
    const uint8_t* blob = shared && e == e_shared ? shared : experts + (size_t)e * stride;
    UnitSrc u;
    u.bq = blob + wo0 + (size_t)cb * C::NCOL * rowb;
    u.bs = blob + so0 + (size_t)cb * C::NCOL * ng * 2;
    const size_t r0 = C::GATHER ? 0 : start;  // gathered rows are addressed by token
    u.ah = reinterpret_cast<const uint8_t*>(ahi_src + r0 * K);
    u.al = reinterpret_cast<const uint8_t*>(alo_src + r0 * K);
    u.xs = reinterpret_cast<const uint8_t*>(gsum + r0 * ng);
    u.cnt = cnt;
    return u;
  };
  // Per-lane byte offsets of one unit's A rows (row pair (dw N_A + i,
  // + 16)) and group-sum rows from its row base: gate/up by the token ids in
  // token buffer `par` (rows past the count hold any value: clamped to a
  // token id), down by the entry row (rows past the count repeat the last
  // one). Results of rows past the count are never stored.
  struct UnitRows {
    uint32_t a[C::N_A];
    uint32_t x[C::NXR > 0 ? C::NXR : 1];
  };
  auto unit_rows = [=](const UnitSrc& u, uint32_t par) {
    const uint32_t* tb = reinterpret_cast<const uint32_t*>(lds + C::OFF_TOK) + par * kPfMC;
    auto row = [&](uint32_t m) { return C::GATHER ? min(tb[m], last_tok) : min(m, u.cnt - 1); };
    UnitRows r;
#pragma unroll
    for (int i = 0; i < C::N_A; ++i) r.a[i] = row(dw * C::N_A + i + 16 * (lane >> 5)) * K * 2;
#pragma unroll
    for (int i = 0; i < C::NXR; ++i) {
      const uint32_t p = dw * ((C::USB ? C::P_UXS : C::P_XS) / C::NW) + i * 64 + lane;
      const uint32_t m = C::USB ? min(p / (uint32_t)(C::NGU / 4), kPfMC - 1) : p % kPfMC;
      r.x[i] = row(m) * ng * 4;
    }
    return r;
  };
  // Gate/up: copy unit v's 32 token ids into token buffer `par` (one wave).
  auto token_dma = [=](uint32_t v, uint32_t par) {
    if (C::GATHER && dw == 0 && lane < kPfMC)
      dma4(item_tok + (size_t)(item_lo + v / ncb) * kPfMC + lane, lds + C::OFF_TOK + par * kPfMC * 4);
  };
  // Issue every copy of chunk c of unit u into stage `slot`. Captures by
  // value: a by-reference capture stores the locals' addresses, and the
  // memory clobbers of the waits below would then keep them in scratch.
  // Unit scale copies into unit buffer ub (before the unit's first chunk).
  auto issue_unit = [=](const UnitSrc& u, const UnitRows& rw, uint32_t ub) {
    uint8_t* ubuf = lds + C::S * C::STAGE + ub * C::UBUF;
#pragma unroll
    for (int i = 0; i < C::N_US; ++i)
      if ((C::P_US / C::NW) % 64 == 0 || i * 64 + lane < (uint32_t)(C::P_US / C::NW))
        dma16(u.bs + pf_voff(off_us[i]), ubuf + (dw * (C::P_US / C::NW) + i * 64) * 16);
    // Group sums: slot p = (row m, slot in row) holds the row's piece
    // (slot ^ m % XPR) under gate/up (pf_unit_bias reads one group of 16
    // rows at once: the XOR spreads them over the banks), else piece p;
    // row offsets from rw.
    constexpr uint32_t XPR = C::NGU / 4;  // pieces per row
#pragma unroll
    for (int i = 0; i < C::N_UXS; ++i) {
      const uint32_t p = dw * (C::P_UXS / C::NW) + i * 64 + lane;
      const uint32_t pc = MODE == 0 ? (p % XPR) ^ ((p / XPR) & (XPR - 1)) : p % XPR;
      if ((C::P_UXS / C::NW) % 64 == 0 || i * 64 + lane < (uint32_t)(C::P_UXS / C::NW))
        dma16(u.xs + rw.x[i] + pc * 16, ubuf + C::OFF_UXS + (dw * (C::P_UXS / C::NW) + i * 64) * 16);
    }
  };
  auto issue = [=](const UnitSrc& u, const UnitRows& rw, uint32_t c, uint32_t slot) {
    const uint32_t cnt = u.cnt;
    uint8_t* st = lds + slot * C::STAGE;
    // Weight codes: slot p = (row, slot part) holds the row's part
    // (slot part ^ row & 7) [4-bit] or ((slot part + row) % 6) [3-bit].
    const uint8_t* bq_base = u.bq + (size_t)c * C::RB;
#pragma unroll
    for (int i = 0; i < C::N_BQ; ++i)
      if ((C::P_BQ / C::NW) % 64 == 0 || i * 64 + lane < (uint32_t)(C::P_BQ / C::NW))
        dma16(bq_base + pf_voff(off_bq[i]), st + C::OFF_BQ + (dw * (C::P_BQ / C::NW) + i * 64) * 16);
    // Scales then biases of each row: [row][array][CG] bf16.
    const uint8_t* bs_base = u.bs + (size_t)c * C::CG * 2;
#pragma unroll
    for (int i = 0; i < C::N_BS; ++i) {
      uint8_t* dst = st + C::OFF_BS + (dw * (C::P_BS / C::NW) + i * 64) * C::SB_SZ;
      if ((C::P_BS / C::NW) % 64 == 0 || i * 64 + lane < (uint32_t)(C::P_BS / C::NW)) {
        if (C::SB_SZ == 16) dma16(bs_base + pf_voff(off_bs[i]), dst); else dma4(bs_base + pf_voff(off_bs[i]), dst);
      }
    }
    // A rows (bf16, MFMA order), one row pair (m, m + 16) per copy; slot
    // part = part ^ (m & 15). Rows 16.. are copied only for a second tile.
#pragma unroll
    for (int hl = 0; hl < (SPLIT ? 2 : 1); ++hl) {
      const uint8_t* a_base = (hl ? u.al : u.ah) + (size_t)c * C::KC * 2;
#pragma unroll
      for (int i = 0; i < C::N_A; ++i) {
        const uint32_t pair = dw * C::N_A + i, half = lane >> 5, sp = lane & 31;
        const uint32_t off = rw.a[i] + (sp ^ pair) * 16;
        if (half == 0 || cnt > 16)
          dma16(a_base + off, st + (hl ? C::OFF_AL : C::OFF_AH) + pair * 64 * 16);
      }
    }
    // Group sums of the A rows, [group][row].
    const uint8_t* xs_base = u.xs + (size_t)c * C::CG * 4;
#pragma unroll
    for (int i = 0; i < C::N_XS; ++i) {
      const uint32_t o = i * 64 + lane;
      const uint32_t p = dw * (C::P_XS / C::NW) + o;
      const uint32_t g = p / kPfMC;
      if ((C::P_XS / C::NW) % 64 == 0 || o < (uint32_t)(C::P_XS / C::NW))
        dma4(xs_base + rw.x[i] + g * 4, st + C::OFF_XS + (dw * (C::P_XS / C::NW) + i * 64) * 4);
    }
  };

  f32x4 tot[C::NMAT][C::CT][2];
#pragma unroll
  for (int mt = 0; mt < C::NMAT; ++mt)
#pragma unroll
    for (int ct = 0; ct < C::CT; ++ct)
#pragma unroll
      for (int t = 0; t < 2; ++t) tot[mt][ct][t] = f32x4{0.f, 0.f, 0.f, 0.f};

  // Issue position (unit iv, chunk ic, stage islot) runs S - 1 chunks ahead
  // of the compute position (unit cv, chunk cc, stage cslot).
  uint32_t iv = lb, ic = 0, islot = 0, issued = 0, iub = 0;
  UnitSrc isrc = unit_src(iv, item_words(iv));
  uint2 inext = iv + per < group_units ? item_words(iv + per) : uint2{0u, 0u};
  UnitRows irows;
  if constexpr (C::GATHER) {
    // The first unit's token ids, visible to every wave before its copies.
    // Later units' ids are copied with the previous unit's first chunk, at
    // least K / 256 - 1 >= S - 1 chunks ahead, so the per-chunk waits and
    // barriers below have made them visible when that unit starts.
    if (copier) token_dma(iv, 0);
    asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
    __builtin_amdgcn_s_barrier();
    asm volatile("" ::: "memory");
  }
  // At a unit's first chunk: its row offsets, and the next unit's token ids.
  auto start_unit = [&]() {
    irows = unit_rows(isrc, iub);
    if (iv + per < group_units) token_dma(iv + per, iub ^ 1u);
  };
  for (; issued + 1 < (uint32_t)C::S && issued < total; ++issued) {
    if (copier) {
      if (ic == 0) start_unit();
      if (C::USB && ic == 0) issue_unit(isrc, irows, iub);
      issue(isrc, irows, ic, islot);
    }
    islot = islot + 1 == (uint32_t)C::S ? 0u : islot + 1;
    if (++ic == nch) {
      ic = 0;
      iub ^= 1u;
      iv += per;
      if (iv < group_units) {
        isrc = unit_src(iv, inext);
        if (iv + per < group_units) inext = item_words(iv + per);
      }
    }
  }
  uint32_t cv = lb, cc = 0, cslot = 0, cub = 0;
  uint32_t c_cb = cv % ncb;
  uint32_t c_w = item_words(cv).y;
  uint32_t c_start = c_w & 0xFFFFu, c_cnt = c_w >> 16;
  uint32_t c_next = cv + per < group_units ? item_words(cv + per).y : 0u;
  // Activation group sums of the last finished unit, still to be written by
  // wave 0 once a block barrier has ordered the column waves' row sums.
  bool ps_pend = false;
  uint32_t ps_start = 0, ps_cnt = 0, ps_cb = 0;
  auto flush_asum = [&]() {
    if (wave == 0) {
      constexpr uint32_t GPU = 64 / G;  // groups per unit
      const float* ps = reinterpret_cast<const float*>(lds + C::OFF_PS);
      const uint32_t m = lane % kPfMC, gl = lane / kPfMC;
      if (gl < GPU && m < ps_cnt) {
        float sum;
        if constexpr (GPU == 1)
          sum = (ps[m] + ps[kPfMC + m]) + (ps[2 * kPfMC + m] + ps[3 * kPfMC + m]);
        else
          sum = ps[2 * gl * kPfMC + m] + ps[(2 * gl + 1) * kPfMC + m];
        asum_out[(size_t)(ps_start + m) * (N / G) + ps_cb * GPU + gl] = sum;
      }
    }
    ps_pend = false;
  };
  for (uint32_t j = 0; j < total; ++j) {
    // Copies of chunks j + 1 .. j + S - 2 may stay in flight: D each, plus
    // DU unit scale copies for a chunk that starts a unit (nch >= 2, so at
    // most one of the next two does).
    const uint32_t ahead = min((uint32_t)C::S - 2, total - 1 - j);
    const bool ustart = C::USB && ((ahead >= 1 && cc + 1 == nch) || (ahead >= 2 && cc + 2 == nch));
    if (!copier)
      asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
    else if (ahead == 0)
      asm volatile("s_waitcnt vmcnt(0) lgkmcnt(0)" ::: "memory");
    else if (ahead == 1 && !ustart)
      asm volatile("s_waitcnt vmcnt(%0) lgkmcnt(0)" ::"n"(C::D) : "memory");
    else if (ahead == 1)
      asm volatile("s_waitcnt vmcnt(%0) lgkmcnt(0)" ::"n"(C::D + C::DU) : "memory");
    else if (!ustart)
      asm volatile("s_waitcnt vmcnt(%0) lgkmcnt(0)" ::"n"(2 * C::D) : "memory");
    else
      asm volatile("s_waitcnt vmcnt(%0) lgkmcnt(0)" ::"n"(2 * C::D + C::DU) : "memory");
    __builtin_amdgcn_s_barrier();
    asm volatile("" ::: "memory");
    if (issued < total) {
      if (copier) {
        if (ic == 0) start_unit();
        if (C::USB && ic == 0) issue_unit(isrc, irows, iub);
        issue(isrc, irows, ic, islot);
      }
      ++issued;
      islot = islot + 1 == (uint32_t)C::S ? 0u : islot + 1;
      if (++ic == nch) {
        ic = 0;
        iub ^= 1u;
        iv += per;
        if (iv < group_units) {
          isrc = unit_src(iv, inext);
          if (iv + per < group_units) inext = item_words(iv + per);
        }
      }
    }
    // The row sums are read before the next unit end writes them again:
    // that comes after one more block barrier, which wave 0 passes with its
    // LDS reads complete.
    if constexpr (C::ASUM)
      if (ps_pend) flush_asum();

    const uint32_t start = c_start, cnt = c_cnt, cb = c_cb;
    uint8_t* st = lds + cslot * C::STAGE;
    cslot = cslot + 1 == (uint32_t)C::S ? 0u : cslot + 1;
    const uint8_t* ub = lds + C::S * C::STAGE + cub * C::UBUF;
    const uint8_t* sbb = C::USB ? ub : st + C::OFF_BS;
    const float* uxs = reinterpret_cast<const float*>(ub + C::OFF_UXS);
    const uint32_t gofs = C::USB ? cc * C::CG : 0u;
    if (computer) {
      if (cnt > 16)
        pf_chunk<BITS, G, MODE, SPLIT, KU, 2>(st, sbb, uxs, gofs, kh * C::CGW, cw, n, q, c43, tot);
      else
        pf_chunk<BITS, G, MODE, SPLIT, KU, 1>(st, sbb, uxs, gofs, kh * C::CGW, cw, n, q, c43, tot);
    }

    if (++cc == nch) {  // unit complete: add the K halves, write it out
      if constexpr (MODE == 0 && C::USB)
        if (computer) pf_unit_bias<BITS, G, MODE, SPLIT, KU>(ub, nch, kh, cw, lane, cnt > 16 ? 2u : 1u, tot);
      cc = 0;
      cub ^= 1u;
      cv += per;
      if (cv < group_units) {
        c_cb = cv % ncb;
        c_start = c_next & 0xFFFFu;
        c_cnt = c_next >> 16;
        if (cv + per < group_units) c_next = item_words(cv + per).y;
      }
      // The K halves swap the partial sums of the rows the other one
      // finishes ([column wave][receiving half][accumulator][lane]).
      if constexpr (!C::EXD) {
        // In the stage just read: every wave must be done reading it.
        asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
        __builtin_amdgcn_s_barrier();
        asm volatile("" ::: "memory");
      }
      constexpr int NTH = C::NT / 2;
      float* const exb = C::EXD ? reinterpret_cast<float*>(lds + C::OFF_EX) : reinterpret_cast<float*>(st);
      if (computer) {
        float* const xo = exb + (cw * 2 + (kh ^ 1u)) * NTH * 64 + lane;
        const uint32_t rp = 2 * (kh ^ 1u);  // first row the other half finishes
#pragma unroll
        for (int mt = 0; mt < C::NMAT; ++mt)
#pragma unroll
          for (int ct = 0; ct < C::CT; ++ct)
#pragma unroll
            for (int t = 0; t < 2; ++t)
#pragma unroll
              for (int rr = 0; rr < 2; ++rr)
                xo[(((mt * C::CT + ct) * 2 + t) * 2 + rr) * 64] = rp ? tot[mt][ct][t][2 + rr] : tot[mt][ct][t][rr];
      }
      asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
      __builtin_amdgcn_s_barrier();
      asm volatile("" ::: "memory");
      if (computer) {
        const float* const xi = exb + (cw * 2 + kh) * NTH * 64 + lane;
        const uint32_t ntiles = cnt > 16 ? 2 : 1;
        float hl[2][2] = {};  // gate/up: this lane's fp16 activation, rows 16 t + 4 q + 2 kh + rr
#pragma unroll
        for (int t = 0; t < 2; ++t) {
          if ((uint32_t)t >= ntiles) continue;
#pragma unroll
          for (int rr = 0; rr < 2; ++rr) {
            const uint32_t m = 16 * t + 4 * q + 2 * kh + rr;
#pragma unroll
            for (int ct = 0; ct < C::CT; ++ct) {
              float o[C::NMAT];
#pragma unroll
              for (int mt = 0; mt < C::NMAT; ++mt)
                o[mt] = (kh ? tot[mt][ct][t][2 + rr] : tot[mt][ct][t][rr]) +
                        xi[(((mt * C::CT + ct) * 2 + t) * 2 + rr) * 64];
              if (m >= cnt) continue;
              const uint32_t colj = cb * C::NCOL + cw * 16 * C::CT + ct * 16 + n;
              if constexpr (MODE == 0) {
                // act as fp16 (round to nearest even) in the MFMA order of
                // the down GEMM.
                const float v = silu_mul(o[0], o[1]);
                const _Float16 h = (_Float16)v;
                const size_t at = (size_t)(start + m) * N + (colj & ~7u) + perm8_pos(colj & 7u);
                act_hi[at] = __builtin_bit_cast(uint16_t, h);
                hl[t][rr] = (float)h;
              } else {
                down[(size_t)(start + m) * N + colj] = o[0];
              }
            }
          }
        }
        // Gate/up with G <= 64: the down GEMM's activation group sums (over
        // what its MFMAs see, the fp16 values), for the 64 / G groups of this
        // unit's 64 columns: each column wave sums its 16 columns per row
        // (the lanes of a 16-lane row); wave 0 adds the column waves of a
        // group after the next block barrier (flush_asum).
        if constexpr (C::ASUM) {
          float* ps = reinterpret_cast<float*>(lds + C::OFF_PS);
#pragma unroll
          for (int t = 0; t < 2; ++t)
#pragma unroll
            for (int rr = 0; rr < 2; ++rr) {
              const float rs = row_sum16_all(hl[t][rr]);
              if (n == 0) ps[cw * kPfMC + 16 * t + 4 * q + 2 * kh + rr] = rs;
            }
        }
      }
      if constexpr (C::ASUM) {
        ps_pend = true;
        ps_start = start;
        ps_cnt = cnt;
        ps_cb = cb;
      }
#pragma unroll
      for (int mt = 0; mt < C::NMAT; ++mt)
#pragma unroll
        for (int ct = 0; ct < C::CT; ++ct)
#pragma unroll
          for (int t = 0; t < 2; ++t) tot[mt][ct][t] = f32x4{0.f, 0.f, 0.f, 0.f};
    }
  }
  if constexpr (C::ASUM) {
    // The last unit's sums (every wave leaves the loop after the same chunk).
    asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
    __builtin_amdgcn_s_barrier();
    asm volatile("" ::: "memory");
    if (ps_pend) flush_asum();
  }
}

// ---------------------------------------------------------------------------
// Gate/up and down GEMMs on 32 x 32 tiles (k_pf_gu64): 4-bit codes, group
// 64; gate/up over bf16 x, down over the fp16 activations.
//
// The staged pipeline of k_pf_mm (persistent block per CU, LDS DMA rings,
// one block barrier per 256-input chunk, four copy-only waves beside eight
// compute waves, the XCD-aware work list), with a wider unit: (item, 128
// output columns) = 256 weight rows. Its 32 token rows are copied once per
// chunk for all 256 rows, so they are a third of a chunk's copies instead
// of a half (16 KB next to 32 KB of codes and 4 KB of scales). The codes
// ring runs two chunks ahead, the token rows (from L2) one, and scales
// with biases go per chunk pair in 16-byte pieces (Gu64). Compute wave (cw, kh) owns
// columns 32 cw .. 32 cw + 31 of both matrices (one v_mfma_f32_32x32x16_bf16
// tile each, the 32 item rows by 32 columns, so SwiGLU pairs are in the same
// lane) and the chunk's groups 2 kh, 2 kh + 1; each A fragment read feeds
// both tiles. The dequant term (b - 128 s) * sum x of the wave's two groups
// is exactly one v_mfma_f32_32x32x2_f32 per tile and chunk (K = 2 groups).
// At a unit's end the K halves swap partial sums through the code slot just
// read (each finishes 16 of the 32 rows), then SwiGLU, fp16 activations in
// the down GEMM's order, and the activations' 64-column group sums.
//
// Lane l: column (or A row) l % 32, k half kq = l / 32. Code words: lane
// (c, kq) reads the 16 bytes of row c at k half kq of group g (words 0-3 =
// MFMA steps 0-3); the A fragment of step s is the 8-input block 8 g + 4 kq
// + s of the item row, stored in the unpack order as for k_pf_mm.
//
// Down (DOWN = true): the same rings over one matrix, a unit = (item, 256
// output columns) = 256 rows of the down matrix, A = the item's entry rows
// of the fp16 activations (rows start .. start + cnt - 1, no token ids) with
// their group sums. Wave (cw, kh) owns one tile, columns 128 kh + 32 cw ..
// + 31, over the whole K of every chunk (its four groups; two dequant-term
// MFMAs per chunk), so a unit's sums are complete in each wave and need no
// exchange (the waves read every A fragment, twice the A reads of a K
// split, which the LDS absorbs); codes enter the fp16 MFMA as 1 + q / 64,
// so the scale is 64 s and the dequant term (b - 64 s) * sum a. The unit's
// end stores the f32 sums per entry (the combine reads them).
// ---------------------------------------------------------------------------
typedef float f32x16 __attribute__((ext_vector_type(16)));

__device__ __forceinline__ f32x16 mfma32(u32x4 a, u32x4 b, f32x16 c) {
  return __builtin_amdgcn_mfma_f32_32x32x16_bf16(__builtin_bit_cast(bf16x8, a), __builtin_bit_cast(bf16x8, b), c,
                                                 0, 0, 0);
}

__device__ __forceinline__ f32x16 mfma32_f16(u32x4 a, u32x4 b, f32x16 c) {
  return __builtin_amdgcn_mfma_f32_32x32x16_f16(__builtin_bit_cast(f16x8, a), __builtin_bit_cast(f16x8, b), c,
                                                0, 0, 0);
}

struct Gu64 {
  static constexpr int NWC = 8, NWD = 4, NWT = NWC + NWD;  // compute, copy, all waves
  static constexpr int G = 64, KC = 256, CG = KC / G;       // inputs per chunk, groups per chunk
  static constexpr int NCOL = 128, ROWS = 2 * NCOL;         // output columns, weight rows per unit
  static constexpr uint32_t SMALL = 16;                     // units of <= SMALL rows take 16-row tiles
  static constexpr int RB = KC / 2;                         // code bytes per row and chunk
  // Three rings: codes two chunks ahead; token rows and their group sums
  // one chunk ahead (they come from L2); scales and biases per chunk pair,
  // copied with the pair's first chunk's token rows in 16-byte pieces (the
  // 8 bytes a chunk needs per row and array would be 4-byte pieces, twice
  // the cache lines per chunk).
  static constexpr int SC = 3, SA = 2, SS = 2;
  static constexpr int BQ_SLOT = ROWS * RB;                 // [row][8 parts of 16 B], part ^ (row & 7)
  static constexpr int OFF_BQ = 0;
  static constexpr int A_BYTES = 32 * KC * 2;               // [32 rows][32 parts of 16 B], part ^ (row & 15)
  static constexpr int A_SLOT = A_BYTES + 32 * CG * 4;      // + [32 rows][CG] f32 group sums of x
  static constexpr int OFF_A = OFF_BQ + SC * BQ_SLOT;
  static constexpr int S_SLOT = ROWS * 2 * 2 * CG * 2;      // [row][scale, bias][2 CG] bf16
  static constexpr int OFF_S = OFF_A + SA * A_SLOT;
  static constexpr int OFF_TOK = OFF_S + SS * S_SLOT;       // [2][32] token ids of two units
  static constexpr int OFF_PS = OFF_TOK + 2 * 32 * 4;       // [4 column waves][32 rows] activation row sums
  static constexpr int LDS = OFF_PS + 4 * 32 * 4;
  // Copies per copy wave: codes (16 B pieces) per chunk, A rows (16 B) and
  // x group sums (16 B, 8 lanes) per chunk, scales and biases (16 B) per
  // chunk pair.
  static constexpr int N_BQ = ROWS * RB / 16 / NWD / 64;
  static constexpr int N_A = A_BYTES / 16 / NWD / 64;
  static constexpr int N_S = S_SLOT / 16 / NWD / 64;
  static constexpr int EX = 8 * 16 * 64 * 4;  // K-half exchange: [cw][receiving half][16 values][lane] f32
  static_assert(N_BQ * NWD * 64 * 16 == BQ_SLOT && N_A * NWD * 64 * 16 == A_BYTES, "equal copy shares");
  static_assert(N_S * NWD * 64 * 16 == S_SLOT, "equal copy shares");
  static_assert(N_BQ * 8 * NWD == ROWS && N_S * 32 * NWD == ROWS, "copy rows per wave");
  static_assert(EX <= BQ_SLOT, "exchange fits a code slot");
  static_assert(LDS <= 160 * 1024, "LDS per CU");
};

// The activation group sums of a finished gate/up unit from the row-sum
// buffer: [column wave][32 rows] after 32 x 32 tiles, [column wave][k half]
// [16 rows] after 16-row tiles; lane (m, gq) = (row, 64-column group).
__device__ __forceinline__ void gu64_flush_asum(const float* ps, float* asum_out, uint32_t lane, uint32_t start,
                                                uint32_t cnt, uint32_t cb, bool small, uint32_t groups) {
  const uint32_t m = lane & 31, gq = lane >> 5;
  if (m < cnt)
    asum_out[(size_t)(start + m) * groups + cb * 2 + gq] =
        small ? (ps[(4 * gq) * 16 + m] + ps[(4 * gq + 1) * 16 + m]) + (ps[(4 * gq + 2) * 16 + m] + ps[(4 * gq + 3) * 16 + m])
              : ps[(2 * gq) * 32 + m] + ps[(2 * gq + 1) * 32 + m];
}

template <bool DOWN>
__global__ __launch_bounds__(64 * Gu64::NWT) void k_pf_gu64(PfArgs a, const uint32_t* __restrict__ items,
                                                             const uint32_t* __restrict__ n_items_p,
                                                             const uint32_t* __restrict__ xr) {
  using C = Gu64;
  extern __shared__ __attribute__((aligned(16))) uint8_t lds[];
  const uint32_t tid = threadIdx.x, lane = tid & 63, wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const bool copier = wave >= (uint32_t)C::NWC;
  const uint32_t dw = copier ? wave - C::NWC : 0u;           // copy share
  const uint32_t cw = wave & 3, kh = (wave >> 2) & 1;        // compute waves: column block, K half
  const uint32_t c32 = lane & 31, kq = lane >> 5;
  const uint32_t K = DOWN ? a.g.inter : a.g.hidden, N = DOWN ? a.g.hidden : a.g.inter;
  const uint32_t ng = K / C::G, nch = K / C::KC, rowb = K / 2;
  constexpr uint32_t UCOL = DOWN ? C::ROWS : C::NCOL;  // output columns per unit
  const uint32_t ncb = N / UCOL;
  const uint32_t nx = gridDim.x % 8 == 0 ? 8 : 1, per = gridDim.x / nx;
  const uint32_t xg = blockIdx.x % nx, lb = blockIdx.x / nx;
  const uint32_t n_items = *n_items_p;
  const uint32_t item_lo = xr && nx == 8 ? xr[xg] : n_items * xg / nx;
  const uint32_t item_hi = xr && nx == 8 ? xr[xg + 1] : n_items * (xg + 1) / nx;
  const uint32_t group_units = (item_hi - item_lo) * ncb;
  const uint32_t my_units = group_units > lb ? (group_units - lb + per - 1) / per : 0;
  const uint32_t total = my_units * nch;
  if (total == 0) return;
  // Kernel arguments into scalar locals (nothing takes the argument
  // block's address).
  const uint8_t* const experts = a.experts;
  const uint8_t* const shared = a.shared_in_list ? a.shared : nullptr;
  const uint32_t e_shared = a.E;
  const uint32_t* const item_tok = a.item_tok;
  const uint32_t last_tok = a.n_tokens - 1;
  const uint64_t stride = a.stride;
  // A rows and their group sums: token rows of x, or entry rows of the
  // activations.
  const uint8_t* const xh = reinterpret_cast<const uint8_t*>(DOWN ? a.act_hi : a.x_hi);
  const uint8_t* const xsum = reinterpret_cast<const uint8_t*>(DOWN ? a.asum : a.xsum);
  uint16_t* const act_out = a.act_hi;
  float* const asum_out = a.asum;
  float* const down_out = a.down;
  const uint64_t wo0 = a.g.w[DOWN ? 2 : 0], wo1 = a.g.w[DOWN ? 2 : 1];
  const uint64_t so0 = a.g.s[DOWN ? 2 : 0], so1 = a.g.s[DOWN ? 2 : 1];
  const uint64_t bso = a.g.b[DOWN ? 2 : 0] - so0;
  const uint32_t c43 = 0x43434343u;

  struct Unit {
    uint32_t e, start, cnt, cb, item;
  };
  auto unit = [=](uint32_t i) {  // unit i of this block (scalar loads of its work-list words)
    const uint32_t v = lb + per * i;
    Unit u;
    u.item = item_lo + v / ncb;
    u.cb = v % ncb;
    const uint2 iw = *reinterpret_cast<const uint2*>(items + 2 * (size_t)u.item);
    u.e = iw.x;
    u.start = iw.y & 0xFFFFu;
    u.cnt = iw.y >> 16;
    return u;
  };
  // Token ids of unit i into token buffer `par`: copy wave d, lanes 0-7,
  // rows 8 d .. 8 d + 7.
  auto token_dma = [=](uint32_t i, uint32_t par) {
    if (!DOWN && lane < 8) dma4(item_tok + (size_t)unit(i).item * kPfMC + 8 * dw + lane, lds + C::OFF_TOK + (par * 32 + 8 * dw) * 4);
  };
  // Per-lane source offsets of one unit's copies (fixed while the unit
  // lasts; the chunk adds a scalar offset). Copy wave d's code pieces are
  // rows 64 d + 8 i + l / 8 (gate/up: gate rows for d < 2, up rows for d >=
  // 2) at 16-byte part (l % 8) ^ (l / 8 % 8), so copy i adds 8 i rows to one
  // lane offset; its scale pieces are rows 64 d + 32 i + l / 2, array l % 2,
  // likewise; its A rows are 8 d + 2 i + l / 32, one token (entry) row each.
  struct SrcC {
    const uint8_t* blob;
    uint32_t bq;  // from the blob, copy 0
  };
  struct SrcA {
    const uint8_t* blob;
    uint32_t s;            // from the blob, copy 0
    uint32_t ar[C::N_A];   // from x_hi (token row + part)
    uint32_t xs;           // from xsum
    bool small;            // a unit of <= 16 rows: rows 16-31 are not copied
  };
  auto srcc_of = [=](const Unit& u) {
    SrcC r;
    r.blob = shared && u.e == e_shared ? shared : experts + (size_t)u.e * stride;
    const uint32_t mat = DOWN ? 0u : dw >= 2;
    const uint32_t row0 = DOWN ? u.cb * C::ROWS + 64 * dw : u.cb * C::NCOL + 64 * (dw & 1u);
    r.bq = (uint32_t)(mat ? wo1 : wo0) + (row0 + lane / 8) * rowb + (((lane & 7u) ^ ((lane >> 3) & 7u)) * 16);
    return r;
  };
  auto srca_of = [=](const Unit& u, uint32_t par) {
    SrcA r;
    r.blob = shared && u.e == e_shared ? shared : experts + (size_t)u.e * stride;
    const uint32_t mat = DOWN ? 0u : dw >= 2;
    const uint32_t row0 = DOWN ? u.cb * C::ROWS + 64 * dw : u.cb * C::NCOL + 64 * (dw & 1u);
    r.s = (uint32_t)((mat ? so1 : so0) + (lane & 1u) * bso) + (row0 + lane / 2) * ng * 2;
    r.small = u.cnt <= C::SMALL;
    if constexpr (DOWN) {
      // Entry rows past the item's count repeat its last row.
      const uint32_t last = u.cnt - 1;
#pragma unroll
      for (int i = 0; i < C::N_A; ++i) {
        const uint32_t row = 8 * dw + 2 * i + lane / 32, part = (lane % 32) ^ (row & 15u);
        r.ar[i] = (u.start + min(row, last)) * K * 2 + part * 16;
      }
      r.xs = (u.start + min(8 * dw + min(lane, 7u), last)) * ng * 4;
    } else {
      const uint32_t* tb = reinterpret_cast<const uint32_t*>(lds + C::OFF_TOK) + par * 32;
#pragma unroll
      for (int i = 0; i < C::N_A; ++i) {
        const uint32_t row = 8 * dw + 2 * i + lane / 32, part = (lane % 32) ^ (row & 15u);
        r.ar[i] = min(tb[row], last_tok) * K * 2 + part * 16;
      }
      r.xs = min(tb[8 * dw + min(lane, 7u)], last_tok) * ng * 4;
    }
    return r;
  };
  // Chunk c's codes into code slot `slot`.
  auto issue_codes = [=](const SrcC& r, uint32_t c, uint32_t slot) {
    uint8_t* st = lds + C::OFF_BQ + slot * C::BQ_SLOT;
    const uint8_t* bq = r.blob + (size_t)c * C::RB;
#pragma unroll
    for (int i = 0; i < C::N_BQ; ++i)
      dma16(bq + (size_t)(8 * i) * rowb + pf_voff(r.bq), st + (dw * C::N_BQ + i) * 64 * 16);
  };
  // Chunk c's token rows and x group sums into A slot `slot`; with `pair`,
  // the scales and biases of chunks c and c + 1 into scale slot `sslot`.
  auto issue_a = [=](const SrcA& r, uint32_t c, uint32_t slot, bool pair, uint32_t sslot) {
    uint8_t* st = lds + C::OFF_A + slot * C::A_SLOT;
    const uint8_t* ab = xh + (size_t)c * C::KC * 2;
    if (!r.small || dw < 2) {  // copy waves 2 and 3 hold rows 16-31
#pragma unroll
      for (int i = 0; i < C::N_A; ++i) dma16(ab + r.ar[i], st + (dw * C::N_A + i) * 64 * 16);
      if (lane < 8) dma16(xsum + (size_t)c * C::CG * 4 + r.xs, st + C::A_BYTES + 8 * dw * 16);
    }
    if (pair) {
      uint8_t* ss = lds + C::OFF_S + sslot * C::S_SLOT;
      const uint8_t* sb = r.blob + (size_t)c * C::CG * 2;
#pragma unroll
      for (int i = 0; i < C::N_S; ++i)
        dma16(sb + (size_t)(32 * i) * ng * 2 + pf_voff(r.s), ss + (dw * C::N_S + i) * 64 * 16);
    }
  };

  // The first unit's token ids, visible to every wave before its copies.
  if (!DOWN && copier) token_dma(0, 0);
  asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
  __builtin_amdgcn_s_barrier();
  asm volatile("" ::: "memory");
  // The copy waves and the compute waves run loops of their own over the
  // same chunk sequence and meet at the same block barriers: one per chunk
  // j >= 0 (chunk j has landed), two more after a unit's last chunk (the K
  // halves' exchange), one after the loop. Separate loops keep each role's
  // loop-carried registers out of the other's.
  if (copier) {
    // Issue positions: token rows and scales (unit au, chunk ac, token
    // buffer apar) one chunk ahead of the compute position, codes (unit
    // qu, chunk qc) two chunks ahead. The next unit's token ids are copied
    // when the first issue position enters a unit. Iterations -2 and -1
    // only issue (the prologue); iteration j >= 0 waits for chunk j's
    // copies (its codes, issued two iterations earlier, and its token rows,
    // issued one earlier before the next chunk's codes: N_BQ copies follow
    // them), then issues chunk j + 1's token rows and chunk j + 2's codes.
    uint32_t au = 0, ac = 0, apar = 0, aiss = 0;
    uint32_t qu = 0, qc = 0, qiss = 0, cc = 0;
    SrcA srca{};
    SrcC srcc{};
    for (int jj = -2; jj < (int)total; ++jj) {
      const uint32_t j = (uint32_t)jj;
      if (jj >= 0) {
        if (j + 1 < total)
          asm volatile("s_waitcnt vmcnt(%0) lgkmcnt(0)" ::"n"(C::N_BQ) : "memory");
        else
          asm volatile("s_waitcnt vmcnt(0) lgkmcnt(0)" ::: "memory");
        __builtin_amdgcn_s_barrier();
        asm volatile("" ::: "memory");
      }
      bool tok_next = false;
      if (jj >= -1 && aiss < total) {
        if (ac == 0) {
          srca = srca_of(unit(au), apar);
          tok_next = !DOWN && au + 1 < my_units;
        }
        issue_a(srca, ac, aiss & 1u, (aiss & 1u) == 0, (aiss >> 1) & 1u);
      }
      if (qiss < total) {
        if (qc == 0) srcc = srcc_of(unit(qu));
        issue_codes(srcc, qc, qiss % C::SC);
      }
      if (tok_next) token_dma(au + 1, apar ^ 1u);
      if (jj >= -1 && aiss < total) {
        ++aiss;
        if (++ac == nch) {
          ac = 0;
          ++au;
          apar ^= 1u;
        }
      }
      if (qiss < total) {
        ++qiss;
        if (++qc == nch) {
          qc = 0;
          ++qu;
        }
      }
      // The compute waves' exchange barriers after a unit's last chunk.
      if (jj >= 0 && ++cc == nch) {
        cc = 0;
        asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
        __builtin_amdgcn_s_barrier();
        asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
        __builtin_amdgcn_s_barrier();
        asm volatile("" ::: "memory");
      }
    }
    asm volatile("s_waitcnt vmcnt(0) lgkmcnt(0)" ::: "memory");
    __builtin_amdgcn_s_barrier();
    asm volatile("" ::: "memory");
    return;
  }
  f32x16 tot[2];
  tot[0] = f32x16{};
  tot[1] = f32x16{};
  // Partial sums of the 16-row tiles (t, h) of a small unit.
  f32x4 ts[2][2];
#pragma unroll
  for (int t = 0; t < 2; ++t)
#pragma unroll
    for (int h = 0; h < 2; ++h) ts[t][h] = f32x4{0.f, 0.f, 0.f, 0.f};
  uint32_t cc = 0, cu = 0;
  Unit ucur = unit(0);
  // Activation row sums of the last finished unit, written out by wave 0
  // after the next block barrier.
  bool ps_pend = false, ps_small = false;
  uint32_t ps_start = 0, ps_cnt = 0, ps_cb = 0;
  for (uint32_t j = 0; j < total; ++j) {
    asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
    __builtin_amdgcn_s_barrier();
    asm volatile("" ::: "memory");
    if (ps_pend) {
      if (wave == 0)
        gu64_flush_asum(reinterpret_cast<const float*>(lds + C::OFF_PS), asum_out, lane, ps_start, ps_cnt, ps_cb,
                        ps_small, N / C::G);
      ps_pend = false;
    }
    const uint8_t* st = lds + C::OFF_BQ + (j % C::SC) * C::BQ_SLOT;      // codes
    const uint8_t* sa = lds + C::OFF_A + (j & 1u) * C::A_SLOT;            // token rows, x sums
    const uint8_t* ss = lds + C::OFF_S + ((j >> 1) & 1u) * C::S_SLOT;     // scales, biases
    const bool small = ucur.cnt <= C::SMALL;
    if constexpr (DOWN) {
      // Down: wave (cw, kh) owns one 32-column tile, columns kh * 128 +
      // 32 cw .. + 31 of the unit, over the chunk's whole K (its four
      // groups), so a unit's sums need no exchange between waves.
      uint32_t lv = lane;
      asm volatile("" : "+v"(lv));
      const uint32_t* scp = reinterpret_cast<const uint32_t*>(ss + 8 * (j & 1u));
      if (small) {
        // 16 x 16 x 32 f16 tiles h = columns 16 h .. 16 h + 15 of the wave's
        // 32, rows 0-15; lane (c16, kb) as in the gate/up 16-row tiles.
        const uint32_t c16 = lv & 15, kb = lv >> 4;
        uint32_t sw[2][2], bw[2][2];
#pragma unroll
        for (int h = 0; h < 2; ++h) {
          const uint32_t row = kh * C::NCOL + 32 * cw + 16 * h + c16;
#pragma unroll
          for (int p = 0; p < 2; ++p) {
            sw[h][p] = scp[row * 8 + p];
            bw[h][p] = scp[row * 8 + 4 + p];
          }
        }
        const uint8_t* ar = sa + c16 * (C::KC * 2);
#pragma unroll
        for (int g = 0; g < 4; ++g) {
          u32x4 af[2];
          uint32_t bq[2][2];
#pragma unroll
          for (int u = 0; u < 2; ++u) af[u] = *reinterpret_cast<const u32x4*>(ar + (((8 * g + 4 * u + kb) ^ c16) * 16));
#pragma unroll
          for (int u = 0; u < 2; ++u)
#pragma unroll
            for (int h = 0; h < 2; ++h) {
              const uint32_t row = kh * C::NCOL + 32 * cw + 16 * h + c16;
              bq[u][h] = *reinterpret_cast<const uint32_t*>(st + row * C::RB + (((2 * g + u) ^ (row & 7u)) * 16) + 4 * kb);
            }
          f32x4 acc[2] = {f32x4{0.f, 0.f, 0.f, 0.f}, f32x4{0.f, 0.f, 0.f, 0.f}};
#pragma unroll
          for (int u = 0; u < 2; ++u)
#pragma unroll
            for (int h = 0; h < 2; ++h) acc[h] = mfma_f16(af[u], codes_f16_4p(bq[u][h]), acc[h]);
#pragma unroll
          for (int h = 0; h < 2; ++h) {
            const float sc = 64.0f * bf16f((uint16_t)(sw[h][g >> 1] >> (16 * (g & 1))));
#pragma unroll
            for (int i = 0; i < 4; ++i) ts[0][h][i] = __builtin_fmaf(sc, acc[h][i], ts[0][h][i]);
          }
        }
        // Dequant term: one v_mfma_f32_16x16x4_f32 per tile over the four
        // groups, lane (., kb) supplying group kb.
        const float xa = reinterpret_cast<const float*>(sa + C::A_BYTES)[c16 * C::CG + kb];
#pragma unroll
        for (int h = 0; h < 2; ++h) {
          const uint32_t sh = 16 * (kb & 1u);
          const float cbv = __builtin_fmaf(-64.0f, bf16f((uint16_t)(sw[h][kb >> 1] >> sh)), bf16f((uint16_t)(bw[h][kb >> 1] >> sh)));
          ts[0][h] = __builtin_amdgcn_mfma_f32_16x16x4f32(xa, cbv, ts[0][h], 0, 0, 0);
        }
      } else {
        const uint32_t c32 = lv & 31, kq = lv >> 5;
        const uint32_t row = kh * C::NCOL + 32 * cw + c32;
        uint32_t sw[2], bw[2];
#pragma unroll
        for (int p = 0; p < 2; ++p) {
          sw[p] = scp[row * 8 + p];
          bw[p] = scp[row * 8 + 4 + p];
        }
        const uint8_t* ar = sa + c32 * (C::KC * 2);
        // Groups in pairs: two independent accumulator chains (one per
        // group) interleaved, so one's MFMAs run while the other's wait.
#pragma unroll
        for (int gp = 0; gp < 2; ++gp) {
          u32x4 af[2][4], bq[2];
#pragma unroll
          for (int q = 0; q < 2; ++q) {
            const int g = 2 * gp + q;
#pragma unroll
            for (int s = 0; s < 4; ++s) af[q][s] = *reinterpret_cast<const u32x4*>(ar + (((8 * g + 4 * kq + s) ^ (c32 & 15u)) * 16));
            bq[q] = *reinterpret_cast<const u32x4*>(st + row * C::RB + (((2 * g + kq) ^ (row & 7u)) * 16));
          }
          f32x16 acc[2] = {f32x16{}, f32x16{}};
#pragma unroll
          for (int s = 0; s < 4; ++s)
#pragma unroll
            for (int q = 0; q < 2; ++q) acc[q] = mfma32_f16(af[q][s], codes_f16_4p(bq[q][s]), acc[q]);
#pragma unroll
          for (int q = 0; q < 2; ++q) {
            const float sc = 64.0f * bf16f((uint16_t)(sw[gp] >> (16 * q)));
#pragma unroll
            for (int v = 0; v < 16; ++v) tot[0][v] = __builtin_fmaf(sc, acc[q][v], tot[0][v]);
          }
        }
        // Dequant term: A = the entry rows' group sums [32 rows x 2 groups],
        // B = (b - 64 s) [2 groups x 32 columns], one MFMA per group pair.
#pragma unroll
        for (int p = 0; p < 2; ++p) {
          const float xa = reinterpret_cast<const float*>(sa + C::A_BYTES)[c32 * C::CG + 2 * p + kq];
          const uint32_t sh = 16 * kq;
          const float cb = __builtin_fmaf(-64.0f, bf16f((uint16_t)(sw[p] >> sh)), bf16f((uint16_t)(bw[p] >> sh)));
          tot[0] = __builtin_amdgcn_mfma_f32_32x32x2f32(xa, cb, tot[0], 0, 0, 0);
        }
      }
    } else if (small) {
      // A unit of <= 16 rows: 16 x 16 x 32 MFMA tiles (bf16; down: f16) (t, h) =
      // columns 16 h .. 16 h + 15 of the wave's 32 in matrix t, rows 0-15;
      // lane (c16, kb) = (A row / output column l % 16, 8-input block
      // l / 16 of the 32 per step). The same codes and A parts as the
      // 32 x 32 tiles, half the MFMA work; partial sums in ts[t][h][i]
      // (row 4 kb + i). The lane's LDS offsets are formed here per chunk
      // (the opaque lane value keeps the compiler from hoisting them out of
      // the loop, where both tile paths' offsets would not fit in the
      // registers together).
      uint32_t lv = lane;
      asm volatile("" : "+v"(lv));
      const uint32_t c16 = lv & 15, kb = lv >> 4;
      uint32_t sw[2][2], bw[2][2];
#pragma unroll
      for (int t = 0; t < 2; ++t)
#pragma unroll
        for (int h = 0; h < 2; ++h) {
          const uint32_t row = t * C::NCOL + 32 * cw + 16 * h + c16;
          const uint32_t* sp = reinterpret_cast<const uint32_t*>(ss + row * 32 + 8 * (j & 1u) + 4 * kh);
          sw[t][h] = sp[0];
          bw[t][h] = sp[4];
        }
#pragma unroll
      for (int gi = 0; gi < 2; ++gi) {
        const uint32_t g = 2 * kh + gi;
        u32x4 af[2];
        uint32_t bq[2][2][2];
        const uint8_t* ar = sa + c16 * (C::KC * 2);
#pragma unroll
        for (int u = 0; u < 2; ++u) af[u] = *reinterpret_cast<const u32x4*>(ar + (((8 * g + 4 * u + kb) ^ c16) * 16));
#pragma unroll
        for (int u = 0; u < 2; ++u)
#pragma unroll
          for (int t = 0; t < 2; ++t)
#pragma unroll
            for (int h = 0; h < 2; ++h) {
              const uint32_t row = t * C::NCOL + 32 * cw + 16 * h + c16;
              bq[u][t][h] = *reinterpret_cast<const uint32_t*>(st + row * C::RB + (((2 * g + u) ^ (row & 7u)) * 16) + 4 * kb);
            }
        f32x4 acc[2][2];
#pragma unroll
        for (int t = 0; t < 2; ++t)
#pragma unroll
          for (int h = 0; h < 2; ++h) acc[t][h] = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
        for (int u = 0; u < 2; ++u)
#pragma unroll
          for (int t = 0; t < 2; ++t)
#pragma unroll
            for (int h = 0; h < 2; ++h) {
              if constexpr (DOWN)
                acc[t][h] = mfma_f16(af[u], codes_f16_4p(bq[u][t][h]), acc[t][h]);
              else
                acc[t][h] = mfma(af[u], codes_bf16_4p(bq[u][t][h], c43), acc[t][h]);
            }
#pragma unroll
        for (int t = 0; t < 2; ++t)
#pragma unroll
          for (int h = 0; h < 2; ++h) {
            const float s = (DOWN ? 64.0f : 1.0f) * bf16f((uint16_t)(sw[t][h] >> (16 * gi)));
#pragma unroll
            for (int i = 0; i < 4; ++i) ts[t][h][i] = __builtin_fmaf(s, acc[t][h][i], ts[t][h][i]);
          }
      }
      // Dequant term: one v_mfma_f32_16x16x4_f32 per tile over the chunk's
      // four groups, lane (., kb) supplying group kb; the other k half's two
      // groups enter as zeros.
      const bool mine = (kb >> 1) == kh;
      const float xa = mine ? reinterpret_cast<const float*>(sa + C::A_BYTES)[c16 * C::CG + kb] : 0.f;
#pragma unroll
      for (int t = 0; t < 2; ++t)
#pragma unroll
        for (int h = 0; h < 2; ++h) {
          const uint32_t sh = 16 * (kb & 1u);
          const float cbv =
              mine ? __builtin_fmaf(DOWN ? -64.0f : -128.0f, bf16f((uint16_t)(sw[t][h] >> sh)), bf16f((uint16_t)(bw[t][h] >> sh)))
                   : 0.f;
          ts[t][h] = __builtin_amdgcn_mfma_f32_16x16x4f32(xa, cbv, ts[t][h], 0, 0, 0);
        }
    } else {
      // Scales and biases of this wave's two groups for both tiles: bf16
      // pairs (group 2 kh, 2 kh + 1). Lane offsets formed per chunk, as in
      // the 16-row path.
      uint32_t lv = lane;
      asm volatile("" : "+v"(lv));
      const uint32_t c32 = lv & 31, kq = lv >> 5;
      uint32_t sw[2], bw[2];
#pragma unroll
      for (int t = 0; t < 2; ++t) {
        const uint32_t row = t * C::NCOL + 32 * cw + c32;
        const uint32_t* sp = reinterpret_cast<const uint32_t*>(ss + row * 32 + 8 * (j & 1u) + 4 * kh);
        sw[t] = sp[0];
        bw[t] = sp[4];
      }
#pragma unroll
      for (int gi = 0; gi < 2; ++gi) {
        const uint32_t g = 2 * kh + gi;
        u32x4 af[4], bq[2];
        const uint8_t* ar = sa + c32 * (C::KC * 2);
#pragma unroll
        for (int s = 0; s < 4; ++s) af[s] = *reinterpret_cast<const u32x4*>(ar + (((8 * g + 4 * kq + s) ^ (c32 & 15u)) * 16));
#pragma unroll
        for (int t = 0; t < 2; ++t) {
          const uint32_t row = t * C::NCOL + 32 * cw + c32;
          bq[t] = *reinterpret_cast<const u32x4*>(st + row * C::RB + (((2 * g + kq) ^ (row & 7u)) * 16));
        }
        f32x16 acc0 = f32x16{}, acc1 = f32x16{};
#pragma unroll
        for (int s = 0; s < 4; ++s) {
          if constexpr (DOWN) {
            acc0 = mfma32_f16(af[s], codes_f16_4p(bq[0][s]), acc0);
            acc1 = mfma32_f16(af[s], codes_f16_4p(bq[1][s]), acc1);
          } else {
            acc0 = mfma32(af[s], codes_bf16_4p(bq[0][s], c43), acc0);
            acc1 = mfma32(af[s], codes_bf16_4p(bq[1][s], c43), acc1);
          }
        }
        constexpr float SQ = DOWN ? 64.0f : 1.0f;  // code scale of the MFMA form
        const float s0 = SQ * bf16f((uint16_t)(sw[0] >> (16 * gi))), s1 = SQ * bf16f((uint16_t)(sw[1] >> (16 * gi)));
#pragma unroll
        for (int v = 0; v < 16; ++v) {
          tot[0][v] = __builtin_fmaf(s0, acc0[v], tot[0][v]);
          tot[1][v] = __builtin_fmaf(s1, acc1[v], tot[1][v]);
        }
      }
      // Dequant term of the two groups: A = the A rows' group sums [32 rows
      // x 2 groups], B = (b - 128 s), down (b - 64 s) [2 groups x 32 columns].
      const float xa = reinterpret_cast<const float*>(sa + C::A_BYTES)[c32 * C::CG + 2 * kh + kq];
#pragma unroll
      for (int t = 0; t < 2; ++t) {
        const uint32_t sh = 16 * kq;
        const float cb = __builtin_fmaf(DOWN ? -64.0f : -128.0f, bf16f((uint16_t)(sw[t] >> sh)), bf16f((uint16_t)(bw[t] >> sh)));
        tot[t] = __builtin_amdgcn_mfma_f32_32x32x2f32(xa, cb, tot[t], 0, 0, 0);
      }
    }
    if (++cc == nch) {  // unit complete
      cc = 0;
      const uint32_t start = ucur.start, cnt = ucur.cnt, cb = ucur.cb;
      if (++cu < my_units) ucur = unit(cu);
      // Every wave is done reading this code slot; the gate/up K halves swap the
      // rows the other one finishes (values 8 kh' .. 8 kh' + 7 of each tile).
      asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
      __builtin_amdgcn_s_barrier();
      asm volatile("" ::: "memory");
      float* ex = reinterpret_cast<float*>(const_cast<uint8_t*>(st));
      if (DOWN) {
        // Down: every wave holds whole sums (no exchange).
      } else if (small) {
        // 16-row tiles: wave kh finishes column half kh of both matrices.
        float* xo = ex + (cw * 2 + (kh ^ 1u)) * 16 * 64 + lane;
#pragma unroll
        for (int t = 0; t < 2; ++t)
#pragma unroll
          for (int i = 0; i < 4; ++i) xo[(t * 4 + i) * 64] = kh ? ts[t][0][i] : ts[t][1][i];
      } else {
        float* xo = ex + (cw * 2 + (kh ^ 1u)) * 16 * 64 + lane;
        const uint32_t vo = 8 * (kh ^ 1u);
#pragma unroll
        for (int t = 0; t < 2; ++t)
#pragma unroll
          for (int i = 0; i < 8; ++i) xo[(t * 8 + i) * 64] = tot[t][vo + i];
      }
      asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
      __builtin_amdgcn_s_barrier();
      asm volatile("" ::: "memory");
      if (DOWN && small) {
        uint32_t lv = lane;
        asm volatile("" : "+v"(lv));
        const uint32_t c16 = lv & 15, kb = lv >> 4;
        const uint32_t col = cb * C::ROWS + kh * C::NCOL + 32 * cw + c16;
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          const uint32_t m = 4 * kb + i;
          if (m < cnt) {
            float* o = down_out + (size_t)(start + m) * N + col;
            o[0] = ts[0][0][i];
            o[16] = ts[0][1][i];
          }
        }
      } else if (DOWN) {
        const uint32_t col = cb * C::ROWS + kh * C::NCOL + 32 * cw + c32;
#pragma unroll
        for (int v = 0; v < 16; ++v) {
          const uint32_t m = 8 * (v / 4) + 4 * kq + (v % 4);
          if (m < cnt) down_out[(size_t)(start + m) * N + col] = tot[0][v];
        }
      } else if (small) {
        const float* xi = ex + (cw * 2 + kh) * 16 * 64 + lane;
        uint32_t lv = lane;
        asm volatile("" : "+v"(lv));
        const uint32_t c16 = lv & 15, kb = lv >> 4;
        const uint32_t col = cb * C::NCOL + 32 * cw + 16 * kh + c16;
        const uint32_t pc = (col & ~7u) + perm8_pos(col & 7u);
        float rs[4];
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          const uint32_t m = 4 * kb + i;
          const float g = (kh ? ts[0][1][i] : ts[0][0][i]) + xi[i * 64];
          const float u = (kh ? ts[1][1][i] : ts[1][0][i]) + xi[(4 + i) * 64];
          const _Float16 h = (_Float16)silu_mul(g, u);
          if (m < cnt) act_out[(size_t)(start + m) * N + pc] = __builtin_bit_cast(uint16_t, h);
          rs[i] = (float)h;
        }
        // Row sums over the wave's 16 columns (a 16-lane row), into
        // [column wave][k half][16 rows].
#pragma unroll
        for (int i = 0; i < 4; ++i) rs[i] = row_sum16_all(rs[i]);
        if (c16 == 0) {
          float* ps = reinterpret_cast<float*>(lds + C::OFF_PS) + (cw * 2 + kh) * 16;
#pragma unroll
          for (int i = 0; i < 4; ++i) ps[4 * kb + i] = rs[i];
        }
      } else {
        const float* xi = ex + (cw * 2 + kh) * 16 * 64 + lane;
        const uint32_t vm = 8 * kh;
        const uint32_t col = cb * C::NCOL + 32 * cw + c32;
        const uint32_t pc = (col & ~7u) + perm8_pos(col & 7u);
        float rs[8];
#pragma unroll
        for (int i = 0; i < 8; ++i) {
          const uint32_t v = vm + i;
          const uint32_t m = 8 * (v / 4) + 4 * kq + (v % 4);
          const float g = tot[0][v] + xi[i * 64], u = tot[1][v] + xi[(8 + i) * 64];
          const _Float16 h = (_Float16)silu_mul(g, u);
          if (m < cnt) act_out[(size_t)(start + m) * N + pc] = __builtin_bit_cast(uint16_t, h);
          rs[i] = (float)h;
        }
        // Row sums over the wave's 32 columns (the lanes of one k half).
#pragma unroll
        for (int i = 0; i < 8; ++i) {
          rs[i] = row_sum16_all(rs[i]);
          rs[i] += __shfl_xor(rs[i], 16, kWave);
        }
        if (c32 == 0) {
          float* ps = reinterpret_cast<float*>(lds + C::OFF_PS) + cw * 32;
#pragma unroll
          for (int i = 0; i < 8; ++i) {
            const uint32_t v = vm + i;
            ps[8 * (v / 4) + 4 * kq + (v % 4)] = rs[i];
          }
        }
      }
      ps_pend = !DOWN;
      ps_small = small;
      ps_start = start;
      ps_cnt = cnt;
      ps_cb = cb;
      tot[0] = f32x16{};
      tot[1] = f32x16{};
#pragma unroll
      for (int t = 0; t < 2; ++t)
#pragma unroll
        for (int h = 0; h < 2; ++h) ts[t][h] = f32x4{0.f, 0.f, 0.f, 0.f};
    }
  }
  // The last unit's sums (every wave leaves its loop after the same chunk).
  asm volatile("s_waitcnt vmcnt(0) lgkmcnt(0)" ::: "memory");
  __builtin_amdgcn_s_barrier();
  asm volatile("" ::: "memory");
  if (ps_pend && wave == 0)
    gu64_flush_asum(reinterpret_cast<const float*>(lds + C::OFF_PS), asum_out, lane, ps_start, ps_cnt, ps_cb, ps_small,
                    N / C::G);
}

// Group sums of the fp16 activations per entry; one block per entry.
__global__ __launch_bounds__(256) void k_pf_act_sum(PfArgs a, uint32_t row0) {
  __shared__ float part8[kPfMaxGroupsK * 128 / 8];
  const uint32_t r = row0 + blockIdx.x, I = a.g.inter, G = a.g.group;
  for (uint32_t k0 = threadIdx.x * 8; k0 < I; k0 += blockDim.x * 8) {
    const u32x4 h = *reinterpret_cast<const u32x4*>(a.act_hi + (size_t)r * I + k0);
    const uint32_t hv[4] = {h.x, h.y, h.z, h.w};
    float p = 0.f;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const f32x2 f = __builtin_convertvector(__builtin_bit_cast(f16x2, hv[i]), f32x2);
      p += f.x + f.y;
    }
    part8[k0 / 8] = p;
  }
  __syncthreads();
  const uint32_t ng = I / G, per = G / 8;
  for (uint32_t g = threadIdx.x; g < ng; g += blockDim.x) {
    float s = 0.f;
    for (uint32_t j = 0; j < per; ++j) s += part8[g * per + j];
    a.asum[(size_t)r * ng + g] = s;
  }
}

// ---------------------------------------------------------------------------
// Combine: moe[t, :] = fold over t's entries in ascending expert order
// (moe_cpu.rs:330-337); the MoE block adds the residual and the shared
// expert as moe_combine_residual_n_tokens_cpu does (backend/cpu/mod.rs:
// 657-680): out = (h_mid + moe) + sigmoid(gate . x_t) * shared (no fused
// multiply-add; the sigmoid with glibc's expf), without a shared expert
// out = h_mid + moe, without h_mid out = moe.
// ---------------------------------------------------------------------------
__global__ __launch_bounds__(512) void k_pf_combine(PfArgs a) {
#pragma clang fp contract(off)
  // Every argument in scalar registers in one batch (lazily loaded, they
  // would cost a dependent round trip per branch level).
  asm volatile("" ::"s"(a.g.hidden), "s"(a.k), "s"(a.n_tokens), "s"(a.down), "s"(a.out), "s"(a.h_mid),
               "s"(a.shared), "s"(a.gate), "s"(a.gscore), "s"(a.tok_pw));
  const uint32_t t = blockIdx.x;
  const uint32_t H = a.g.hidden, k = a.k;
  const float* const down = a.down;
  float* const out = a.out;
  const float* const h_mid = a.h_mid;
  const bool shared = a.shared != nullptr;
  // Loops over the k slots run to kPfMaxK with a guard, so that the arrays
  // stay in registers and every load of a pass is issued before the first
  // FMA waits for one.
  uint32_t pos[kPfMaxK];
  float wt[kPfMaxK];
  const uint32_t nk = a.n_tokens * k;
  // The token's (position, weight) words in one load: lane r < k reads
  // slot r (later lanes reread slot k - 1), and every slot is broadcast
  // from its lane; the gate score's load goes out with it.
  const uint32_t lane = threadIdx.x & 63u;
  const uint2 mine = a.tok_pw[t * k + (lane < k ? lane : k - 1u)];
  const float gs = shared && a.gate ? a.gscore[t] : 0.f;
#pragma unroll
  for (uint32_t r = 0; r < kPfMaxK; ++r) {
    // In range even when bucketing rejected the input (then *err is set).
    pos[r] = min((uint32_t)__builtin_amdgcn_readlane((int)mine.x, (int)r), nk - 1);
    wt[r] = __uint_as_float((uint32_t)__builtin_amdgcn_readlane((int)mine.y, (int)r));
  }
  const float sg = shared && a.gate ? sigmoid_ref(gs) : 1.0f;
  const float* const sh_row = down + (size_t)(nk + t) * H;
  for (uint32_t h = threadIdx.x * 4; h < H; h += 512u * 4u) {  // 512 threads (the launch bound)
    float4 d[kPfMaxK];
#pragma unroll
    for (uint32_t r = 0; r < kPfMaxK; ++r)
      if (r < k) d[r] = *reinterpret_cast<const float4*>(down + (size_t)pos[r] * H + h);
    float4 hm = make_float4(0.f, 0.f, 0.f, 0.f), sh = hm;
    if (h_mid) hm = *reinterpret_cast<const float4*>(h_mid + (size_t)t * H + h);
    if (h_mid && shared) sh = *reinterpret_cast<const float4*>(sh_row + h);
    float4 o = make_float4(0.f, 0.f, 0.f, 0.f);
#pragma unroll
    for (uint32_t r = 0; r < kPfMaxK; ++r)
      if (r < k) {
        o.x = __builtin_fmaf(d[r].x, wt[r], o.x);
        o.y = __builtin_fmaf(d[r].y, wt[r], o.y);
        o.z = __builtin_fmaf(d[r].z, wt[r], o.z);
        o.w = __builtin_fmaf(d[r].w, wt[r], o.w);
      }
    if (h_mid) {
      o.x = hm.x + o.x;
      o.y = hm.y + o.y;
      o.z = hm.z + o.z;
      o.w = hm.w + o.w;
      if (shared) {
        o.x = o.x + sg * sh.x;
        o.y = o.y + sg * sh.y;
        o.z = o.z + sg * sh.z;
        o.w = o.w + sg * sh.w;
      }
    }
    *reinterpret_cast<float4*>(out + (size_t)t * H + h) = o;
  }
}

// ---------------------------------------------------------------------------
// Host side.
// ---------------------------------------------------------------------------
static uint64_t al256(uint64_t n) { return (n + 255) & ~255ull; }

uint64_t prefill_workspace(uint32_t hidden, uint32_t inter, uint32_t group, uint32_t n_tokens,
                           uint32_t n_experts, uint32_t k, bool shared, PfArgs* a, uint8_t* base) {
  const uint64_t nk = (uint64_t)n_tokens * k;
  const uint64_t ns = shared ? (n_tokens + kPfMC - 1) / kPfMC : 0;  // shared-expert items
  const uint64_t ne = nk + (shared ? n_tokens : 0);                 // entry rows
  const uint64_t max_items = n_experts + nk / kPfMC + 1 + ns;
  uint64_t off = 0;
  auto take = [&](uint64_t bytes) {
    const uint64_t o = off;
    off += al256(bytes);
    return base ? base + o : nullptr;
  };
  uint8_t* p_items = take(max_items * 2 * 4);
  uint8_t* p_nitems = take(4);
  uint8_t* p_itok = take(max_items * kPfMC * 4);
  uint8_t* p_pw = take(nk * 8);
  uint8_t* p_xsum = take((uint64_t)n_tokens * (hidden / group) * 4);
  uint8_t* p_asum = take(ne * (inter / group) * 4);
  uint8_t* p_xhi = take((uint64_t)n_tokens * hidden * 2);
  uint8_t* p_xlo = take((uint64_t)n_tokens * hidden * 2);
  uint8_t* p_ahi = take(ne * inter * 2);
  uint8_t* p_down = take(ne * hidden * 4);
  uint8_t* p_xr = take(9 * 4);
  uint8_t* p_gs = take(shared ? (uint64_t)n_tokens * 4 : 0);
  uint8_t* p_sitems = take(ns * 2 * 4);
  uint8_t* p_snitems = take(shared ? 4 : 0);
  uint8_t* p_sitok = take(ns * kPfMC * 4);
  uint8_t* p_sxr = take(shared ? 9 * 4 : 0);
  if (a) {
    a->xr = reinterpret_cast<uint32_t*>(p_xr);
    a->gscore = shared ? reinterpret_cast<float*>(p_gs) : nullptr;
    a->sitems = shared ? reinterpret_cast<uint32_t*>(p_sitems) : nullptr;
    a->sn_items = shared ? reinterpret_cast<uint32_t*>(p_snitems) : nullptr;
    a->sitem_tok = shared ? reinterpret_cast<uint32_t*>(p_sitok) : nullptr;
    a->sxr = shared ? reinterpret_cast<uint32_t*>(p_sxr) : nullptr;
    a->items = reinterpret_cast<uint32_t*>(p_items);
    a->n_items = reinterpret_cast<uint32_t*>(p_nitems);
    a->item_tok = reinterpret_cast<uint32_t*>(p_itok);
    a->tok_pw = reinterpret_cast<uint2*>(p_pw);
    a->xsum = reinterpret_cast<float*>(p_xsum);
    a->asum = reinterpret_cast<float*>(p_asum);
    a->x_hi = reinterpret_cast<uint16_t*>(p_xhi);
    a->x_lo = reinterpret_cast<uint16_t*>(p_xlo);
    a->act_hi = reinterpret_cast<uint16_t*>(p_ahi);
    a->act_lo = nullptr;
    a->down = reinterpret_cast<float*>(p_down);
    a->max_items = (uint32_t)max_items;
  }
  return off;
}

bool prefill_supported(uint32_t hidden, uint32_t inter, uint32_t group, uint32_t bits,
                       uint32_t n_tokens, uint32_t n_experts, uint32_t k) {
  if (bits != 4 && bits != 3) return false;
  if (group != 32 && group != 64 && group != 128) return false;
  if (hidden % kPfKC || inter % kPfKC || hidden < kPfMinHidden) return false;
  if (hidden / group > kPfMaxGroupsK || inter / group > kPfMaxGroupsK) return false;
  if (n_tokens < 1 || n_tokens > kPfMaxTokens || n_experts < 1 || n_experts > kPfMaxExperts) return false;
  if (k < 1 || k > kPfMaxK || k > n_experts) return false;
  if ((uint64_t)n_tokens * k > 0xFFFFu) return false;
  return true;
}

template <int BITS, int G, int MODE, bool SPLIT, int KU, int NWD = 0>
static hipError_t launch_mm(const PfArgs& a, uint32_t n_units_max, uint32_t n_cu, hipStream_t st) {
  using C = PfMM<BITS, G, MODE, SPLIT, KU, NWD>;
  const auto fn = reinterpret_cast<const void*>(&k_pf_mm<BITS, G, MODE, SPLIT, KU, NWD>);
  const size_t lds = (size_t)C::LDS;
  static std::atomic<uint64_t> raised{0};
  const hipError_t e = raise_lds_limit(fn, (int)lds, raised);
  if (e != hipSuccess) return e;
  const uint32_t grid = n_units_max < n_cu ? n_units_max : n_cu;
  hipLaunchKernelGGL((k_pf_mm<BITS, G, MODE, SPLIT, KU, NWD>), dim3(grid), dim3(64 * C::NWT), lds, st, a,
                     (const uint32_t*)a.items, (const uint32_t*)a.n_items, (const uint32_t*)a.xr);
  return hipGetLastError();
}

// Per-unit scale staging (KU = K) where it fits in LDS: the A3B-shape gate/up
// GEMM (bf16 x, hidden 2048, group 64 or 128) and down GEMM (inter 512,
// group 64); other shapes copy scales per chunk.
// act_rows: the entry rows [row0, row0 + n_rows) whose activation group
// sums the G > 64 pass computes.
template <bool DOWN>
static hipError_t launch_gu64(const PfArgs& a, uint32_t n_units_max, uint32_t n_cu, hipStream_t st) {
  const auto fn = reinterpret_cast<const void*>(&k_pf_gu64<DOWN>);
  static std::atomic<uint64_t> raised{0};
  const hipError_t e = raise_lds_limit(fn, Gu64::LDS, raised);
  if (e != hipSuccess) return e;
  const uint32_t grid = n_units_max < n_cu ? n_units_max : n_cu;
  hipLaunchKernelGGL(k_pf_gu64<DOWN>, dim3(grid), dim3(64 * Gu64::NWT), (size_t)Gu64::LDS, st, a, (const uint32_t*)a.items,
                     (const uint32_t*)a.n_items, (const uint32_t*)a.xr);
  return hipGetLastError();
}

template <int BITS, int G>
static hipError_t launch_gemms(const PfArgs& a, uint32_t row0, uint32_t n_rows, uint32_t n_cu, hipStream_t st) {
  const uint32_t gu_units = a.max_items * (a.g.inter / 64);
  hipError_t e;
  // The 32 x 32 tiles take the chunks of a unit in pairs (their scales
  // come per pair): K a multiple of 512. Gate/up and down on them by
  // default; gemm_path 2 keeps the down GEMM on k_pf_mm.
  const bool tiles32 = BITS == 4 && G == 64 && a.gemm_path != 1;
  if (tiles32 && a.x_bf16 && a.g.inter % Gu64::NCOL == 0 && a.g.hidden % (2 * Gu64::KC) == 0)
    e = launch_gu64<false>(a, a.max_items * (a.g.inter / Gu64::NCOL), n_cu, st);
  else if (!a.x_bf16)
    e = launch_mm<BITS, G, 0, true, 0>(a, gu_units, n_cu, st);
  else if ((G == 64 || G == 128) && a.g.hidden == 2048)
    e = launch_mm<BITS, G, 0, false, (G == 64 || G == 128) ? 2048 : 0, (G == 64 || G == 128) ? 4 : 0>(a, gu_units, n_cu, st);
  else
    e = launch_mm<BITS, G, 0, false, 0>(a, gu_units, n_cu, st);
  if (e != hipSuccess) return e;
  // With G <= 64 the gate/up GEMM writes the activation group sums itself.
  if (G > 64) hipLaunchKernelGGL(k_pf_act_sum, dim3(n_rows), dim3(256), 0, st, a, row0);
  const uint32_t dn_units = a.max_items * (a.g.hidden / 256);
  if (tiles32 && a.gemm_path != 2 && a.g.hidden % Gu64::ROWS == 0 && a.g.inter % (2 * Gu64::KC) == 0)
    return launch_gu64<true>(a, a.max_items * (a.g.hidden / Gu64::ROWS), n_cu, st);
  if (G == 64 && a.g.inter == 512) return launch_mm<BITS, G, 2, false, G == 64 ? 512 : 0>(a, dn_units, n_cu, st);
  return launch_mm<BITS, G, 2, false, 0>(a, dn_units, n_cu, st);
}

hipError_t launch_prefill(const PfArgs& a, uint32_t n_cu, hipStream_t st) {
  const uint32_t route_lds = pf_route_lds(a.E, a.n_tokens);
  static std::atomic<uint64_t> raised{0};
  if (route_lds > 64 * 1024) {
    const hipError_t e = raise_lds_limit(reinterpret_cast<const void*>(&k_pf_route), (int)pf_route_lds(kPfMaxExperts, kPfMaxTokens), raised);
    if (e != hipSuccess) return e;
  }
  hipLaunchKernelGGL(k_pf_route, dim3(pf_bucket_blocks(a.n_tokens) + (a.n_tokens + kPfPrepTokens - 1) / kPfPrepTokens),
                     dim3(1024), route_lds, st, a);
  const uint32_t G = a.g.group, nk = a.n_tokens * a.k;
  const uint32_t rows = nk + (a.shared && a.shared_in_list ? a.n_tokens : 0u);
  hipError_t e;
  if (a.g.bits == 4)
    e = G == 32 ? launch_gemms<4, 32>(a, 0, rows, n_cu, st) : G == 64 ? launch_gemms<4, 64>(a, 0, rows, n_cu, st)
                                                              : launch_gemms<4, 128>(a, 0, rows, n_cu, st);
  else
    e = G == 32 ? launch_gemms<3, 32>(a, 0, rows, n_cu, st) : G == 64 ? launch_gemms<3, 64>(a, 0, rows, n_cu, st)
                                                              : launch_gemms<3, 128>(a, 0, rows, n_cu, st);
  if (e != hipSuccess) return e;
  if (a.shared && !a.shared_in_list) {
    // The 4-bit shared expert beside 3-bit routed experts: its own work list
    // through the 4-bit GEMM instances (entry rows n k + t).
    PfArgs s = a;
    s.g = a.sg;
    s.experts = a.shared;
    s.stride = 0;
    s.E = 1;
    s.items = a.sitems;
    s.n_items = a.sn_items;
    s.item_tok = a.sitem_tok;
    s.xr = a.sxr;
    s.max_items = (a.n_tokens + kPfMC - 1) / kPfMC;
    s.shared = nullptr;
    e = G == 32 ? launch_gemms<4, 32>(s, nk, a.n_tokens, n_cu, st)
                : G == 64 ? launch_gemms<4, 64>(s, nk, a.n_tokens, n_cu, st)
                          : launch_gemms<4, 128>(s, nk, a.n_tokens, n_cu, st);
    if (e != hipSuccess) return e;
  }
  hipLaunchKernelGGL(k_pf_combine, dim3(a.n_tokens), dim3(512), 0, st, a);
  return hipGetLastError();
}

// ---------------------------------------------------------------------------
// Dense quantized GEMM (affine_qmm_t, metal/lib.rs:684-734 QmmCall):
// y[n, N] = x[n, K] . dequant(W)[N, K]^T, run as the down-GEMM instance of
// k_pf_mm over one weight matrix: the "items" are 32-token row blocks of
// expert 0 at stride 0, A = x split into bf16 hi + lo in the MFMA order.
// ---------------------------------------------------------------------------
__global__ __launch_bounds__(256) void k_qmm_prep(const float* x, uint32_t n, uint32_t K, uint32_t G,
                                                  uint16_t* hi, uint16_t* lo, float* sums, uint32_t* items,
                                                  uint32_t* n_items) {
  __shared__ float part8[kPfMaxGroupsK * 128 / 8];
  const uint32_t r = blockIdx.x;
  for (uint32_t k0 = threadIdx.x * 8; k0 < K; k0 += blockDim.x * 8) {
    float f[8];
    const f32x4* p = reinterpret_cast<const f32x4*>(x + (size_t)r * K + k0);
    const f32x4 u = p[0], v = p[1];
    f[0] = u.x, f[1] = u.y, f[2] = u.z, f[3] = u.w, f[4] = v.x, f[5] = v.y, f[6] = v.z, f[7] = v.w;
    u32x4 h, l;
    split_f32(f, h, l);
    *reinterpret_cast<u32x4*>(hi + (size_t)r * K + k0) = h;
    *reinterpret_cast<u32x4*>(lo + (size_t)r * K + k0) = l;
    const uint32_t hv[4] = {h.x, h.y, h.z, h.w}, lv[4] = {l.x, l.y, l.z, l.w};
    float s = 0.f;
#pragma unroll
    for (int i = 0; i < 4; ++i)
      s += __uint_as_float(hv[i] << 16) + __uint_as_float(hv[i] & 0xFFFF0000u) + __uint_as_float(lv[i] << 16) +
           __uint_as_float(lv[i] & 0xFFFF0000u);
    part8[k0 / 8] = s;
  }
  __syncthreads();
  const uint32_t ng = K / G, per = G / 8;
  for (uint32_t g = threadIdx.x; g < ng; g += blockDim.x) {
    float s = 0.f;
    for (uint32_t j = 0; j < per; ++j) s += part8[g * per + j];
    sums[(size_t)r * ng + g] = s;
  }
  if (r == 0) {
    const uint32_t nb = (n + kPfMC - 1) / kPfMC;
    for (uint32_t i = threadIdx.x; i < nb; i += blockDim.x) {
      items[2 * i] = 0;
      items[2 * i + 1] = (i * kPfMC) | (min(kPfMC, n - i * kPfMC) << 16);
    }
    if (threadIdx.x == 0) *n_items = nb;
  }
}

uint64_t qmm_workspace(uint32_t in_dim, uint32_t group, uint32_t n_tokens, PfArgs* a, uint8_t* base) {
  const uint64_t n = n_tokens, nb = (n + kPfMC - 1) / kPfMC;
  uint64_t off = 0;
  auto take = [&](uint64_t bytes) {
    const uint64_t o = off;
    off += al256(bytes);
    return base ? base + o : nullptr;
  };
  uint8_t* p_items = take(nb * 2 * 4);
  uint8_t* p_nitems = take(4);
  uint8_t* p_sums = take(n * (in_dim / group) * 4);
  uint8_t* p_hi = take(n * in_dim * 2);
  uint8_t* p_lo = take(n * in_dim * 2);
  if (a) {
    a->items = reinterpret_cast<uint32_t*>(p_items);
    a->n_items = reinterpret_cast<uint32_t*>(p_nitems);
    a->asum = reinterpret_cast<float*>(p_sums);
    a->act_hi = reinterpret_cast<uint16_t*>(p_hi);
    a->act_lo = reinterpret_cast<uint16_t*>(p_lo);
    a->max_items = (uint32_t)nb;
  }
  return off;
}

bool qmm_supported(uint32_t in_dim, uint32_t out_dim, uint32_t group, uint32_t bits, uint32_t n_tokens) {
  if (bits != 4 && bits != 3) return false;
  if (group != 32 && group != 64 && group != 128) return false;
  if (in_dim % kPfKC || out_dim % 256 || in_dim / group > kPfMaxGroupsK || in_dim / 8 > kPfMaxGroupsK * 128 / 8)
    return false;
  return n_tokens >= 1 && n_tokens <= 0xFFFFu - kPfMC;
}

hipError_t launch_qmm(const PfArgs& a, const float* x, uint32_t n_cu, hipStream_t st) {
  hipLaunchKernelGGL(k_qmm_prep, dim3(a.n_tokens), dim3(256), 0, st, x, a.n_tokens, a.g.inter, a.g.group,
                     a.act_hi, a.act_lo, a.asum, a.items, a.n_items);
  const uint32_t units = a.max_items * (a.g.hidden / 256), G = a.g.group;
  if (a.g.bits == 4)
    return G == 32 ? launch_mm<4, 32, 1, true, 0>(a, units, n_cu, st)
                   : G == 64 ? launch_mm<4, 64, 1, true, 0>(a, units, n_cu, st)
                             : launch_mm<4, 128, 1, true, 0>(a, units, n_cu, st);
  return G == 32 ? launch_mm<3, 32, 1, true, 0>(a, units, n_cu, st)
                 : G == 64 ? launch_mm<3, 64, 1, true, 0>(a, units, n_cu, st)
                           : launch_mm<3, 128, 1, true, 0>(a, units, n_cu, st);
}

}  // namespace smoe
