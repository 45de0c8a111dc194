// fused.hip — one decode token through one MoE layer as three kernels
// (gfx950), meant to be replayed from a HIP graph.
//
// A decode layer has three all-to-all dependencies: the hidden state feeds
// every router row, the router's top-k feeds every expert row, and every
// activation feeds every down row. On MI355X the cheapest grid-wide
// synchronisation is a kernel boundary inside a graph (~1.6 us, and it
// makes the producer's stores visible through every XCD's L2); in-kernel
// broadcasts through agent-scope atomics cost 2.7-9 us at 256 consumer
// blocks and a cooperative grid.sync() ~33 us. So each dependency is one
// kernel boundary, and everything a kernel can compute redundantly instead
// of waiting for (RMSNorm's sum of squares, softmax and the top-k set) it
// computes in every wave.
//
// With T <= 4 tokens (multi-token decode), K_A reads each router row once
// for all T tokens (at hidden 4096, once per pair of tokens), and K_B / K_C
// run one grid slice per token (grid dimension y). Hidden 2048 or 4096: a
// lane holds HC = hidden / 2048 chunks of 32 values of every row it reads.
//
//   K_A  k_fa_route    one wave per router row: x = RMSNorm(r) * w (or the
//                      given input), logits[e] = W_e . x; 4 HC more waves
//                      per token store x as integer limbs for K_B
//                      (common.h, chunk_dot_i).
//   K_B  k_fa_gateup   one wave per RW rows of one routed slot: the slot's
//                      expert from the logits (every wave), then
//                      act[s, i] = silu(gate_i . x) * (up_i . x); one wave
//                      per RW rows of the shared expert (slot k), which
//                      needs no routing and so streams its rows while the
//                      routed waves select; one wave that publishes the
//                      route table (expert blobs and renormalised weights,
//                      the shared gate score gate . x) and, when asked,
//                      the reference's exact slot order.
//   K_C  k_fa_down     one block per kFaRB hidden rows, one lane per (slot,
//                      chunk of 32 activations): every slot's down rows,
//                      combined in table order moe = fma(out_s, w_s, moe)
//                      (deferred.rs:458-466) plus the shared term and the
//                      residual.
//
// Weights are read exactly once per token with 128-bit (4-bit) or 96-bit
// (3-bit) loads: non-temporal for the routed experts, temporal for the
// router rows and the shared expert (reused by every token, they stay in
// the memory-side cache); x limbs and logits (<= 18 KB) are re-read from
// L2 by every wave that needs them, and each K_C block stages the
// activations (<= 78 KB) in LDS once.
#include "common.h"
#include "kernels.h"
#include "topk.h"

namespace smoe {

// Hidden sizes of this path: HC x 2048, HC = 1 or 2 chunks of 32 values
// per lane (lane l holds chunks l + 64 h, h < HC).
constexpr uint32_t kFaH = 2048;              // hidden values per chunk column (64 lanes x 32)
// Work per wave / block. K_B waves take 4 gate/up row pairs (their sums
// are reduced together, gateup_rows); the K_C row count is a build-time
// tunable. Both are the measured best on MI355X (2 or 8 rows per K_B wave,
// 2 or 8 rows per K_C block: 0.4-1.4 us per layer slower).
constexpr int kFaRW = 4;                     // routed rows per K_B wave

// Optional timestamps (100 MHz s_memrealtime) for latency analysis. They
// stay in registers until fa_flush at the end of the kernel, so tracing adds
// no memory operation in between; with `drain` the wave first waits for all
// its outstanding memory operations.
struct FaClock {
  uint64_t t[6] = {0, 0, 0, 0, 0, 0};
};

__device__ __forceinline__ void fa_stamp(const FusedLayer& a, FaClock& c, int point, bool drain) {
  if (!a.trace) return;
  if (drain) __builtin_amdgcn_s_waitcnt(0);
  c.t[point] = __builtin_amdgcn_s_memrealtime();
}

__device__ __forceinline__ void fa_flush(const FusedLayer& a, const FaClock& c, int q) {
  if (!a.trace || threadIdx.x != 0) return;
  uint64_t* d = a.trace + ((size_t)q * kFaTraceBlocks + blockIdx.x) * kFaTracePoints;
#pragma unroll
  for (int p = 0; p < 6; ++p) d[p] = c.t[p];
}

// x chunk of this lane: the given input, or RMSNorm(r) * w (bf16 weights)
// with the sum of squares reduced over the wave (rms_norm_bf16_n_tokens_cpu,
// backend/cpu/mod.rs:406-430: inv = 1 / sqrt(sum_sq / dim + eps),
// x = r * inv * w), or r itself when w is null. The vector and the norm
// weights are loaded together (one memory round trip): a missing operand
// reads a harmless stand-in and is then ignored.
template <int HC>
struct FaX {
  float x[HC][kChunk];
  u32x4 w[HC][4];
};

template <int HC>
__device__ __forceinline__ void fa_x_load(const FusedLayer& a, int lane, FaX<HC>& f) {
  const float* src = a.x_in ? a.x_in : a.resid;
  const uint16_t* nw = a.norm ? a.norm : reinterpret_cast<const uint16_t*>(src);
#pragma unroll
  for (int h = 0; h < HC; ++h) {
    const size_t c = (size_t)lane + 64 * h;
    const u32x4* wp = reinterpret_cast<const u32x4*>(nw + c * kChunk);
#pragma unroll
    for (int i = 0; i < 4; ++i) f.w[h][i] = wp[i];
    load_x32(src + c * kChunk, f.x[h]);
  }
}

// 1 / rms of the hidden vector whose chunks every lane holds in f.x.
// Every rounding is written out (no contraction left to the compiler), so
// all instantiations (T = 1..4 tokens) compute x bit for bit alike.
template <int HC>
__device__ __forceinline__ float fa_inv_rms(const FusedLayer& a, const FaX<HC>& f) {
  float ss = 0.f;
#pragma unroll
  for (int h = 0; h < HC; ++h)
#pragma unroll
    for (int j = 0; j < kChunk; ++j) ss = __builtin_fmaf(f.x[h][j], f.x[h][j], ss);
  ss = readlane_f(group_sum_last<64>(ss), 63);
  return 1.0f / sqrtf(__builtin_fmaf(ss, 1.0f / (float)(HC * kFaH), a.eps));
}

// x[j] = r[j] * inv * w[j] for eight consecutive values (w: 8 bf16).
__device__ __forceinline__ void fa_norm8(float* x, float inv, const u32x4& w) {
  const uint32_t w4[4] = {w.x, w.y, w.z, w.w};
#pragma unroll
  for (int h = 0; h < 4; ++h) {
    x[2 * h] = x[2 * h] * inv * bf16f((uint16_t)(w4[h] & 0xFFFFu));
    x[2 * h + 1] = x[2 * h + 1] * inv * bf16f((uint16_t)(w4[h] >> 16));
  }
}

template <int HC>
__device__ __forceinline__ void fa_x_finish(const FusedLayer& a, FaX<HC>& f) {
  if (a.x_in || !a.norm) return;
  const float inv = fa_inv_rms<HC>(a, f);
#pragma unroll
  for (int h = 0; h < HC; ++h)
#pragma unroll
    for (int i = 0; i < 4; ++i) fa_norm8(f.x[h] + 8 * i, inv, f.w[h][i]);
}

// x as integer limbs (common.h, make_limbs) with four lanes per 32-value
// chunk: lane q of the quad holds values 8q .. 8q + 7 and writes limb words
// 2q and 2q + 1 of every limb; the chunk's exponent and sum come from the
// quad (DPP).
__device__ __forceinline__ void store_limbs_quad(uint32_t* dst, const float (&x)[8], int q, bool live = true) {
  float amax = 0.f;
#pragma unroll
  for (int j = 0; j < 8; ++j) amax = fmaxf(amax, fabsf(x[j]));
  amax = fmaxf(amax, dpp_f<0xB1>(amax, 0.f));  // quad lanes ^ 1
  amax = fmaxf(amax, dpp_f<0x4E>(amax, 0.f));  // quad lanes ^ 2
  const int f = amax > 0.f ? 22 - __builtin_amdgcn_frexp_expf(amax) : 0;
  int32_t d[3][8];
#pragma unroll
  for (int j = 0; j < 8; ++j) {
    const int32_t m = (int32_t)__builtin_rintf(__builtin_ldexpf(x[j], f));
    const int32_t d0 = (m << 24) >> 24;
    const int32_t m1 = (m - d0) >> 8;
    const int32_t d1 = (m1 << 24) >> 24;
    d[0][j] = d0;
    d[1][j] = d1;
    d[2][j] = (m1 - d1) >> 8;
  }
#pragma unroll
  for (int L = 0; L < 3; ++L) {
    uint2 v;
    v.x = pack_bytes(d[L][0], d[L][2], d[L][4], d[L][6]);
    v.y = pack_bytes(d[L][1], d[L][3], d[L][5], d[L][7]);
    if (live) *reinterpret_cast<uint2*>(dst + 8 * L + 2 * q) = v;
  }
  float xs = ((x[0] + x[1]) + (x[2] + x[3])) + ((x[4] + x[5]) + (x[6] + x[7]));
  xs += dpp_f<0xB1>(xs, 0.f);
  xs += dpp_f<0x4E>(xs, 0.f);
  if (q == 0 && live) {
    uint2 v;
    v.x = __float_as_uint(__builtin_ldexpf(1.0f, -f));
    v.y = __float_as_uint(xs);
    *reinterpret_cast<uint2*>(dst + 24) = v;
  }
}

// Token t's view of a multi-token layer: the same arguments with every
// per-token pointer moved to token t's rows. Branch-free (selects), so it
// adds no branch level in front of the first loads.
template <int HC>
__host__ __device__ __forceinline__ FusedLayer token_view(const FusedLayer& a, uint32_t t) {
  FusedLayer b = a;
  const size_t hs = (size_t)t * HC * kFaH;
  b.x_in = a.x_in ? a.x_in + hs : nullptr;
  b.resid = a.resid ? a.resid + hs : nullptr;
  b.h_mid += hs;
  b.out += hs;
  b.logits += (size_t)t * a.lstride;
  b.act += (size_t)t * a.astride;
  b.xl += (size_t)t * a.xstride;
  b.table += t;
  b.idx_out = a.idx_out ? a.idx_out + (size_t)t * a.k : nullptr;
  b.w_out = a.w_out ? a.w_out + (size_t)t * a.k : nullptr;
  return b;
}

// Pins the listed kernel arguments in SGPRs at this point, so that all their
// scalar loads go out as one batch before the first branch. Left to itself
// the compiler loads arguments lazily, one dependent batch per branch level,
// and every batch is a memory round trip: a kernel's argument block is not in
// L2 when the kernel starts.
#define FA_ARGS_IN_SGPRS(...) asm volatile("" ::__VA_ARGS__)

// A 2048-wide f32 row (router row or shared-expert gate), chunk c per lane.
// Router rows and the shared-gate row are read by every token, so they are
// loaded temporally: all 40 layers' routers and shared experts (155 MB at
// the A3B shape) then stay in the 256 MB memory-side cache while the routed
// experts stream past it non-temporally (measured on MI355X: a 2 MB
// temporal read after a 512 MB non-temporal stream takes 0.74 us, against
// 1.49 us from HBM).
template <int HC>
__device__ __forceinline__ void fa_row_load(const float* row, uint32_t lane, f32x4 (&wr)[HC][kChunk / 4]) {
#pragma unroll
  for (int h = 0; h < HC; ++h) {
    const f32x4* rp = reinterpret_cast<const f32x4*>(row + ((size_t)lane + 64 * h) * kChunk);
#pragma unroll
    for (int i = 0; i < kChunk / 4; ++i) wr[h][i] = ld_w<false>(rp + i);
  }
}

// An 8-bit row's chunks (chunk c = lane + 64 h): 32 code bytes and the
// bf16 scale and bias of the chunk's group (a group holds whole chunks),
// raw until fa_row_dequant_q8; loaded temporally like fa_row_load.
template <int HC>
struct FaQ8Row {
  u32x4 q[HC][2];
  uint32_t s[HC], b[HC];
};

template <int HC>
__device__ __forceinline__ void fa_row_load_q8(const Q8Rows& m, uint32_t row, uint32_t lane, FaQ8Row<HC>& o) {
  constexpr uint32_t K = HC * kFaH;
  const uint32_t gsh = __builtin_ctz(m.group);
#pragma unroll
  for (int h = 0; h < HC; ++h) {
    const uint32_t c = lane + 64 * h;
    const u32x4* p = reinterpret_cast<const u32x4*>(m.q + (size_t)row * K + (size_t)c * kChunk);
    o.q[h][0] = p[0];
    o.q[h][1] = p[1];
    const size_t gi = (size_t)row * (K >> gsh) + ((c * kChunk) >> gsh);
    o.s[h] = m.s[gi];
    o.b[h] = m.b[gi];
  }
}

// The row's weights fma(q, s, b) (dequant_matvec_8bit_gs_cpu, cpu_matvec.rs:
// 205-283; byte n of code word i is input 4 i + n) in fa_row_load's layout.
template <int HC>
__device__ __forceinline__ void fa_row_dequant_q8(const FaQ8Row<HC>& r, f32x4 (&wr)[HC][kChunk / 4]) {
#pragma unroll
  for (int h = 0; h < HC; ++h) {
    const float s = bf16f((uint16_t)r.s[h]), b = bf16f((uint16_t)r.b[h]);
#pragma unroll
    for (int i = 0; i < kChunk / 4; ++i) {
      const uint32_t w = r.q[h][i / 4][i % 4];
      wr[h][i] = f32x4{__builtin_fmaf((float)(w & 0xFFu), s, b), __builtin_fmaf((float)((w >> 8) & 0xFFu), s, b),
                       __builtin_fmaf((float)((w >> 16) & 0xFFu), s, b), __builtin_fmaf((float)(w >> 24), s, b)};
    }
  }
}

// row . x over the wave (valid in lane 63): four FMA chains per lane over
// its chunks, then the wave sum.
template <int HC>
__device__ __forceinline__ float fa_row_dot(const f32x4 (&wr)[HC][kChunk / 4], const float (&x)[HC][kChunk]) {
  float a0 = 0.f, a1 = 0.f, a2 = 0.f, a3 = 0.f;
#pragma unroll
  for (int h = 0; h < HC; ++h)
#pragma unroll
    for (int i = 0; i < kChunk / 4; ++i) {
      a0 = __builtin_fmaf(wr[h][i].x, x[h][4 * i + 0], a0);
      a1 = __builtin_fmaf(wr[h][i].y, x[h][4 * i + 1], a1);
      a2 = __builtin_fmaf(wr[h][i].z, x[h][4 * i + 2], a2);
      a3 = __builtin_fmaf(wr[h][i].w, x[h][4 * i + 3], a3);
    }
  return group_sum_last<64>((a0 + a1) + (a2 + a3));
}

// ---------------------------------------------------------------------------
// K_A: router logits for T tokens: each wave reads its
// router row once and applies it to every token's x. The last 4 HC T waves
// write x of the tokens as integer limbs for K_B. Q8: the router is 8-bit
// (r8); its row is dequantized in registers after the loads.
// ---------------------------------------------------------------------------
template <int T, int HC, bool Q8>
__device__ __forceinline__ void fa_route(const FusedLayer& a, const Q8Rows& r8) {
  FA_ARGS_IN_SGPRS("s"(a.x_in), "s"(a.resid), "s"(a.norm), "s"(a.eps), "s"(a.router), "s"(a.E),
                   "s"(a.logits), "s"(a.xl), "s"(a.trace), "s"(a.lstride), "s"(a.xstride));
  FaClock clk;
  fa_stamp(a, clk, 0, false);
  const int lane = threadIdx.x;
  const uint32_t w = blockIdx.x;
  const uint32_t nrouter = a.E;

  if (w >= nrouter) {
    // Limb waves, 4 HC per token: wave p of token t converts chunks
    // [16p, 16p + 16), four lanes per chunk (8 values each). Every lane also
    // loads its own chunks for the sum of squares.
    const uint32_t lw = w - nrouter;
    const FusedLayer at = token_view<HC>(a, lw / (4 * HC));
    const uint32_t ch = (lw % (4 * HC)) * 16 + (uint32_t)(lane >> 2);
    const int q = lane & 3;
    FaX<HC> f;
    fa_x_load<HC>(at, lane, f);
    const float* src = at.x_in ? at.x_in : at.resid;
    const uint16_t* nw = at.norm ? at.norm : reinterpret_cast<const uint16_t*>(src);
    const uint32_t e0 = ch * kChunk + q * 8;
    const f32x4 v0 = *reinterpret_cast<const f32x4*>(src + e0);
    const f32x4 v1 = *reinterpret_cast<const f32x4*>(src + e0 + 4);
    const u32x4 w8 = *reinterpret_cast<const u32x4*>(nw + e0);
    __builtin_amdgcn_sched_barrier(0);
    fa_stamp(a, clk, 3, true);
    float x[8] = {v0.x, v0.y, v0.z, v0.w, v1.x, v1.y, v1.z, v1.w};
    if (!at.x_in && at.norm) fa_norm8(x, fa_inv_rms<HC>(at, f), w8);
    store_limbs_quad(at.xl + (size_t)ch * kXLimbWords, x, q);
    fa_stamp(a, clk, 5, true);
    fa_flush(a, clk, 0);
    return;
  }
  f32x4 wr[HC][kChunk / 4];
  FaQ8Row<HC> wq;
  if constexpr (Q8)
    fa_row_load_q8<HC>(r8, w, lane, wq);
  else
    fa_row_load<HC>(a.router + (size_t)w * (HC * kFaH), lane, wr);
  FaX<HC> f[T];
#pragma unroll
  for (int t = 0; t < T; ++t) fa_x_load<HC>(token_view<HC>(a, t), lane, f[t]);
  __builtin_amdgcn_sched_barrier(0);
  fa_stamp(a, clk, 3, true);
  if constexpr (Q8) fa_row_dequant_q8<HC>(wq, wr);
#pragma unroll
  for (int t = 0; t < T; ++t) {
    const FusedLayer at = token_view<HC>(a, t);
    if (at.x_in || !at.norm) {
      const float s = fa_row_dot<HC>(wr, f[t].x);
      if (lane == 63) at.logits[w] = s;
    } else {
      // logit = (1 / rms(r)) * (W . (r * w)): the dot and the sum of
      // squares run side by side instead of the dot waiting for the norm.
      float rw[HC][kChunk];
#pragma unroll
      for (int hc = 0; hc < HC; ++hc)
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          const uint32_t w4[4] = {f[t].w[hc][i].x, f[t].w[hc][i].y, f[t].w[hc][i].z, f[t].w[hc][i].w};
#pragma unroll
          for (int h = 0; h < 4; ++h) {
            rw[hc][8 * i + 2 * h] = f[t].x[hc][8 * i + 2 * h] * bf16f((uint16_t)(w4[h] & 0xFFFFu));
            rw[hc][8 * i + 2 * h + 1] = f[t].x[hc][8 * i + 2 * h + 1] * bf16f((uint16_t)(w4[h] >> 16));
          }
        }
      float ss = 0.f;
#pragma unroll
      for (int hc = 0; hc < HC; ++hc)
#pragma unroll
        for (int j = 0; j < kChunk; ++j) ss = __builtin_fmaf(f[t].x[hc][j], f[t].x[hc][j], ss);
      const float dot = fa_row_dot<HC>(wr, rw);
      ss = group_sum_last<64>(ss);
      if (lane == 63)
        at.logits[w] = dot * (1.0f / sqrtf(__builtin_fmaf(ss, 1.0f / (float)(HC * kFaH), at.eps)));
    }
  }
  fa_stamp(a, clk, 4, false);
  fa_stamp(a, clk, 5, true);
  fa_flush(a, clk, 0);
}

template <int T, int HC>
__global__ __launch_bounds__(64) void k_fa_route(FusedLayer a) {
  fa_route<T, HC, false>(a, Q8Rows{});
}

// K_A of a layer with an 8-bit router (Q8) and / or an 8-bit shared-expert
// gate (g8.q set). Its own kernel, so that the f32 layers' kernels keep
// their argument block. With g8, one more wave (the last block) writes the
// gate row's weights fma(q, s, b) as f32 to gate_f32, which K_B's route
// table wave reads as an f32 gate: the same values, so the same gate score
// as a dot over the 8-bit row.
template <int T, int HC, bool Q8>
__global__ __launch_bounds__(64) void k_fa_route_q8(FusedLayer a, Q8Rows r8, Q8Rows g8, float* gate_f32) {
  if (g8.q && blockIdx.x == gridDim.x - 1) {
    const uint32_t lane = threadIdx.x;
    FaQ8Row<HC> q;
    fa_row_load_q8<HC>(g8, 0, lane, q);
    f32x4 wr[HC][kChunk / 4];
    fa_row_dequant_q8<HC>(q, wr);
#pragma unroll
    for (int h = 0; h < HC; ++h) {
      f32x4* o = reinterpret_cast<f32x4*>(gate_f32 + ((size_t)lane + 64 * h) * kChunk);
#pragma unroll
      for (int i = 0; i < kChunk / 4; ++i) o[i] = wr[h][i];
    }
    return;
  }
  fa_route<T, HC, Q8>(a, r8);
}

// The E logits, P per lane (lane l holds [l*P, l*P + P)); positions >= E
// read as -inf. The logits buffer holds at least 64 * P floats per token.
template <int P>
__device__ __forceinline__ void load_logits(const float* logits, uint32_t E, int lane, float (&v)[P]) {
  if constexpr (P == 4 || P == 8) {
#pragma unroll
    for (int h = 0; h < P / 4; ++h) {
      const f32x4 q = *reinterpret_cast<const f32x4*>(logits + lane * P + 4 * h);
      v[4 * h] = q.x;
      v[4 * h + 1] = q.y;
      v[4 * h + 2] = q.z;
      v[4 * h + 3] = q.w;
    }
  } else {
#pragma unroll
    for (int e = 0; e < P; ++e) v[e] = logits[lane * P + e];
  }
#pragma unroll
  for (int e = 0; e < P; ++e)
    if ((uint32_t)(lane * P + e) >= E) v[e] = -INFINITY;
}

// gate and up rows [r0, r0 + kFaRW) of one expert blob against x (limbs),
// SwiGLU, stored to act[r0 ..]. All loads are issued before any arithmetic.
// NT: non-temporal weight loads (routed experts) or temporal (the shared
// expert, reused by every token).
template <int BITS, bool NT, int HC>
__device__ __forceinline__ void gateup_rows(const FusedLayer& a, FaClock& clk, const uint8_t* blob,
                                            const BlobGeom& g, uint32_t r0, int lane,
                                            const XLimbs (&xl)[HC], float* act) {
  constexpr int CB = chunk_bytes<BITS>();
  constexpr uint32_t RB = HC * kFaH / kChunk * CB;  // row bytes
  const uint32_t gpr = HC * kFaH / g.group;
  const uint32_t cps = __builtin_ctz(g.group / kChunk);
  Raw<BITS> rg[kFaRW][HC], ru[kFaRW][HC];
  uint16_t sg[kFaRW][HC], bg[kFaRW][HC], su[kFaRW][HC], bu[kFaRW][HC];
#pragma unroll
  for (int p = 0; p < kFaRW; ++p) {
    const uint32_t row = r0 + p;
#pragma unroll
    for (int h = 0; h < HC; ++h) {
      const uint32_t c = lane + 64 * h;
      // Scalar row bases, 32-bit lane offsets.
      const uint32_t oc = lane_off(c * CB), os = lane_off((c >> cps) * 2);
      const size_t rs = (size_t)row * gpr * 2;
      rg[p][h] = load_raw<BITS, NT>(blob + g.w[0] + (size_t)row * RB + oc);
      ru[p][h] = load_raw<BITS, NT>(blob + g.w[1] + (size_t)row * RB + oc);
      sg[p][h] = *reinterpret_cast<const uint16_t*>(blob + g.s[0] + rs + os);
      bg[p][h] = *reinterpret_cast<const uint16_t*>(blob + g.b[0] + rs + os);
      su[p][h] = *reinterpret_cast<const uint16_t*>(blob + g.s[1] + rs + os);
      bu[p][h] = *reinterpret_cast<const uint16_t*>(blob + g.b[1] + rs + os);
    }
  }
  __builtin_amdgcn_sched_barrier(0);
  fa_stamp(a, clk, 3, true);
  float gp[kFaRW], up[kFaRW];
#pragma unroll
  for (int p = 0; p < kFaRW; ++p) {
    gp[p] = chunk_dot_i<BITS>(rg[p][0], xl[0], bf16f(sg[p][0]), bf16f(bg[p][0]));
    up[p] = chunk_dot_i<BITS>(ru[p][0], xl[0], bf16f(su[p][0]), bf16f(bu[p][0]));
#pragma unroll
    for (int h = 1; h < HC; ++h) {
      gp[p] += chunk_dot_i<BITS>(rg[p][h], xl[h], bf16f(sg[p][h]), bf16f(bg[p][h]));
      up[p] += chunk_dot_i<BITS>(ru[p][h], xl[h], bf16f(su[p][h]), bf16f(bu[p][h]));
    }
  }
  // The eight rows' lane partials are summed together: after the two swaps
  // the 16-lane rows hold gate/up rows 0, 2, 1, 3, and every lane of a row
  // ends with its totals, so one SwiGLU serves all four outputs.
  const float gs = row_sum16_all(swap16_add(swap32_add(gp[0], gp[1]), swap32_add(gp[2], gp[3])));
  const float us = row_sum16_all(swap16_add(swap32_add(up[0], up[1]), swap32_add(up[2], up[3])));
  const float v = silu_mul(gs, us);
  const int row16 = lane >> 4;
  if ((lane & 15) == 0) act[r0 + ((row16 >> 1) | ((row16 & 1) << 1))] = v;
}

// ---------------------------------------------------------------------------
// K_B: routed gate/up, shared-expert gate/up and the route table.
//
// Blocks [0, k * tiles): one routed slot's kFaRW rows. The wave takes its
// slot's expert from the logits (topk_slot_logits: ascending index order;
// the exact scan when the set is ambiguous), then its rows.
// Blocks [k * tiles, k * tiles + tiles): the shared expert's rows (slot k),
// with no routing dependency, so their loads overlap the top-k of the
// routed waves.
// Last block: the route table (expert blobs, renormalised weights, shared
// gate score) in the order the act slots use, and, when asked, the
// reference's exact slot order.
// ---------------------------------------------------------------------------
template <int BITS, int P, int KC, int HC>
__global__ __launch_bounds__(64) void k_fa_gateup(FusedLayer a_all) {
  FA_ARGS_IN_SGPRS("s"(a_all.logits), "s"(a_all.xl), "s"(a_all.act), "s"(a_all.table), "s"(a_all.E),
                   "s"(a_all.k), "s"(a_all.normalize), "s"(a_all.experts), "s"(a_all.stride),
                   "s"(a_all.shared), "s"(a_all.gate), "s"(a_all.idx_out), "s"(a_all.w_out),
                   "s"(a_all.trace), "s"(a_all.lstride), "s"(a_all.astride), "s"(a_all.xstride),
                   "s"(a_all.routed.inter), "s"(a_all.routed.group), "s"(a_all.routed.w[0]),
                   "s"(a_all.routed.w[1]), "s"(a_all.routed.s[0]), "s"(a_all.routed.s[1]),
                   "s"(a_all.routed.b[0]), "s"(a_all.routed.b[1]));
  FA_ARGS_IN_SGPRS("s"(a_all.sgeom.group), "s"(a_all.sgeom.w[0]), "s"(a_all.sgeom.w[1]),
                   "s"(a_all.sgeom.s[0]), "s"(a_all.sgeom.s[1]), "s"(a_all.sgeom.b[0]),
                   "s"(a_all.sgeom.b[1]));
  const FusedLayer a = token_view<HC>(a_all, blockIdx.y);
  __shared__ int32_t sid[kMaxK];
  __shared__ float sval[kMaxK];
  __shared__ float sprob[64 * P];  // the exact softmax's values (softmax_ref)
  FaClock clk;
  fa_stamp(a, clk, 0, false);
  const int lane = threadIdx.x;
  const uint32_t I = a.routed.inter, E = a.E, k = a.k;
  const uint32_t tiles = I / kFaRW;
  const uint32_t nrouted = k * tiles;
  const uint32_t nshared = a.shared ? tiles : 0u;

  if (blockIdx.x < nrouted) {
    // tiles is a power of two (inter 512 or 1024): shifts, no division.
    const uint32_t tsh = __builtin_ctz(tiles);
    const uint32_t slot = blockIdx.x >> tsh;
    const uint32_t r0 = (blockIdx.x & (tiles - 1)) * kFaRW;
    float v[P];
    load_logits<P>(a.logits, E, lane, v);
    XLimbs xl[HC];
#pragma unroll
    for (int h = 0; h < HC; ++h) load_limbs(a.xl + ((size_t)lane + 64 * h) * kXLimbWords, xl[h]);
    fa_stamp(a, clk, 1, true);
    int32_t id;
    if (!topk_slot_logits<P, KC>(v, E, k, slot, lane, id)) {
      // Ambiguous set (a tie or a near-tie at the k/k+1 boundary, NaN): the
      // reference's probabilities bit for bit and its running-minimum scan.
      softmax_ref<P>(v, E, lane, sprob, load_exp_tab(lane));
      exact_topk<P>(v, k, lane, sid, sval);
      __syncthreads();
      id = sid[slot];
    }
    fa_stamp(a, clk, 2, false);
    gateup_rows<BITS, true, HC>(a, clk, a.experts + (uint64_t)id * a.stride, a.routed, r0, lane, xl,
                                a.act + (size_t)slot * I);
  } else if (blockIdx.x < nrouted + nshared) {
    const uint32_t r0 = (blockIdx.x - nrouted) * kFaRW;
    XLimbs xl[HC];
#pragma unroll
    for (int h = 0; h < HC; ++h) load_limbs(a.xl + ((size_t)lane + 64 * h) * kXLimbWords, xl[h]);
    gateup_rows<4, false, HC>(a, clk, a.shared, a.sgeom, r0, lane, xl, a.act + (size_t)k * I);
  } else {
    // Route table (normalize_weights, moe_router.rs:130-141). The
    // reference's probabilities bit for bit (softmax_ref) wherever they
    // decide the set or are returned to the caller.
    // The shared-expert gate score gate . x is computed here, off the
    // critical path (in the router kernel its extra wave ended last): its
    // loads go out with the logits'.
    const bool gated = a.gate != nullptr;
    f32x4 gw[HC][kChunk / 4];
    FaX<HC> gx;
    const ExpTabReg tab = load_exp_tab(lane);
    fa_row_load<HC>(gated ? a.gate : a.router, lane, gw);
    fa_x_load<HC>(a, lane, gx);
    float v[P];
    load_logits<P>(a.logits, E, lane, v);
    const bool is_set = topk_set_logits<P, KC>(v, E, k, lane, sid);
    float lg[P];  // the logits, for the caller's exact slot order below
#pragma unroll
    for (int e = 0; e < P; ++e) lg[e] = v[e];
    if (is_set) {
      // Unambiguous set: the weights only enter the combine (compared within
      // a tolerance), so the fast softmax; the exact one's sequential sum
      // would make this wave the last of the kernel. The same whether or
      // not the caller asks for idx / weights, so the combine does not
      // depend on it.
      wave_softmax_fast<P>(v, E, lane);
#pragma unroll
      for (int e = 0; e < P; ++e) sprob[lane * P + e] = v[e];
    } else {
      softmax_ref<P>(v, E, lane, sprob, tab);
      exact_topk<P>(v, k, lane, sid, sval);
    }
    __syncthreads();
    if (is_set && lane < (int)k) sval[lane] = sprob[sid[lane]];
    __syncthreads();
    if (lane < (int)k) {
      float wt = sval[lane];
      if (a.normalize) {
        float sum = 0.f;
        for (uint32_t i = 0; i < k; ++i) sum += sval[i];
        if (sum > 0.f) wt = sval[lane] * (1.0f / sum);
      }
      a.table->blob[lane] = a.experts + (uint64_t)sid[lane] * a.stride;
      a.table->weight[lane] = wt;
    }
    fa_x_finish<HC>(a, gx);
    const float gate_dot = readlane_f(fa_row_dot<HC>(gw, gx.x), 63);
    const float gate_score = gated ? gate_dot : __builtin_nanf("");
    if (lane == 0) {
      a.table->k = k;
      a.table->has_shared = a.shared != nullptr;
      if (a.shared) {
        a.table->blob[k] = a.shared;
        a.table->weight[k] = 1.0f;
      }
      a.table->shared_gate = gate_score;
    }
    if (a.idx_out || a.w_out) {
      // The reference's exact slot order for the caller.
      __shared__ int32_t eid[kMaxK];
      __shared__ float evl[kMaxK];
      if (is_set) {
        __syncthreads();  // sprob is reused
        softmax_ref<P>(lg, E, lane, sprob, tab);
        exact_topk<P>(lg, k, lane, eid, evl);
      } else if (lane < (int)k) {
        eid[lane] = sid[lane];
        evl[lane] = sval[lane];
      }
      __syncthreads();
      if (lane < (int)k) {
        float wt = evl[lane];
        if (a.normalize) {
          float sum = 0.f;
          for (uint32_t i = 0; i < k; ++i) sum += evl[i];
          if (sum > 0.f) wt = evl[lane] * (1.0f / sum);
        }
        if (a.idx_out) a.idx_out[lane] = eid[lane];
        if (a.w_out) a.w_out[lane] = wt;
      }
    }
  }
  fa_stamp(a, clk, 4, false);
  fa_stamp(a, clk, 5, true);
  fa_flush(a, clk, 1);
}

// ---------------------------------------------------------------------------
// K_C: down rows of every slot + combine + residual.
//
// One block per kFaRB = 8 hidden rows. Every block needs all (k + 1) * inter
// activations, so a block stages them in LDS once (one cooperative load, a
// quarter of what per-wave loads would move through the vector L1), as
// integer limbs: four lanes per 32-activation chunk convert it while the
// weights are in flight (common.h, make_limbs; the same block floating
// point as x in K_B), and every lane's dots then run on v_dot4c_i32_i8
// (chunk_dot_i) instead of converting each code to a float.
//
// Lanes are slot-major: lane (s, c) owns chunk c (LI = inter / 32 chunks per
// row) of slot s. Routed waves: ceil(k / SPW) slot groups (SPW = 64 / LI
// slots per wave) x H row parts, so a lane covers 8 / H rows (H = 2 while the
// block stays within 16 waves, else 1); one shared-expert wave (4-bit) splits
// its 64 lanes into 64 / LI row groups. Loads go out in dependency order:
// the expert pointers (route table), the activation staging, then, once the
// pointers land, every row's codes, scales and biases; the staging is
// converted and written to LDS while the weights are in flight.
// Per-(row, slot) sums go through LDS to 8 combine threads, which apply the
// reference's order: moe = fma(out_s, w_s, moe) over the routed slots, then
// the shared term and the residual (deferred.rs:441-490).
// ---------------------------------------------------------------------------
constexpr int kFaRB = 8;           // hidden rows per K_C block
constexpr int kFaStageRounds = 4;  // staged chunks per quad of threads, at most
constexpr int kChunkPad = 36;      // LDS dwords per staged chunk (conflict-free 16-byte reads)

template <int BITS, int NR>
struct DownLoads {
  Raw<BITS> raw[NR];
  uint16_t sr[NR], br[NR];
};

template <int BITS, int LI, int NR, bool NT = true>
__device__ __forceinline__ void down_load(const uint8_t* blob, const BlobGeom& g, uint32_t row0,
                                          uint32_t c, DownLoads<BITS, NR>& d) {
  constexpr int CB = chunk_bytes<BITS>();
  constexpr uint32_t RB = LI * CB;
  const uint32_t gpr = g.inter >> __builtin_ctz(g.group);  // groups are powers of two
  const uint32_t cps = __builtin_ctz(g.group / kChunk);
  const gbytes gb = as_global(blob);
#pragma unroll
  for (int r = 0; r < NR; ++r) {
    const uint32_t row = row0 + r;
    d.raw[r] = load_raw_g<BITS, NT>(gb + g.w[2] + (size_t)row * RB + c * CB);
    const size_t gi = ((size_t)row * gpr + (c >> cps)) * 2;
    d.sr[r] = gld<false, uint16_t>(gb + g.s[2] + gi);
    d.br[r] = gld<false, uint16_t>(gb + g.b[2] + gi);
  }
}

// The NR rows' sums of this lane's chunk (limbs in LDS), each reduced over
// the LI lanes of its slot (valid in the last lane of the group).
template <int BITS, int LI, int NR>
__device__ __forceinline__ void down_dot(const DownLoads<BITS, NR>& d, const uint32_t* limbs, float (&o)[NR]) {
  XLimbs xl;
  load_limbs(limbs, xl);
#pragma unroll
  for (int r = 0; r < NR; ++r)
    o[r] = group_sum_last<LI>(chunk_dot_i<BITS>(d.raw[r], xl, bf16f(d.sr[r]), bf16f(d.br[r])));
}

// Routed row parts per K_C block: 2 while 2 * ceil(k / SPW) + 1 waves fit in
// 16, else 1.
template <int LI>
__host__ __device__ constexpr uint32_t fa_down_parts(uint32_t k) {
  return 2u * ((k + kWave / LI - 1) / (kWave / LI)) + 1u <= 16u ? 2u : 1u;
}

template <int BITS, int LI, int H, int HC>
__global__ __launch_bounds__(1024) void k_fa_down(FusedLayer a_all) {
  FA_ARGS_IN_SGPRS("s"(a_all.act), "s"(a_all.table), "s"(a_all.h_mid), "s"(a_all.out), "s"(a_all.trace),
                   "s"(a_all.k), "s"(a_all.shared), "s"(a_all.astride), "s"(a_all.routed.inter),
                   "s"(a_all.routed.group), "s"(a_all.routed.w[2]), "s"(a_all.routed.s[2]),
                   "s"(a_all.routed.b[2]), "s"(a_all.sgeom.inter), "s"(a_all.sgeom.group),
                   "s"(a_all.sgeom.w[2]), "s"(a_all.sgeom.s[2]), "s"(a_all.sgeom.b[2]));
  const FusedLayer a = token_view<HC>(a_all, blockIdx.y);
  constexpr int SPW = kWave / LI;
  constexpr int NR = kFaRB / H;             // rows per routed lane
  constexpr int NRS = kFaRB / (kWave / LI); // rows per shared lane
  extern __shared__ f32x4 sact4[];          // staged activation limbs, kChunkPad dwords per chunk
  __shared__ float so[kFaRB][kMaxSlots];
  __shared__ float sw[kMaxSlots];
  FaClock clk;
  fa_stamp(a, clk, 0, false);
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const uint32_t k = a.k;
  const uint32_t rwaves = (k + SPW - 1) / SPW * H;
  const uint32_t row0 = blockIdx.x * kFaRB;
  const uint32_t c = lane % LI;
  const uint32_t I = a.routed.inter;
  const bool routed = (uint32_t)wave < rwaves;

  // Combine threads: residual, routing weights and the shared-expert gate.
  float hm = 0.f, wk = 0.f, gate = 0.f;
  if (threadIdx.x < (unsigned)kFaRB) {
    hm = a.h_mid[row0 + threadIdx.x];
    gate = a.table->shared_gate;
  }
  if (threadIdx.x < k) wk = a.table->weight[threadIdx.x];

  // Lane roles. Routed: slot group wave / H, rows part wave % H; lanes of a
  // slot >= k compute slot 0 and store nothing. Shared: row group lane / LI.
  const uint32_t slot = routed ? (wave / H) * SPW + lane / LI : k;
  const bool valid = routed ? slot < k : true;
  const uint32_t sl = valid ? slot : 0u;
  const uint32_t lrow0 = routed ? row0 + (wave % H) * NR : row0 + (lane / LI) * NRS;
  const uint8_t* blob = routed ? a.table->blob[sl] : a.shared;

  // Activation staging: quad qd of the block's threads takes chunks qd,
  // qd + nquads, ...; lane q of the quad loads values 8q .. 8q + 7 of its
  // chunk (quads past the last chunk reload it and store nothing).
  const uint32_t nch = (k + (a.shared ? 1u : 0u)) * (I / kChunk);
  const uint32_t nquads = blockDim.x >> 2, qd = threadIdx.x >> 2;
  const int q = threadIdx.x & 3;
  const f32x4* act4 = reinterpret_cast<const f32x4*>(a.act);
  f32x4 st[kFaStageRounds][2];
#pragma unroll
  for (int i = 0; i < kFaStageRounds; ++i) {
    const uint32_t ch = min(qd + i * nquads, nch - 1);
    st[i][0] = act4[ch * 8 + 2 * q];
    st[i][1] = act4[ch * 8 + 2 * q + 1];
  }
  uint32_t* slimbs = reinterpret_cast<uint32_t*>(sact4);
  const auto stage = [=](void) {
#pragma unroll
    for (int i = 0; i < kFaStageRounds; ++i) {
      const uint32_t ch = qd + i * nquads;
      if (i * nquads >= nch) break;  // uniform: no quad has a chunk this round
      const float x[8] = {st[i][0].x, st[i][0].y, st[i][0].z, st[i][0].w,
                          st[i][1].x, st[i][1].y, st[i][1].z, st[i][1].w};
      store_limbs_quad(slimbs + (size_t)min(ch, nch - 1) * kChunkPad, x, q, ch < nch);
    }
  };

  fa_stamp(a, clk, 1, true);
  // One barrier on either path: the staging is complete in LDS after it.
  if (routed) {
    DownLoads<BITS, NR> d;
    down_load<BITS, LI, NR>(blob, a.routed, lrow0, c, d);
    stage();
    __syncthreads();
    fa_stamp(a, clk, 3, true);
    float od[NR];
    down_dot<BITS, LI, NR>(d, slimbs + (sl * (I / kChunk) + c) * kChunkPad, od);
    if (c == LI - 1 && valid) {
#pragma unroll
      for (int r = 0; r < NR; ++r) so[lrow0 - row0 + r][slot] = od[r];
    }
  } else {
    DownLoads<4, NRS> d;
    down_load<4, LI, NRS, false>(blob, a.sgeom, lrow0, c, d);
    stage();
    __syncthreads();
    float od[NRS];
    down_dot<4, LI, NRS>(d, slimbs + (k * (I / kChunk) + c) * kChunkPad, od);
    if (c == LI - 1) {
#pragma unroll
      for (int r = 0; r < NRS; ++r) so[lrow0 - row0 + r][k] = od[r];
    }
  }
  if (threadIdx.x < k) sw[threadIdx.x] = wk;
  // The gate's sigmoid is ready before the partial sums are.
  const float sig = sigmoidf_ref(gate);
  fa_stamp(a, clk, 4, false);
  __syncthreads();
  if (threadIdx.x < (unsigned)kFaRB) {
    const uint32_t r = threadIdx.x;
    float moe = 0.f;
    for (uint32_t s = 0; s < k; ++s) moe = __builtin_fmaf(so[r][s], sw[s], moe);
    float sum = moe;
    if (a.shared) {
      const float sh = so[r][k];
      sum = __builtin_isnan(gate) ? moe + sh : __builtin_fmaf(sh, sig, moe);
    }
    a.out[row0 + r] = hm + sum;
  }
  fa_stamp(a, clk, 5, true);
  fa_flush(a, clk, 2);
}

// ---------------------------------------------------------------------------
// Host side.
// ---------------------------------------------------------------------------
bool fused_supported(uint32_t hidden, uint32_t inter, uint32_t group, uint32_t bits,
                     uint32_t n_experts, uint32_t k) {
  if (hidden != kFaH && hidden != 2 * kFaH) return false;
  if (inter != 512 && inter != 1024) return false;
  if (group % kChunk != 0 || (group & (group - 1)) != 0 || inter % group != 0) return false;
  if (bits != 4 && bits != 3) return false;
  if (n_experts < 1 || n_experts > kFaMaxExperts || k < 1 || k > (uint32_t)kMaxK || k > n_experts) return false;
  return true;
}

// K_B instance: logits per lane P = ceil(E / 64); k = 8 (the A3B and OLMoE
// shapes) and k = 10 (Qwen3.5-397B-A17B) have their own instances with
// unrolled top-k rounds.
template <int BITS, int KC, int HC>
static void launch_gateup_fa_k(const FusedLayer& a, uint32_t blocks, hipStream_t st) {
  const uint32_t p = (a.E + 63) / 64;
  const dim3 grid(blocks, a.n_tokens);
  if (p <= 1)
    hipLaunchKernelGGL((k_fa_gateup<BITS, 1, KC, HC>), grid, dim3(64), 0, st, a);
  else if (p <= 2)
    hipLaunchKernelGGL((k_fa_gateup<BITS, 2, KC, HC>), grid, dim3(64), 0, st, a);
  else if (p <= 4)
    hipLaunchKernelGGL((k_fa_gateup<BITS, 4, KC, HC>), grid, dim3(64), 0, st, a);
  else
    hipLaunchKernelGGL((k_fa_gateup<BITS, 8, KC, HC>), grid, dim3(64), 0, st, a);
}

template <int BITS, int HC>
static void launch_gateup_fa(const FusedLayer& a, uint32_t blocks, hipStream_t st) {
  if (a.k == 8)
    launch_gateup_fa_k<BITS, 8, HC>(a, blocks, st);
  else if (a.k == 10)
    launch_gateup_fa_k<BITS, 10, HC>(a, blocks, st);
  else
    launch_gateup_fa_k<BITS, 0, HC>(a, blocks, st);
}

// K_C launch: 8 rows per block; LDS for the staged activations. Blocks of
// more than 64 KB (k = 16 at inter 1024) need the attribute raised (once
// per device).
template <int BITS, int LI, int H, int HC>
static hipError_t launch_down_fa_h(const FusedLayer& a, hipStream_t st) {
  constexpr uint32_t SPW = kWave / LI;
  const uint32_t waves = (a.k + SPW - 1) / SPW * H + (a.shared ? 1u : 0u);
  const uint32_t chunks = (a.k + (a.shared ? 1u : 0u)) * (a.routed.inter / kChunk);
  const size_t lds = (size_t)chunks * kChunkPad * sizeof(uint32_t);
  // Every staged chunk has a quad of threads (kFaStageRounds chunks per quad
  // at most); true for all k <= 16 and inter 512 / 1024, checked anyway.
  if (chunks > (uint32_t)kFaStageRounds * waves * (kWave / 4) || waves > 16 || lds > 96 * 1024)
    return hipErrorInvalidValue;
  static std::atomic<uint64_t> raised{0};
  if (lds > 64 * 1024) {
    const hipError_t e =
        raise_lds_limit(reinterpret_cast<const void*>(&k_fa_down<BITS, LI, H, HC>), 96 * 1024, raised);
    if (e != hipSuccess) return e;
  }
  hipLaunchKernelGGL((k_fa_down<BITS, LI, H, HC>), dim3(HC * kFaH / kFaRB, a.n_tokens), dim3(waves * kWave), lds,
                     st, a);
  return hipSuccess;
}

template <int BITS, int LI, int HC>
static hipError_t launch_down_fa(const FusedLayer& a, hipStream_t st) {
  return fa_down_parts<LI>(a.k) == 2 ? launch_down_fa_h<BITS, LI, 2, HC>(a, st)
                                     : launch_down_fa_h<BITS, LI, 1, HC>(a, st);
}

template <int HC, bool Q8>
static void launch_route_q8(const FusedLayer& a, const FaQ8& q, uint32_t grid, hipStream_t st) {
  switch (a.n_tokens) {
    case 1:
      hipLaunchKernelGGL((k_fa_route_q8<1, HC, Q8>), dim3(grid), dim3(64), 0, st, a, q.router, q.gate, q.gate_f32);
      break;
    case 2:
      hipLaunchKernelGGL((k_fa_route_q8<2, HC, Q8>), dim3(grid), dim3(64), 0, st, a, q.router, q.gate, q.gate_f32);
      break;
    case 3:
      if constexpr (HC == 1)
        hipLaunchKernelGGL((k_fa_route_q8<3, HC, Q8>), dim3(grid), dim3(64), 0, st, a, q.router, q.gate,
                           q.gate_f32);
      break;
    default:
      if constexpr (HC == 1)
        hipLaunchKernelGGL((k_fa_route_q8<4, HC, Q8>), dim3(grid), dim3(64), 0, st, a, q.router, q.gate,
                           q.gate_f32);
      break;
  }
}

// K_A over a.n_tokens tokens. At hidden 4096 a router wave holds two
// tokens' x at most (289 VGPRs), so 3 or 4 tokens take two launches of 2
// and n - 2 tokens (the router rows are read twice, from the memory-side
// cache the second time).
template <int HC>
static void launch_route_fa(const FusedLayer& a, const FaQ8& q, hipStream_t st) {
  if (HC == 2 && a.n_tokens > 2) {
    FusedLayer lo = a, hi = token_view<HC>(a, 2);
    lo.n_tokens = 2;
    hi.n_tokens = a.n_tokens - 2;
    launch_route_fa<HC>(lo, q, st);
    launch_route_fa<HC>(hi, q, st);
    return;
  }
  const uint32_t ka = a.E + 4u * HC * a.n_tokens;
  if (!q.router.q && !q.gate.q) {
    switch (a.n_tokens) {
      case 1: hipLaunchKernelGGL((k_fa_route<1, HC>), dim3(ka), dim3(64), 0, st, a); break;
      case 2: hipLaunchKernelGGL((k_fa_route<2, HC>), dim3(ka), dim3(64), 0, st, a); break;
      case 3:
        if constexpr (HC == 1) hipLaunchKernelGGL((k_fa_route<3, HC>), dim3(ka), dim3(64), 0, st, a);
        break;
      default:
        if constexpr (HC == 1) hipLaunchKernelGGL((k_fa_route<4, HC>), dim3(ka), dim3(64), 0, st, a);
        break;
    }
    return;
  }
  const uint32_t kq = ka + (q.gate.q ? 1u : 0u);
  if (q.router.q)
    launch_route_q8<HC, true>(a, q, kq, st);
  else
    launch_route_q8<HC, false>(a, q, kq, st);
}

template <int HC>
static hipError_t launch_fused_layer_h(const FusedLayer& a, const FaQ8& q, hipStream_t st) {
  const uint32_t I = a.routed.inter;
  launch_route_fa<HC>(a, q, st);
  const uint32_t kb = (a.k + (a.shared ? 1u : 0u)) * (I / kFaRW) + 1u;
  if (a.routed.bits == 4)
    launch_gateup_fa<4, HC>(a, kb, st);
  else
    launch_gateup_fa<3, HC>(a, kb, st);
  hipError_t e;
  if (a.routed.bits == 4)
    e = I == 512 ? launch_down_fa<4, 16, HC>(a, st) : launch_down_fa<4, 32, HC>(a, st);
  else
    e = I == 512 ? launch_down_fa<3, 16, HC>(a, st) : launch_down_fa<3, 32, HC>(a, st);
  if (e != hipSuccess) return e;
  return hipGetLastError();
}

hipError_t launch_fused_layer(const FusedLayer& a, hipStream_t st, const FaQ8& q) {
  const uint32_t H = a.hidden;
  if ((H != kFaH && H != 2 * kFaH) || a.n_tokens < 1 || a.n_tokens > kMaxDecodeTokens ||
      (a.trace && a.n_tokens != 1) || (q.gate.q && !q.gate_f32))
    return hipErrorInvalidValue;
  return H == kFaH ? launch_fused_layer_h<1>(a, q, st) : launch_fused_layer_h<2>(a, q, st);
}

}  // namespace smoe
