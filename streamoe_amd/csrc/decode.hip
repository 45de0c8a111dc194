// decode.hip — single-token kernels of the routed-expert path (gfx950).
//
//   k_qmv            dense quantized matvec (LM head), persistent waves,
//                    x held in registers, loads of the next rows issued
//                    before the current ones are reduced.
//   k_router_logits  f32 router GEMV, one block per expert row.
//   k_topk           softmax + running-minimum top-k + renorm, one wave
//                    per token, exact slot order of the reference.
//   k_gateup         fused gate + up + SwiGLU over all routed slots and
//                    the shared expert; one wave reads whole rows with
//                    one 16-byte (4-bit) / 12-byte (3-bit) load per lane.
//   k_down_combine   down projection of every slot for a few output rows
//                    plus the fixed-order weighted combine and residual,
//                    no atomics.
#include "common.h"
#include "kernels.h"
#include "topk.h"

namespace smoe {

static_assert(sizeof(FfnTable) < 4096, "FfnTable must fit a kernel argument");

BlobGeom blob_geom(uint32_t hidden, uint32_t inter, uint32_t group, uint32_t bits) {
  BlobGeom g{};
  g.bits = bits;
  g.hidden = hidden;
  g.inter = inter;
  g.group = group;
  const uint64_t wb = (uint64_t)inter * hidden * bits / 8;
  const uint64_t sb = (uint64_t)inter * (hidden / group) * 2;
  const uint64_t blk = wb + 2 * sb;
  for (int i = 0; i < 3; ++i) {
    g.w[i] = i * blk;
    g.s[i] = i * blk + wb;
    g.b[i] = i * blk + wb + sb;
  }
  return g;
}

// ---------------------------------------------------------------------------
// Dense qmv.  CPR = in_dim / 32 chunks per row; a row is read by
// L = min(CPR, 64) lanes, each owning CPL = CPR / L chunks; a wave covers
// RPP = 64 / L rows per pass and U passes per step.
// ---------------------------------------------------------------------------
// (value, index) merge that keeps the larger value and, on ties, the lower
// index (the sequential scan's first maximum); NaN never wins.
__device__ __forceinline__ void argmax_merge(float& bv, uint32_t& bi, float v, uint32_t i) {
  if (v > bv || (v == bv && i < bi)) {
    bv = v;
    bi = i;
  }
}

// One step of a wave argmax on DPP: merge with the lane CTRL names (lanes
// without a source in range, or outside ROW_MASK, see the identity).
template <int CTRL, int ROW_MASK = 0xF>
__device__ __forceinline__ void argmax_dpp(float& bv, uint32_t& bi) {
  const float v = __int_as_float(
      __builtin_amdgcn_update_dpp(__float_as_int(-INFINITY), __float_as_int(bv), CTRL, ROW_MASK, 0xF, false));
  const uint32_t i = (uint32_t)__builtin_amdgcn_update_dpp(-1, (int)bi, CTRL, ROW_MASK, 0xF, false);
  argmax_merge(bv, bi, v, i);
}

// Wave argmax into lane 63: DPP row shifts, then the row broadcasts.
__device__ __forceinline__ void argmax_wave_last(float& bv, uint32_t& bi) {
  argmax_dpp<0x111>(bv, bi);
  argmax_dpp<0x112>(bv, bi);
  argmax_dpp<0x114>(bv, bi);
  argmax_dpp<0x118>(bv, bi);
  argmax_dpp<0x142, 0xA>(bv, bi);
  argmax_dpp<0x143, 0xC>(bv, bi);
}

// Padded instances (PAD): CPR is a power of two >= the row's cpr chunks (any
// multiple of 32 inputs). A lane's chunk c >= cpr reads the row's last
// chunk instead (in bounds) and multiplies it by a zero input, so it adds
// nothing; an exact instance (cpr == CPR) compiles without the clamps.
__device__ __forceinline__ uint32_t pad_chunk(uint32_t c, uint32_t cpr) { return c < cpr ? c : cpr - 1; }

__device__ __forceinline__ void load_x32_pad(const float* base, uint32_t c, uint32_t cpr, float (&x)[kChunk]) {
  load_x32(base + (size_t)pad_chunk(c, cpr) * kChunk, x);
  if (c >= cpr) {
#pragma unroll
    for (int j = 0; j < kChunk; ++j) x[j] = 0.f;
  }
}

template <int BITS, int CPR, int U, bool PAD = false>
__global__ __launch_bounds__(256) void k_qmv(const uint8_t* __restrict__ codes,
                                             const uint16_t* __restrict__ scales,
                                             const uint16_t* __restrict__ biases,
                                             const float* __restrict__ x, float* __restrict__ y,
                                             uint32_t rows, uint32_t group, uint32_t n_waves,
                                             float* __restrict__ arg_v, uint32_t* __restrict__ arg_i,
                                             uint32_t cpr_rt) {
  constexpr int L = CPR < kWave ? CPR : kWave;
  constexpr int CPL = CPR / L;
  constexpr int RPP = kWave / L;
  constexpr int CB = chunk_bytes<BITS>();
  const uint32_t cpr = PAD ? cpr_rt : (uint32_t)CPR;
  const uint32_t ROW_BYTES = cpr * CB;
  const int lane = threadIdx.x & 63;
  // Wave-uniform (the compiler cannot tell from threadIdx.x): keeps the step
  // loop and the row bases scalar.
  const uint32_t wave = __builtin_amdgcn_readfirstlane(blockIdx.x * (blockDim.x >> 6) + (threadIdx.x >> 6));
  const int lrow = lane / L, lch = lane % L;
  const uint32_t gpr = cpr * kChunk / group;  // groups per row
  const uint32_t cpg_shift = __builtin_ctz(group / kChunk);

  // x in integer-limb form, built once per wave and reused for every row.
  XLimbs xl[CPL];
#pragma unroll
  for (int i = 0; i < CPL; ++i) {
    float xr[kChunk];
    if (PAD)
      load_x32_pad(x, lch + L * i, cpr, xr);
    else
      load_x32(x + (size_t)(lch + L * i) * kChunk, xr);
    make_limbs(xr, xl[i]);
  }

  constexpr uint32_t STEP_ROWS = RPP * U;
  const uint32_t n_steps = (rows + STEP_ROWS - 1) / STEP_ROWS;
  Raw<BITS> cur[U][CPL];
  // bf16 scales and biases stay raw (one per 32-bit register, so the
  // compiler does not pack pairs) until the step is computed: widening them
  // where they are loaded would make the wave wait for the next step's
  // loads before computing the current one.
  uint32_t cs[U][CPL], cb[U][CPL];

  auto issue = [&](uint32_t step, Raw<BITS>(&raw)[U][CPL], uint32_t(&sv)[U][CPL],
                   uint32_t(&bv)[U][CPL]) {
#pragma unroll
    for (int u = 0; u < U; ++u) {
      uint32_t row = step * STEP_ROWS + u * RPP + lrow;
      row = row < rows ? row : rows - 1;
#pragma unroll
      for (int i = 0; i < CPL; ++i) {
        const uint32_t c = PAD ? pad_chunk(lch + L * i, cpr) : lch + L * i;
        // Row bases (scalar for whole-wave rows) plus 32-bit lane offsets.
        raw[u][i] = load_raw<BITS>(codes + (size_t)row * ROW_BYTES + lane_off(c * CB));
        const uint32_t go = lane_off(c >> cpg_shift);
        sv[u][i] = scales[(size_t)row * gpr + go];
        bv[u][i] = biases[(size_t)row * gpr + go];
      }
    }
  };

  float best = -INFINITY;
  uint32_t best_i = 0xFFFFFFFFu;
  auto compute = [&](uint32_t step, const Raw<BITS>(&raw)[U][CPL], const uint32_t(&sv)[U][CPL],
                     const uint32_t(&bv)[U][CPL]) {
    if constexpr (L == kWave && U == 4) {
      // Whole-wave rows: the four rows' lane partials are reduced together
      // (two permlane swaps leave 16-lane rows holding rows 0, 2, 1, 3, then
      // one 16-lane sum), ~10 instructions for the four rows instead of four
      // 6-step butterflies; lane 0 of each 16-lane row stores its row.
      float part[U];
#pragma unroll
      for (int u = 0; u < U; ++u) {
        part[u] = 0.f;
#pragma unroll
        for (int i = 0; i < CPL; ++i)
          part[u] += chunk_dot_i<BITS>(raw[u][i], xl[i], __uint_as_float(sv[u][i] << 16),
                                       __uint_as_float(bv[u][i] << 16));
      }
      const float sum = row_sum16_all(swap16_add(swap32_add(part[0], part[1]), swap32_add(part[2], part[3])));
      const int r16 = lane >> 4;
      const uint32_t row = step * STEP_ROWS + ((r16 >> 1) | ((r16 & 1) << 1));
      if ((lane & 15) == 0 && row < rows) {
        y[row] = sum;
        argmax_merge(best, best_i, sum, row);
      }
    } else {
#pragma unroll
      for (int u = 0; u < U; ++u) {
        float part = 0.f;
#pragma unroll
        for (int i = 0; i < CPL; ++i)
          part += chunk_dot_i<BITS>(raw[u][i], xl[i], __uint_as_float(sv[u][i] << 16),
                                    __uint_as_float(bv[u][i] << 16));
        const float sum = group_sum<L>(part);
        const uint32_t row = step * STEP_ROWS + u * RPP + lrow;
        if (lch == 0 && row < rows) {
          y[row] = sum;
          argmax_merge(best, best_i, sum, row);
        }
      }
    }
  };
  // Fused argmax: the wave's (max, first index) over its rows, written to
  // arg_v / arg_i[wave] when they are given (lanes that store no row keep
  // -inf).
  auto publish = [&]() {
    if (!arg_v) return;
    argmax_wave_last(best, best_i);
    if (lane == 63) {
      arg_v[wave] = best;
      arg_i[wave] = best_i;
    }
  };

  // Ping-pong between two register sets (no copies between them, which
  // would make the compiler wait for the loads at the copy): the loads of
  // step s + n_waves are in flight while step s is computed. The loop runs
  // an even number of steps with every issue unconditional: a step past the
  // end loads the last row again (an L2 hit) and stores nothing, and a
  // branch around the loads would merge the two paths' wait counts into a
  // wait for the new loads before the computation.
  const uint32_t step0 = wave;
  if (step0 >= n_steps) {
    publish();
    return;
  }
  const uint32_t my_steps = (n_steps - step0 + n_waves - 1) / n_waves;
  Raw<BITS> rb[U][CPL];
  uint32_t sb[U][CPL], bb[U][CPL];
  issue(step0, cur, cs, cb);
  for (uint32_t i = 0; i < my_steps; i += 2) {
    const uint32_t s0 = step0 + i * n_waves, s1 = s0 + n_waves, s2 = s1 + n_waves;
    issue(s1, rb, sb, bb);
    compute(s0, cur, cs, cb);
    issue(s2, cur, cs, cb);
    compute(s1, rb, sb, bb);
  }
  publish();
}

__global__ __launch_bounds__(1024) void k_argmax_final(const float* __restrict__ pv,
                                                       const uint32_t* __restrict__ pi, uint32_t n,
                                                       const float* __restrict__ v0, int32_t* __restrict__ out);

template <int BITS, int CPR, bool PAD = false>
static hipError_t qmv_inst(const QView& w, const float* x, float* y, uint32_t rows,
                           hipStream_t st, float* arg_v, uint32_t* arg_i, int32_t* arg_out,
                           uint32_t cpr = CPR) {
  constexpr int L = CPR < kWave ? CPR : kWave;
  constexpr int RPP = kWave / L;
  // Rows per wave and step, and the persistent grid: 4 rows x 3072 waves
  // (12 per CU on 256 CUs, the occupancy this instance's registers allow)
  // measured best on MI355X for the 151,936 x 2048 LM head (45.6 us per
  // token with the argmax and one butterfly per row, against 48-69 us for
  // 8 or 16 rows and 1024-5120 waves; 40.6 us with the four rows reduced
  // together).
  constexpr int U = 4;
  const uint32_t n_steps = (rows + RPP * U - 1) / (RPP * U);
  uint32_t n_waves = n_steps < kQmvMaxWaves ? n_steps : kQmvMaxWaves;
  const uint32_t wpb = 4;
  const uint32_t blocks = (n_waves + wpb - 1) / wpb;
  n_waves = blocks * wpb;
  hipLaunchKernelGGL((k_qmv<BITS, CPR, U, PAD>), dim3(blocks), dim3(wpb * 64), 0, st, w.codes, w.scales,
                     w.biases, x, y, rows, w.group, n_waves, arg_out ? arg_v : nullptr, arg_i, cpr);
  if (arg_out)
    hipLaunchKernelGGL(k_argmax_final, dim3(1), dim3(1024), 0, st, arg_v, arg_i, n_waves, (const float*)y, arg_out);
  return hipGetLastError();
}

template <int BITS>
static hipError_t qmv_bits(const QView& w, const float* x, float* y, uint32_t rows,
                           uint32_t in_dim, hipStream_t st, bool* unsupported, float* av, uint32_t* ai,
                           int32_t* ao) {
  const uint32_t cpr = in_dim / kChunk;
  switch (cpr) {
    case 16: return qmv_inst<BITS, 16>(w, x, y, rows, st, av, ai, ao);
    case 32: return qmv_inst<BITS, 32>(w, x, y, rows, st, av, ai, ao);
    case 64: return qmv_inst<BITS, 64>(w, x, y, rows, st, av, ai, ao);
    case 128: return qmv_inst<BITS, 128>(w, x, y, rows, st, av, ai, ao);
    case 256: return qmv_inst<BITS, 256>(w, x, y, rows, st, av, ai, ao);
    default: break;
  }
  // Other multiples of 32 inputs up to 8192: the padded instances.
  if (cpr == 0) {
    *unsupported = true;
    return hipSuccess;
  }
  if (cpr <= 8) return qmv_inst<BITS, 8, true>(w, x, y, rows, st, av, ai, ao, cpr);
  if (cpr <= 16) return qmv_inst<BITS, 16, true>(w, x, y, rows, st, av, ai, ao, cpr);
  if (cpr <= 32) return qmv_inst<BITS, 32, true>(w, x, y, rows, st, av, ai, ao, cpr);
  if (cpr <= 64) return qmv_inst<BITS, 64, true>(w, x, y, rows, st, av, ai, ao, cpr);
  if (cpr <= 128) return qmv_inst<BITS, 128, true>(w, x, y, rows, st, av, ai, ao, cpr);
  if (cpr <= 256) return qmv_inst<BITS, 256, true>(w, x, y, rows, st, av, ai, ao, cpr);
  *unsupported = true;
  return hipSuccess;
}

// ---------------------------------------------------------------------------
// 8-bit affine matvec (dequant_matvec_8bit_gs_cpu, cpu_matvec.rs:205-283;
// the reference's GPU kernel is dequant_matvec_8bit_v3, shaders.metal:
// 619-677): the small 8-bit projections of the A3B models (router, shared-
// expert gate). Persistent waves, one row at a time; lane l takes the
// 16-input pieces starting at 16 l + 1024 i (all of a row's pieces are
// loaded before the first FMA), forms each weight as fma(q, s, b) and adds
// it into one FMA chain, then the wave sum.
// ---------------------------------------------------------------------------
constexpr int kQ8Pieces = 8;  // 16-input pieces per lane: in_dim <= 8192

__global__ __launch_bounds__(256) void k_qmv8(const uint8_t* __restrict__ codes,
                                              const uint16_t* __restrict__ scales,
                                              const uint16_t* __restrict__ biases,
                                              const float* __restrict__ x, float* __restrict__ y,
                                              uint32_t rows, uint32_t in_dim, uint32_t gsh, uint32_t n_waves) {
  const uint32_t lane = threadIdx.x & 63;
  const uint32_t wave = __builtin_amdgcn_readfirstlane(blockIdx.x * (blockDim.x >> 6) + (threadIdx.x >> 6));
  const uint32_t gpr = in_dim >> gsh;
  for (uint32_t r = wave; r < rows; r += n_waves) {
    u32x4 q[kQ8Pieces];
    uint32_t s[kQ8Pieces], b[kQ8Pieces];
#pragma unroll
    for (int i = 0; i < kQ8Pieces; ++i) {
      const uint32_t c = lane * 16 + 1024u * i;
      if (c < in_dim) {
        q[i] = *reinterpret_cast<const u32x4*>(codes + (size_t)r * in_dim + c);
        const size_t gi = (size_t)r * gpr + (c >> gsh);
        s[i] = scales[gi];
        b[i] = biases[gi];
      }
    }
    float acc = 0.f;
#pragma unroll
    for (int i = 0; i < kQ8Pieces; ++i) {
      const uint32_t c = lane * 16 + 1024u * i;
      if (c < in_dim) {
        const float sf = bf16f((uint16_t)s[i]), bf = bf16f((uint16_t)b[i]);
        const uint32_t wd[4] = {q[i].x, q[i].y, q[i].z, q[i].w};
#pragma unroll
        for (int j = 0; j < 4; ++j) {
          const f32x4 x4 = *reinterpret_cast<const f32x4*>(x + c + 4 * j);
          const float xv[4] = {x4.x, x4.y, x4.z, x4.w};
#pragma unroll
          for (int n = 0; n < 4; ++n)
            acc = __builtin_fmaf(__builtin_fmaf((float)((wd[j] >> (8 * n)) & 0xFFu), sf, bf), xv[n], acc);
        }
      }
    }
    acc = group_sum<64>(acc);
    if (lane == 0) y[r] = acc;
  }
}

static hipError_t qmv8(const QView& w, const float* x, float* y, uint32_t rows, uint32_t in_dim,
                       hipStream_t st, bool* unsupported, float* arg_v, uint32_t* arg_i, int32_t* arg_out) {
  if (in_dim % 16 || in_dim > 1024u * kQ8Pieces || w.group < 16) {
    *unsupported = true;
    return hipSuccess;
  }
  const uint32_t wpb = 4;
  uint32_t n_waves = rows < kQmvMaxWaves ? rows : kQmvMaxWaves;
  const uint32_t blocks = (n_waves + wpb - 1) / wpb;
  n_waves = blocks * wpb;
  hipLaunchKernelGGL(k_qmv8, dim3(blocks), dim3(wpb * 64), 0, st, w.codes, w.scales, w.biases, x, y, rows,
                     in_dim, (uint32_t)__builtin_ctz(w.group), n_waves);
  if (arg_out) return launch_argmax(y, rows, arg_out, arg_v, arg_i, st);
  return hipGetLastError();
}

hipError_t launch_qmv(const QView& w, const float* x, float* y, uint32_t out_dim, uint32_t in_dim,
                      hipStream_t st, bool* unsupported, float* arg_v, uint32_t* arg_i, int32_t* arg_out) {
  *unsupported = false;
  if (w.bits == 8) return qmv8(w, x, y, out_dim, in_dim, st, unsupported, arg_v, arg_i, arg_out);
  if (in_dim % kChunk) {
    *unsupported = true;
    return hipSuccess;
  }
  return w.bits == 4 ? qmv_bits<4>(w, x, y, out_dim, in_dim, st, unsupported, arg_v, arg_i, arg_out)
                     : qmv_bits<3>(w, x, y, out_dim, in_dim, st, unsupported, arg_v, arg_i, arg_out);
}

// ---------------------------------------------------------------------------
// Dequant probe: out[r, c] = fma(q, s, b) for rows [row0, row0 + n_rows).
// ---------------------------------------------------------------------------
template <int BITS>
__global__ __launch_bounds__(256) void k_dequant(const uint8_t* __restrict__ codes,
                                                 const uint16_t* __restrict__ scales,
                                                 const uint16_t* __restrict__ biases,
                                                 uint32_t in_dim, uint32_t group, uint32_t row0,
                                                 uint32_t n_rows, float* __restrict__ out) {
  const uint32_t cpr = in_dim / kChunk;
  const uint64_t t = (uint64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (t >= (uint64_t)n_rows * cpr) return;
  const uint32_t r = row0 + (uint32_t)(t / cpr), c = (uint32_t)(t % cpr);
  const Raw<BITS> raw = load_raw<BITS>(codes + (size_t)r * cpr * chunk_bytes<BITS>() +
                                       (size_t)c * chunk_bytes<BITS>());
  const size_t gi = (size_t)r * (in_dim / group) + (size_t)c * kChunk / group;
  const float s = bf16f(scales[gi]), b = bf16f(biases[gi]);
  float* o = out + (size_t)(r - row0) * in_dim + (size_t)c * kChunk;
#pragma unroll
  for (int j = 0; j < kChunk; ++j) o[j] = __builtin_fmaf((float)code_at(raw, j), s, b);
}

// 8-bit rows: one thread per 16 consecutive inputs (byte n of word i is
// input 4i + n); in_dim is a multiple of the group (>= 32), so a piece never
// straddles a group.
__global__ __launch_bounds__(256) void k_dequant8(const uint8_t* __restrict__ codes,
                                                  const uint16_t* __restrict__ scales,
                                                  const uint16_t* __restrict__ biases,
                                                  uint32_t in_dim, uint32_t group, uint32_t row0,
                                                  uint32_t n_rows, float* __restrict__ out) {
  const uint32_t ppr = in_dim / 16;
  const uint64_t t = (uint64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (t >= (uint64_t)n_rows * ppr) return;
  const uint32_t r = row0 + (uint32_t)(t / ppr), c = (uint32_t)(t % ppr) * 16;
  const u32x4 q = *reinterpret_cast<const u32x4*>(codes + (size_t)r * in_dim + c);
  const size_t gi = (size_t)r * (in_dim / group) + c / group;
  const float s = bf16f(scales[gi]), b = bf16f(biases[gi]);
  const uint32_t wd[4] = {q.x, q.y, q.z, q.w};
  float* o = out + (size_t)(r - row0) * in_dim + c;
#pragma unroll
  for (int j = 0; j < 16; ++j) o[j] = __builtin_fmaf((float)((wd[j >> 2] >> (8 * (j & 3))) & 0xFFu), s, b);
}

hipError_t launch_dequant(const QView& w, uint32_t in_dim, uint32_t row0, uint32_t n_rows,
                          float* out, hipStream_t st) {
  if (w.bits == 8) {
    const uint64_t n = (uint64_t)n_rows * (in_dim / 16);
    hipLaunchKernelGGL(k_dequant8, dim3((uint32_t)((n + 255) / 256)), dim3(256), 0, st, w.codes,
                       w.scales, w.biases, in_dim, w.group, row0, n_rows, out);
    return hipGetLastError();
  }
  const uint64_t n = (uint64_t)n_rows * (in_dim / kChunk);
  const uint32_t blocks = (uint32_t)((n + 255) / 256);
  if (w.bits == 4)
    hipLaunchKernelGGL(k_dequant<4>, dim3(blocks), dim3(256), 0, st, w.codes, w.scales, w.biases,
                       in_dim, w.group, row0, n_rows, out);
  else
    hipLaunchKernelGGL(k_dequant<3>, dim3(blocks), dim3(256), 0, st, w.codes, w.scales, w.biases,
                       in_dim, w.group, row0, n_rows, out);
  return hipGetLastError();
}

// ---------------------------------------------------------------------------
// Argmax (first index on ties) in two stages: kArgBlocks blocks each reduce
// a contiguous slice with 128-bit loads to (value, index), then one block
// reduces the partials. (value, index) pairs order by value, then by lower
// index, so the result is the first maximal index, as a sequential scan.
// ---------------------------------------------------------------------------
constexpr uint32_t kArgBlocks = 256;

// Block-wide (value, index) reduction; result valid in thread 0.
// Block argmax, valid in every lane of wave 0 (threads 0..63): each wave
// reduces on DPP row shifts and row broadcasts into its last lane (no LDS
// permutes), then wave 0 merges the waves' results the same way.
__device__ __forceinline__ void argmax_block(float& best, uint32_t& bi) {
  __shared__ float sv[16];
  __shared__ uint32_t si[16];
  argmax_wave_last(best, bi);
  const uint32_t w = threadIdx.x >> 6, nw = blockDim.x >> 6;
  if ((threadIdx.x & 63) == 63) {
    sv[w] = best;
    si[w] = bi;
  }
  __syncthreads();
  if (threadIdx.x < 64) {
    const bool live = threadIdx.x < nw;
    best = live ? sv[threadIdx.x] : -INFINITY;
    bi = live ? si[threadIdx.x] : 0xFFFFFFFFu;
    argmax_dpp<0x111>(best, bi);
    argmax_dpp<0x112>(best, bi);
    argmax_dpp<0x114>(best, bi);
    argmax_dpp<0x118>(best, bi);
    best = readlane_f(best, 15);
    bi = (uint32_t)__builtin_amdgcn_readlane((int)bi, 15);
  }
}

__global__ __launch_bounds__(256) void k_argmax_part(const float* __restrict__ v, uint32_t n,
                                                     float* __restrict__ pv, uint32_t* __restrict__ pi) {
  const uint32_t per = ((n + kArgBlocks - 1) / kArgBlocks + 3) & ~3u;  // multiple of 4
  const uint32_t lo = blockIdx.x * per, hi = min(n, lo + per);
  float best = -INFINITY;
  uint32_t bi = 0xFFFFFFFFu;
  for (uint32_t i = lo + threadIdx.x * 4; i < hi; i += blockDim.x * 4) {
    if (i + 3 < hi) {
      const float4 q = *reinterpret_cast<const float4*>(v + i);
      argmax_merge(best, bi, q.x, i);
      argmax_merge(best, bi, q.y, i + 1);
      argmax_merge(best, bi, q.z, i + 2);
      argmax_merge(best, bi, q.w, i + 3);
    } else {
      for (uint32_t j = i; j < hi; ++j) argmax_merge(best, bi, v[j], j);
    }
  }
  argmax_block(best, bi);
  if (threadIdx.x == 0) {
    pv[blockIdx.x] = best;
    pi[blockIdx.x] = bi;
  }
}

// The merge of the partials. The reference's greedy pick is the scan
// `best = 0; if v[i] > v[best] then best = i` (engine_tests.rs:105-107,
// orc_argmax): NaN never replaces the best, and a NaN at index 0 is never
// replaced, so the pick is 0 then; v0 = the vector's first element.
__global__ __launch_bounds__(1024) void k_argmax_final(const float* __restrict__ pv,
                                                       const uint32_t* __restrict__ pi, uint32_t n,
                                                       const float* __restrict__ v0, int32_t* __restrict__ out) {
  float best = -INFINITY;
  uint32_t bi = 0xFFFFFFFFu;
  // v[0] is read with the partials, not after the block reduction: loads
  // cannot move across its barriers, so a late read is one more memory
  // round trip at the end of the launch.
  const float first = *v0;
  // Four partials per thread per round, loaded before they are merged (the
  // merges form a dependency chain; the loads must not).
  for (uint32_t i0 = threadIdx.x; i0 < n; i0 += 4 * blockDim.x) {
    float v[4];
    uint32_t ix[4];
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const uint32_t i = min(i0 + j * blockDim.x, n - 1);
      v[j] = pv[i];
      ix[j] = pi[i];
    }
#pragma unroll
    for (int j = 0; j < 4; ++j) argmax_merge(best, bi, v[j], ix[j]);
  }
  argmax_block(best, bi);
  if (threadIdx.x == 0) *out = first != first ? 0 : (int32_t)bi;
}

hipError_t launch_argmax(const float* v, uint32_t n, int32_t* out, float* part_v, uint32_t* part_i,
                         hipStream_t st) {
  hipLaunchKernelGGL(k_argmax_part, dim3(kArgBlocks), dim3(256), 0, st, v, n, part_v, part_i);
  hipLaunchKernelGGL(k_argmax_final, dim3(1), dim3(256), 0, st, part_v, part_i, kArgBlocks, v, out);
  return hipGetLastError();
}

// ---------------------------------------------------------------------------
// Router logits: one 256-thread block per (expert row, token); row
// n_experts is the shared-expert gate when gate_w is not null.
// ---------------------------------------------------------------------------
// With norm_w, x is the residual and every block applies the next layer's
// RMSNorm itself (rms_norm_bf16_n_tokens_cpu, backend/cpu/mod.rs:406-430:
// inv = 1 / sqrt(sum_sq / dim + eps), x = r * inv * w; each block forms the
// same sum in the same order), and block (0, t) stores the normalised row
// in x_out for the expert kernels: one launch instead of a norm kernel
// before the router.
// An 8-bit router or gate (Wq / gq) has the same loop over 4-input pieces:
// each weight is dequantized as fma(q, s, b) (dequant_matvec_8bit_gs_cpu,
// cpu_matvec.rs:205-283) and then enters the same FMA chain.
__global__ __launch_bounds__(256) void k_router_logits(const float* __restrict__ W,
                                                       const float* __restrict__ gate_w,
                                                       const float* __restrict__ x,
                                                       uint32_t n_experts, uint32_t hidden,
                                                       float* __restrict__ logits,
                                                       float* __restrict__ gate_scores,
                                                       const uint16_t* __restrict__ norm_w, float eps,
                                                       float* __restrict__ x_out, Q8Rows Wq, Q8Rows gq) {
  __shared__ float red[4];
  __shared__ float inv_sh;
  const uint32_t e = blockIdx.x, t = blockIdx.y;
  const float* row = e < n_experts ? W + (size_t)e * hidden : gate_w;
  const Q8Rows rq = e < n_experts ? Wq : gq;
  const uint32_t qrow = e < n_experts ? e : 0u;
  const uint32_t gsh = rq.q ? __builtin_ctz(rq.group) : 0u;
  const float* xt = x + (size_t)t * hidden;
  float inv = 1.f;
  if (norm_w) {
    float ss = 0.f;
    for (uint32_t c = threadIdx.x * 4; c < hidden; c += 1024) {
      const float4 r4 = *reinterpret_cast<const float4*>(xt + c);
      ss = __builtin_fmaf(r4.x, r4.x, ss);
      ss = __builtin_fmaf(r4.y, r4.y, ss);
      ss = __builtin_fmaf(r4.z, r4.z, ss);
      ss = __builtin_fmaf(r4.w, r4.w, ss);
    }
    ss = group_sum<64>(ss);
    if ((threadIdx.x & 63) == 0) red[threadIdx.x >> 6] = ss;
    __syncthreads();
    if (threadIdx.x == 0) inv_sh = 1.0f / sqrtf(((red[0] + red[1]) + (red[2] + red[3])) / (float)hidden + eps);
    __syncthreads();
    inv = inv_sh;
  }
  float acc = 0.f;
  for (uint32_t c = threadIdx.x * 4; c < hidden; c += 1024) {
    f32x4 w4;
    if (rq.q) {
      const uint32_t q4 = *reinterpret_cast<const uint32_t*>(rq.q + (size_t)qrow * hidden + c);
      const size_t gi = (size_t)qrow * (hidden >> gsh) + (c >> gsh);
      const float s = bf16f(rq.s[gi]), b = bf16f(rq.b[gi]);
      w4 = f32x4{__builtin_fmaf((float)(q4 & 0xFFu), s, b), __builtin_fmaf((float)((q4 >> 8) & 0xFFu), s, b),
                 __builtin_fmaf((float)((q4 >> 16) & 0xFFu), s, b), __builtin_fmaf((float)(q4 >> 24), s, b)};
    } else {
      w4 = __builtin_nontemporal_load(reinterpret_cast<const f32x4*>(row + c));
    }
    float4 x4 = *reinterpret_cast<const float4*>(xt + c);
    if (norm_w) {
      x4.x = x4.x * inv * bf16f(norm_w[c]);
      x4.y = x4.y * inv * bf16f(norm_w[c + 1]);
      x4.z = x4.z * inv * bf16f(norm_w[c + 2]);
      x4.w = x4.w * inv * bf16f(norm_w[c + 3]);
      if (e == 0) *reinterpret_cast<float4*>(x_out + (size_t)t * hidden + c) = x4;
    }
    acc = __builtin_fmaf(w4.x, x4.x, acc);
    acc = __builtin_fmaf(w4.y, x4.y, acc);
    acc = __builtin_fmaf(w4.z, x4.z, acc);
    acc = __builtin_fmaf(w4.w, x4.w, acc);
  }
  acc = group_sum<64>(acc);
  if ((threadIdx.x & 63) == 0) red[threadIdx.x >> 6] = acc;
  __syncthreads();
  if (threadIdx.x == 0) {
    const float s = (red[0] + red[1]) + (red[2] + red[3]);
    if (e < n_experts)
      logits[(size_t)t * n_experts + e] = s;
    else
      gate_scores[t] = s;
  }
}

hipError_t launch_router_logits(const float* W, const float* gate_w, const float* x,
                                uint32_t n_tokens, uint32_t n_experts, uint32_t hidden,
                                float* logits, float* gate_scores, hipStream_t st,
                                const uint16_t* norm_w, float eps, float* x_out, const Q8Rows& Wq,
                                const Q8Rows& gq) {
  const uint32_t rows = n_experts + (gate_w || gq.q ? 1 : 0);
  hipLaunchKernelGGL(k_router_logits, dim3(rows, n_tokens), dim3(256), 0, st, W, gate_w, x,
                     n_experts, hidden, logits, gate_scores, norm_w, eps, x_out, Wq, gq);
  return hipGetLastError();
}

// ---------------------------------------------------------------------------
// Top-k: one wave per token, lane l holding elements l, l + 64, ... The
// reference scans the scores in index order and replaces the running-
// minimum slot (lowest slot on ties) with every score strictly greater
// than it (moe_router.rs:83-124); exact_topk_t does the same scan, one
// ballot per replacement.
// ---------------------------------------------------------------------------

template <int P>
__global__ __launch_bounds__(64) void k_topk(const float* __restrict__ scores, uint32_t n,
                                             uint32_t k, int softmax, int normalize,
                                             RouteOut out) {
  const uint32_t t = blockIdx.x;
  const int lane = threadIdx.x;
  const float* s = scores + (size_t)t * n;
  // Lane l holds elements l, l + 64, ... (coalesced loads; the layout
  // exact_topk_t scans).
  float v[P];
#pragma unroll
  for (int e = 0; e < P; ++e) {
    const uint32_t j = e * 64 + lane;
    v[e] = j < n ? s[j] : -INFINITY;
  }
  if (softmax) {
    // moe_router.rs:52-72, the reference's probabilities bit for bit.
    __shared__ float sprob[64 * P];
    softmax_ref<P, true>(v, n, lane, sprob, load_exp_tab(lane));
    if (out.probs) {
#pragma unroll
      for (int e = 0; e < P; ++e) {
        const uint32_t j = e * 64 + lane;
        if (j < n) out.probs[(size_t)t * n + j] = v[e];
      }
    }
  }
  // The reference's running-minimum top-k (moe_router.rs:83-124); lane s < k
  // then holds slot s.
  __shared__ int32_t sid[kMaxK];
  __shared__ float sval[kMaxK];
  exact_topk_t<P>(v, k, lane, sid, sval);
  __syncthreads();
  const int32_t sidx = lane < (int)k ? sid[lane] : 0;
  const float sv = lane < (int)k ? sval[lane] : 0.f;
  // normalize_weights, moe_router.rs:130-141: sequential sum in slot order.
  float w = sv;
  if (normalize) {
    float sum = 0.f;
    for (uint32_t i = 0; i < k; ++i) sum += readlane_f(sv, (int)i);
    if (sum > 0.f) {
      const float inv = 1.0f / sum;
      w = sv * inv;
    }
  }
  if (lane < (int)k) {
    if (out.idx) out.idx[(size_t)t * k + lane] = sidx;
    if (out.weight) out.weight[(size_t)t * k + lane] = w;
    if (out.table && t == 0) {
      out.table->blob[lane] = out.experts + (uint64_t)sidx * out.stride;
      out.table->weight[lane] = w;
    }
  }
  if (out.table && t == 0 && lane == 0) {
    out.table->k = k;
    out.table->has_shared = out.shared_blob != nullptr;
    if (out.shared_blob) {
      out.table->blob[k] = out.shared_blob;
      out.table->weight[k] = 1.0f;
      out.table->shared_gate = out.gate_scores ? out.gate_scores[0] : __builtin_nanf("");
    }
  }
}

// glibc's expf over a buffer: one element per lane, whole waves (the table
// lookup is a lane permute), grid-stride.
__global__ __launch_bounds__(256) void k_expf(const float* __restrict__ x, float* __restrict__ y, uint64_t n) {
  const ExpTabReg tab = load_exp_tab((int)(threadIdx.x & 63));
  const uint64_t stride = (uint64_t)gridDim.x * blockDim.x;
  // Every wave runs the same number of iterations (n rounded up to whole
  // grid strides), so the permute always sees all 64 lanes active.
  const uint64_t iters = (n + stride - 1) / stride;
  for (uint64_t it = 0; it < iters; ++it) {
    const uint64_t i = it * stride + (uint64_t)blockIdx.x * blockDim.x + threadIdx.x;
    const float v = x[i < n ? i : n - 1];
    const float r = wave_expf_ref(v, tab);
    if (i < n) y[i] = r;
  }
}

hipError_t launch_expf(const float* x, float* y, uint64_t n, hipStream_t st) {
  if (n == 0) return hipSuccess;
  const uint64_t blocks = (n + 255) / 256;
  hipLaunchKernelGGL(k_expf, dim3((unsigned)(blocks < 4096 ? blocks : 4096)), dim3(256), 0, st, x, y, n);
  return hipGetLastError();
}

hipError_t launch_topk(const float* scores, uint32_t n_tokens, uint32_t n, uint32_t k,
                       bool softmax, bool normalize, const RouteOut& out, hipStream_t st) {
  const uint32_t p = (n + 63) / 64;
  const int sm = softmax, nm = normalize;
  if (p <= 1)
    hipLaunchKernelGGL(k_topk<1>, dim3(n_tokens), dim3(64), 0, st, scores, n, k, sm, nm, out);
  else if (p <= 2)
    hipLaunchKernelGGL(k_topk<2>, dim3(n_tokens), dim3(64), 0, st, scores, n, k, sm, nm, out);
  else if (p <= 4)
    hipLaunchKernelGGL(k_topk<4>, dim3(n_tokens), dim3(64), 0, st, scores, n, k, sm, nm, out);
  else if (p <= 8)
    hipLaunchKernelGGL(k_topk<8>, dim3(n_tokens), dim3(64), 0, st, scores, n, k, sm, nm, out);
  else
    hipLaunchKernelGGL(k_topk<16>, dim3(n_tokens), dim3(64), 0, st, scores, n, k, sm, nm, out);
  return hipGetLastError();
}

// ---------------------------------------------------------------------------
// Fused gate/up + SwiGLU.  CPR = hidden / 32. One block = one wave handling
// RW rows (gate and up) of one slot; the block index enumerates
// (slot, row tile), slots 0..k-1 routed, slot k the shared expert.
// ---------------------------------------------------------------------------
template <int BITS, int CPR, int P, bool PAD>
__device__ __forceinline__ void gateup_body(const uint8_t* __restrict__ blob, const BlobGeom& g,
                                            uint32_t row0, const float (&xr)[CPR < 64 ? 1 : CPR / 64][kChunk],
                                            const float (&xs)[CPR < 64 ? 1 : CPR / 64],
                                            float* __restrict__ act_slot) {
  constexpr int L = CPR < kWave ? CPR : kWave;
  constexpr int CPL = CPR / L;
  constexpr int RPP = kWave / L;
  constexpr int CB = chunk_bytes<BITS>();
  const uint32_t cpr = PAD ? g.hidden / kChunk : (uint32_t)CPR;
  const uint32_t ROW_BYTES = cpr * CB;
  const int lane = threadIdx.x & 63;
  const int lrow = lane / L, lch = lane % L;
  const uint32_t gpr = g.hidden / g.group;
  const uint32_t cpg_shift = __builtin_ctz(g.group / kChunk);
  const uint32_t inter = g.inter;

  Raw<BITS> rg[P][CPL], ru[P][CPL];
  float sg[P][CPL], bg[P][CPL], su[P][CPL], bu[P][CPL];
#pragma unroll
  for (int p = 0; p < P; ++p) {
    uint32_t row = row0 + p * RPP + lrow;
    row = row < inter ? row : inter - 1;
#pragma unroll
    for (int i = 0; i < CPL; ++i) {
      const uint32_t c = PAD ? pad_chunk(lch + L * i, cpr) : lch + L * i;
      const size_t off = (size_t)row * ROW_BYTES + c * CB;
      rg[p][i] = load_raw<BITS>(blob + g.w[0] + off);
      ru[p][i] = load_raw<BITS>(blob + g.w[1] + off);
      const size_t gi = ((size_t)row * gpr + (c >> cpg_shift)) * 2;
      sg[p][i] = bf16f(*reinterpret_cast<const uint16_t*>(blob + g.s[0] + gi));
      bg[p][i] = bf16f(*reinterpret_cast<const uint16_t*>(blob + g.b[0] + gi));
      su[p][i] = bf16f(*reinterpret_cast<const uint16_t*>(blob + g.s[1] + gi));
      bu[p][i] = bf16f(*reinterpret_cast<const uint16_t*>(blob + g.b[1] + gi));
    }
  }
  if constexpr (L == kWave && P == 4) {
    // Whole-wave rows: the four gate and four up rows are reduced together
    // (after the permlane swaps the 16-lane rows hold rows 0, 2, 1, 3), and
    // one SwiGLU per lane serves the four outputs.
    float pg[P], pu[P];
#pragma unroll
    for (int p = 0; p < P; ++p) {
      pg[p] = 0.f;
      pu[p] = 0.f;
#pragma unroll
      for (int i = 0; i < CPL; ++i) {
        pg[p] += chunk_dot<BITS>(rg[p][i], xr[i], xs[i], sg[p][i], bg[p][i]);
        pu[p] += chunk_dot<BITS>(ru[p][i], xr[i], xs[i], su[p][i], bu[p][i]);
      }
    }
    const float gsum = row_sum16_all(swap16_add(swap32_add(pg[0], pg[1]), swap32_add(pg[2], pg[3])));
    const float usum = row_sum16_all(swap16_add(swap32_add(pu[0], pu[1]), swap32_add(pu[2], pu[3])));
    const int r16 = lane >> 4;
    const uint32_t row = row0 + ((r16 >> 1) | ((r16 & 1) << 1));
    if ((lane & 15) == 0 && row < inter) act_slot[row] = silu_mul(gsum, usum);
  } else {
#pragma unroll
    for (int p = 0; p < P; ++p) {
      float pg = 0.f, pu = 0.f;
#pragma unroll
      for (int i = 0; i < CPL; ++i) {
        pg += chunk_dot<BITS>(rg[p][i], xr[i], xs[i], sg[p][i], bg[p][i]);
        pu += chunk_dot<BITS>(ru[p][i], xr[i], xs[i], su[p][i], bu[p][i]);
      }
      const float gsum = group_sum<L>(pg);
      const float usum = group_sum<L>(pu);
      const uint32_t row = row0 + p * RPP + lrow;
      if (lch == 0 && row < inter) act_slot[row] = silu_mul(gsum, usum);
    }
  }
}

template <int BITS, int CPR, int P, bool PAD>
__global__ __launch_bounds__(64) void k_gateup(BlobGeom routed, BlobGeom shared,
                                               const FfnTable* __restrict__ tab_dev,
                                               FfnTable tab_val, uint32_t tiles_per_slot,
                                               const float* __restrict__ x,
                                               float* __restrict__ act) {
  constexpr int L = CPR < kWave ? CPR : kWave;
  constexpr int CPL = CPR / L;
  constexpr int RPP = kWave / L;
  constexpr uint32_t RW = RPP * P;  // rows per wave
  const int lane = threadIdx.x & 63;
  const int lch = lane % L;
  const uint32_t slot = blockIdx.x / tiles_per_slot;
  const uint32_t tile = blockIdx.x % tiles_per_slot;
  const uint32_t k = tab_dev ? tab_dev->k : tab_val.k;
  const uint8_t* blob = tab_dev ? tab_dev->blob[slot] : tab_val.blob[slot];

  float xr[CPL][kChunk];
  float xs[CPL];
#pragma unroll
  for (int i = 0; i < CPL; ++i) {
    if (PAD)
      load_x32_pad(x, lch + L * i, routed.hidden / kChunk, xr[i]);
    else
      load_x32(x + (size_t)(lch + L * i) * kChunk, xr[i]);
    xs[i] = xsum(xr[i]);
  }
  const uint32_t row0 = tile * RW;
  if (slot < k) {
    if (row0 >= routed.inter) return;
    gateup_body<BITS, CPR, P, PAD>(blob, routed, row0, xr, xs, act + (size_t)slot * routed.inter);
  } else {
    if (row0 >= shared.inter) return;
    gateup_body<4, CPR, P, PAD>(blob, shared, row0, xr, xs, act + (size_t)slot * routed.inter);
  }
}

template <int BITS, int CPR, bool PAD = false>
static hipError_t gateup_inst(const BlobGeom& routed, const BlobGeom& shared,
                              const FfnTable* tab_dev, const FfnTable& tab_val, uint32_t n_slots,
                              const float* x, float* act, hipStream_t st) {
  constexpr int L = CPR < kWave ? CPR : kWave;
  constexpr int RPP = kWave / L;
  constexpr int P = CPR / L >= 4 ? 2 : 4;  // rows per lane group: 4, or 2 with 4 chunks per lane
  const uint32_t rw = RPP * P;
  const uint32_t tiles = (routed.inter + rw - 1) / rw;
  hipLaunchKernelGGL((k_gateup<BITS, CPR, P, PAD>), dim3(tiles * n_slots), dim3(64), 0, st, routed,
                     shared, tab_dev, tab_val, tiles, x, act);
  return hipGetLastError();
}

template <int BITS>
static hipError_t gateup_bits(const BlobGeom& routed, const BlobGeom& shared,
                              const FfnTable* tab_dev, const FfnTable& tab_val, uint32_t n_slots,
                              const float* x, float* act, hipStream_t st, bool* unsupported) {
  const uint32_t cpr = routed.hidden / kChunk;
  switch (cpr) {
    case 32: return gateup_inst<BITS, 32>(routed, shared, tab_dev, tab_val, n_slots, x, act, st);
    case 64: return gateup_inst<BITS, 64>(routed, shared, tab_dev, tab_val, n_slots, x, act, st);
    case 128: return gateup_inst<BITS, 128>(routed, shared, tab_dev, tab_val, n_slots, x, act, st);
    default: break;
  }
  // Other hidden sizes (multiples of 32 up to 8192): the padded instances.
  if (cpr == 0) {
    *unsupported = true;
    return hipSuccess;
  }
  if (cpr <= 8) return gateup_inst<BITS, 8, true>(routed, shared, tab_dev, tab_val, n_slots, x, act, st);
  if (cpr <= 16) return gateup_inst<BITS, 16, true>(routed, shared, tab_dev, tab_val, n_slots, x, act, st);
  if (cpr <= 32) return gateup_inst<BITS, 32, true>(routed, shared, tab_dev, tab_val, n_slots, x, act, st);
  if (cpr <= 64) return gateup_inst<BITS, 64, true>(routed, shared, tab_dev, tab_val, n_slots, x, act, st);
  if (cpr <= 128) return gateup_inst<BITS, 128, true>(routed, shared, tab_dev, tab_val, n_slots, x, act, st);
  if (cpr <= 256) return gateup_inst<BITS, 256, true>(routed, shared, tab_dev, tab_val, n_slots, x, act, st);
  *unsupported = true;
  return hipSuccess;
}

hipError_t launch_gateup(const BlobGeom& routed, const BlobGeom& shared, const FfnTable* tab_dev,
                         const FfnTable& tab_val, uint32_t n_slots, const float* x, float* act,
                         hipStream_t st, bool* unsupported) {
  *unsupported = false;
  return routed.bits == 4
             ? gateup_bits<4>(routed, shared, tab_dev, tab_val, n_slots, x, act, st, unsupported)
             : gateup_bits<3>(routed, shared, tab_dev, tab_val, n_slots, x, act, st, unsupported);
}

// ---------------------------------------------------------------------------
// Down + combine.  CPR = inter / 32. One wave = RPP output rows; it loads
// every slot's chunk of those rows up front, then reduces slot by slot in
// the reference's order: moe = fma(out_k, w_k, moe) (deferred.rs:458-466),
// then the shared term and the residual.
// ---------------------------------------------------------------------------
template <int BITS, int CPR, int MAXS, bool PAD>
__global__ __launch_bounds__(64) void k_down_combine(BlobGeom routed, BlobGeom shared,
                                                     const FfnTable* __restrict__ tab_dev,
                                                     FfnTable tab_val,
                                                     const float* __restrict__ act,
                                                     const float* __restrict__ h_mid,
                                                     const float* __restrict__ shared_out,
                                                     float* __restrict__ hidden_out) {
  constexpr int L = CPR < kWave ? CPR : kWave;
  constexpr int CPL = CPR / L;
  constexpr int RPP = kWave / L;
  constexpr int CB = chunk_bytes<BITS>();
  constexpr int CB4 = chunk_bytes<4>();
  const uint32_t cpr = PAD ? routed.inter / kChunk : (uint32_t)CPR;
  const uint32_t ROW_BYTES = cpr * CB;
  const uint32_t ROW_BYTES4 = cpr * CB4;
  const int lane = threadIdx.x & 63;
  const int lrow = lane / L, lch = lane % L;
  const uint32_t H = routed.hidden, I = routed.inter;
  const uint32_t gpr = I / routed.group;
  const uint32_t cpg_shift = __builtin_ctz(routed.group / kChunk);
  uint32_t row = blockIdx.x * RPP + lrow;
  const bool valid = row < H;
  row = valid ? row : H - 1;

  const uint32_t k = tab_dev ? tab_dev->k : tab_val.k;
  const uint32_t has_shared = tab_dev ? tab_dev->has_shared : tab_val.has_shared;

  // Every slot up to MAXS is loaded and computed without a branch (slots
  // past k re-read slot k - 1 and are not added), so the loads and lane
  // reductions of different slots overlap instead of running one by one.
  Raw<BITS> raw[MAXS][CPL];
  Raw<4> rsh[CPL];
  float sv[MAXS][CPL], bv[MAXS][CPL], ssh[CPL], bsh[CPL];
#pragma unroll
  for (int s = 0; s < MAXS; ++s) {
    const uint32_t sl = (uint32_t)s < k ? (uint32_t)s : k - 1;
    const uint8_t* blob = tab_dev ? tab_dev->blob[sl] : tab_val.blob[sl];
#pragma unroll
    for (int i = 0; i < CPL; ++i) {
      const uint32_t c = PAD ? pad_chunk(lch + L * i, cpr) : lch + L * i;
      raw[s][i] = load_raw<BITS>(blob + routed.w[2] + (size_t)row * ROW_BYTES + c * CB);
      const size_t gi = ((size_t)row * gpr + (c >> cpg_shift)) * 2;
      sv[s][i] = bf16f(*reinterpret_cast<const uint16_t*>(blob + routed.s[2] + gi));
      bv[s][i] = bf16f(*reinterpret_cast<const uint16_t*>(blob + routed.b[2] + gi));
    }
  }
  if (has_shared) {
    const uint8_t* blob = tab_dev ? tab_dev->blob[k] : tab_val.blob[k];
#pragma unroll
    for (int i = 0; i < CPL; ++i) {
      const uint32_t c = PAD ? pad_chunk(lch + L * i, cpr) : lch + L * i;
      rsh[i] = load_raw<4>(blob + shared.w[2] + (size_t)row * ROW_BYTES4 + c * CB4);
      const size_t gi = ((size_t)row * gpr + (c >> cpg_shift)) * 2;
      ssh[i] = bf16f(*reinterpret_cast<const uint16_t*>(blob + shared.s[2] + gi));
      bsh[i] = bf16f(*reinterpret_cast<const uint16_t*>(blob + shared.b[2] + gi));
    }
  }

  float o[MAXS];
#pragma unroll
  for (int s = 0; s < MAXS; ++s) {
    const uint32_t sl = (uint32_t)s < k ? (uint32_t)s : k - 1;
    float part = 0.f;
#pragma unroll
    for (int i = 0; i < CPL; ++i) {
      float a[kChunk];
      if (PAD)
        load_x32_pad(act + (size_t)sl * I, lch + L * i, cpr, a);
      else
        load_x32(act + (size_t)sl * I + (size_t)(lch + L * i) * kChunk, a);
      part += chunk_dot<BITS>(raw[s][i], a, xsum(a), sv[s][i], bv[s][i]);
    }
    o[s] = part;
  }
#pragma unroll
  for (int s = 0; s < MAXS; ++s) o[s] = group_sum<L>(o[s]);
  // moe = fma(out_k, w_k, moe) in slot order (deferred.rs:458-466).
  float moe = 0.f;
#pragma unroll
  for (int s = 0; s < MAXS; ++s) {
    const float w = tab_dev ? tab_dev->weight[s < (int)k ? s : 0] : tab_val.weight[s < (int)k ? s : 0];
    moe = s < (int)k ? __builtin_fmaf(o[s], w, moe) : moe;
  }
  float res;
  if (has_shared) {
    float part = 0.f;
#pragma unroll
    for (int i = 0; i < CPL; ++i) {
      float a[kChunk];
      if (PAD)
        load_x32_pad(act + (size_t)k * I, lch + L * i, cpr, a);
      else
        load_x32(act + (size_t)k * I + (size_t)(lch + L * i) * kChunk, a);
      part += chunk_dot<4>(rsh[i], a, xsum(a), ssh[i], bsh[i]);
    }
    const float sh = group_sum<L>(part);
    const float gate = tab_dev ? tab_dev->shared_gate : tab_val.shared_gate;
    const float sum = __builtin_isnan(gate) ? moe + sh : __builtin_fmaf(sh, sigmoidf_ref(gate), moe);
    res = h_mid[row] + sum;
  } else if (shared_out) {
    const float gate = tab_dev ? tab_dev->shared_gate : tab_val.shared_gate;
    const float sh = shared_out[row];
    const float sum = __builtin_isnan(gate) ? moe + sh : __builtin_fmaf(sh, sigmoidf_ref(gate), moe);
    res = h_mid[row] + sum;
  } else {
    res = h_mid[row] + moe;
  }
  if (lch == 0 && valid) hidden_out[row] = res;
}

template <int BITS, int CPR, bool PAD = false>
static hipError_t down_inst(const BlobGeom& routed, const BlobGeom& shared,
                            const FfnTable* tab_dev, const FfnTable& tab_val, uint32_t k,
                            const float* act, const float* h_mid, const float* shared_out,
                            float* hidden_out, hipStream_t st) {
  constexpr int L = CPR < kWave ? CPR : kWave;
  constexpr int RPP = kWave / L;
  const uint32_t blocks = (routed.hidden + RPP - 1) / RPP;
  if (k <= 8)
    hipLaunchKernelGGL((k_down_combine<BITS, CPR, 8, PAD>), dim3(blocks), dim3(64), 0, st, routed,
                       shared, tab_dev, tab_val, act, h_mid, shared_out, hidden_out);
  else
    hipLaunchKernelGGL((k_down_combine<BITS, CPR, 16, PAD>), dim3(blocks), dim3(64), 0, st, routed,
                       shared, tab_dev, tab_val, act, h_mid, shared_out, hidden_out);
  return hipGetLastError();
}

template <int BITS>
static hipError_t down_bits(const BlobGeom& routed, const BlobGeom& shared,
                            const FfnTable* tab_dev, const FfnTable& tab_val, uint32_t k,
                            const float* act, const float* h_mid, const float* shared_out,
                            float* hidden_out, hipStream_t st, bool* unsupported) {
  const uint32_t cpr = routed.inter / kChunk;
  switch (cpr) {
    case 8: return down_inst<BITS, 8>(routed, shared, tab_dev, tab_val, k, act, h_mid, shared_out, hidden_out, st);
    case 16: return down_inst<BITS, 16>(routed, shared, tab_dev, tab_val, k, act, h_mid, shared_out, hidden_out, st);
    case 32: return down_inst<BITS, 32>(routed, shared, tab_dev, tab_val, k, act, h_mid, shared_out, hidden_out, st);
    case 64: return down_inst<BITS, 64>(routed, shared, tab_dev, tab_val, k, act, h_mid, shared_out, hidden_out, st);
    default: break;
  }
  // Other intermediate sizes (multiples of 32 up to 2048): the padded instances.
  if (cpr == 0) {
    *unsupported = true;
    return hipSuccess;
  }
  if (cpr <= 2) return down_inst<BITS, 2, true>(routed, shared, tab_dev, tab_val, k, act, h_mid, shared_out, hidden_out, st);
  if (cpr <= 4) return down_inst<BITS, 4, true>(routed, shared, tab_dev, tab_val, k, act, h_mid, shared_out, hidden_out, st);
  if (cpr <= 8) return down_inst<BITS, 8, true>(routed, shared, tab_dev, tab_val, k, act, h_mid, shared_out, hidden_out, st);
  if (cpr <= 16) return down_inst<BITS, 16, true>(routed, shared, tab_dev, tab_val, k, act, h_mid, shared_out, hidden_out, st);
  if (cpr <= 32) return down_inst<BITS, 32, true>(routed, shared, tab_dev, tab_val, k, act, h_mid, shared_out, hidden_out, st);
  if (cpr <= 64) return down_inst<BITS, 64, true>(routed, shared, tab_dev, tab_val, k, act, h_mid, shared_out, hidden_out, st);
  *unsupported = true;
  return hipSuccess;
}

hipError_t launch_down_combine(const BlobGeom& routed, const BlobGeom& shared,
                               const FfnTable* tab_dev, const FfnTable& tab_val, uint32_t n_slots,
                               const float* act, const float* h_mid, const float* shared_out,
                               float* hidden_out, hipStream_t st, bool* unsupported) {
  *unsupported = false;
  (void)n_slots;
  const uint32_t k = tab_val.k;
  return routed.bits == 4 ? down_bits<4>(routed, shared, tab_dev, tab_val, k, act, h_mid,
                                         shared_out, hidden_out, st, unsupported)
                          : down_bits<3>(routed, shared, tab_dev, tab_val, k, act, h_mid,
                                         shared_out, hidden_out, st, unsupported);
}

// ---------------------------------------------------------------------------
// Prefill through the per-phase kernels, for expert shapes the grouped GEMMs
// have no tiles for (hidden or inter not a multiple of 256, hidden below
// 1024): per token, a route table of its k experts in ascending expert
// order (the order moe_permute_fuse_cpu, moe_cpu.rs:282-339, adds them in),
// then k_gateup and k_down_combine over that table with a zero residual.
// ---------------------------------------------------------------------------
// One wave: token t's table. An expert id out of range or repeated within
// the token sets the device error word (as the grouped path's bucketing
// does) and reads expert 0 instead, so nothing is read out of bounds.
__global__ __launch_bounds__(64) void k_pt_table(const int32_t* __restrict__ idx, const float* __restrict__ w,
                                                 uint32_t k, uint32_t E, const uint8_t* experts, uint64_t stride,
                                                 FfnTable* tab, uint32_t* err) {
  const int lane = threadIdx.x;
  const bool live = lane < (int)k;
  const int32_t id = live ? idx[lane] : 0x7FFFFFFF;
  const float wt = live ? w[lane] : 0.f;
  bool bad = live && (id < 0 || (uint32_t)id >= E);
  // Rank: entries with a smaller id, or the same id in an earlier slot.
  uint32_t rank = 0;
  for (uint32_t s = 0; s < k; ++s) {
    const int32_t o = __shfl(id, s, kWave);
    rank += (o < id || (o == id && (int)s < lane)) ? 1u : 0u;
    bad |= live && o == id && (int)s != lane;
  }
  if (__ballot(bad) && lane == 0) *err = 2u;
  if (live) {
    const uint32_t e = (id >= 0 && (uint32_t)id < E) ? (uint32_t)id : 0u;
    tab->blob[rank] = experts + (uint64_t)e * stride;
    tab->weight[rank] = wt;
  }
  if (lane == 0) {
    tab->k = k;
    tab->has_shared = 0;
    tab->shared_gate = __builtin_nanf("");
  }
}

// x as f32 rows (bf16 widened; f32 input is used in place) and the zero
// residual.
__global__ __launch_bounds__(256) void k_pt_prep(const uint16_t* __restrict__ xb, uint64_t n, float* __restrict__ xf,
                                                 uint32_t hidden, float* __restrict__ zero) {
  for (uint64_t i = (uint64_t)blockIdx.x * 256 + threadIdx.x; i < n; i += (uint64_t)gridDim.x * 256)
    xf[i] = bf16f(xb[i]);
  if (blockIdx.x == 0)
    for (uint32_t i = threadIdx.x; i < hidden; i += 256) zero[i] = 0.f;
}

uint64_t prefill_tokens_workspace(uint32_t hidden, uint32_t inter, uint32_t n_tokens, uint32_t k, bool x_bf16) {
  auto al = [](uint64_t b) { return (b + 255) / 256 * 256; };
  return al(sizeof(FfnTable)) + al((uint64_t)hidden * 4) + al((uint64_t)(k + 1) * inter * 4) +
         (x_bf16 ? al((uint64_t)n_tokens * hidden * 4) : 0u);
}

hipError_t launch_prefill_tokens(const BlobGeom& g, const uint8_t* experts, uint64_t stride, uint32_t E,
                                 const int32_t* idx, const float* w, const void* x, bool x_bf16, uint32_t n,
                                 uint32_t k, float* out, uint8_t* ws, uint32_t* err, hipStream_t st,
                                 bool* unsupported) {
  *unsupported = false;
  auto al = [](uint64_t b) { return (b + 255) / 256 * 256; };
  FfnTable* tab = reinterpret_cast<FfnTable*>(ws);
  float* zero = reinterpret_cast<float*>(ws + al(sizeof(FfnTable)));
  float* act = reinterpret_cast<float*>(reinterpret_cast<uint8_t*>(zero) + al((uint64_t)g.hidden * 4));
  float* xf = x_bf16 ? reinterpret_cast<float*>(reinterpret_cast<uint8_t*>(act) + al((uint64_t)(k + 1) * g.inter * 4))
                     : const_cast<float*>(static_cast<const float*>(x));
  const uint64_t nx = x_bf16 ? (uint64_t)n * g.hidden : 0u;
  const uint32_t pb = x_bf16 ? (uint32_t)((nx + 255) / 256 < 1024 ? (nx + 255) / 256 : 1024) : 1u;
  hipLaunchKernelGGL(k_pt_prep, dim3(pb), dim3(256), 0, st, static_cast<const uint16_t*>(x), nx, xf, g.hidden, zero);
  hipError_t e = hipGetLastError();
  FfnTable tv{};
  tv.k = k;
  for (uint32_t t = 0; t < n && e == hipSuccess; ++t) {
    hipLaunchKernelGGL(k_pt_table, dim3(1), dim3(64), 0, st, idx + (size_t)t * k, w + (size_t)t * k, k, E, experts,
                       stride, tab, err);
    e = hipGetLastError();
    if (e == hipSuccess) e = launch_gateup(g, g, tab, tv, k, xf + (size_t)t * g.hidden, act, st, unsupported);
    if (e == hipSuccess && !*unsupported)
      e = launch_down_combine(g, g, tab, tv, k, act, zero, nullptr, out + (size_t)t * g.hidden, st, unsupported);
    if (*unsupported) break;
  }
  return e;
}

}  // namespace smoe
