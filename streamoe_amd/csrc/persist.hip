// persist.hip — one persistent kernel for a token's MoE decode through many
// layers (gfx950).
//
// A kernel launch costs ~1.6 us even inside a HIP graph, and a grid-wide
// counter barrier ~10 us at 256 blocks on MI355X (atomics on one address
// serialise). A decode layer has three all-to-all dependencies:
// hidden -> router logits -> expert activations -> hidden. This kernel
// keeps one cooperative grid resident for all layers and passes every
// value between blocks as a tagged 64-bit word (epoch << 32 | bits):
// consumers poll the data itself, so there is no barrier counter and no
// separate flag round trip. Epochs are unique per (launch, layer), so a
// stale value can never be mistaken for a fresh one.
//
// Grid: nb worker blocks + 1 coordinator block.
//   phase 1  every worker: x = RMSNorm(hidden) (or the input at layer 0),
//            then its share of the router rows (weights were loaded before
//            the wait) -> tagged logits.
//   phase 2  every worker: wave 0 takes the logits, softmax, top-k SET
//            (k largest; the reference's running-minimum scan keeps exactly
//            these when the k-th and (k+1)-th probabilities differ), then
//            all waves load their gate/up rows and their down rows and
//            compute act = silu(gate) * up -> tagged act.
//            coordinator: the exact running-minimum slot order of the
//            reference (moe_router.rs:83-124), renormalised weights ->
//            tagged route table. It runs beside the gate/up work.
//   phase 3  every worker: take act and the route table, down rows for its
//            own output rows, combine in slot order, residual -> tagged
//            hidden.
// Every wait is bounded: on timeout a block records an error code and the
// whole grid drains.
#include "common.h"
#include "kernels.h"
#include "persist.h"
#include "topk.h"

namespace smoe {

constexpr unsigned kSpinLimit = 1u << 21;
constexpr int kKP = 8;  // max routed k on this path

__device__ __forceinline__ uint64_t pack(uint32_t tag, uint32_t v) {
  return ((uint64_t)tag << 32) | v;
}
__device__ __forceinline__ uint64_t ld_tagged(const uint64_t* p) {
  return __hip_atomic_load(p, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ void st_tagged(uint64_t* p, uint32_t tag, float v) {
  __hip_atomic_store(p, pack(tag, __float_as_uint(v)), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ void st_tagged_u(uint64_t* p, uint32_t tag, uint32_t v) {
  __hip_atomic_store(p, pack(tag, v), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ uint32_t ld_err(const uint32_t* e) {
  return __hip_atomic_load(e, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

// Wait until *p carries `tag`; returns false on timeout or grid error.
__device__ __forceinline__ bool wait_tagged(const uint64_t* p, uint32_t tag, uint32_t* val,
                                            const uint32_t* err) {
  unsigned spins = 0;
  while (true) {
    const uint64_t v = ld_tagged(p);
    if ((uint32_t)(v >> 32) == tag) {
      *val = (uint32_t)v;
      return true;
    }
    if ((spins & 63) == 0 && ld_err(err)) return false;
    if (++spins > kSpinLimit) {
      __hip_atomic_store(const_cast<uint32_t*>(err), 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
      return false;
    }
  }
}

// Wait until all N words p[idx[n]] carry `tag`: the N loads of one poll are
// independent, so a poll costs one memory round trip. Returns false on
// timeout or grid error.
template <int N>
__device__ __forceinline__ bool wait_tagged_n(const uint64_t* p, const uint32_t (&idx)[N],
                                              const bool (&valid)[N], uint32_t tag,
                                              uint32_t (&val)[N], const uint32_t* err) {
  bool done[N];
#pragma unroll
  for (int n = 0; n < N; ++n) done[n] = !valid[n];
  unsigned spins = 0;
  while (true) {
    uint64_t v[N];
#pragma unroll
    for (int n = 0; n < N; ++n) v[n] = done[n] ? 0 : ld_tagged(p + idx[n]);
    bool all = true;
#pragma unroll
    for (int n = 0; n < N; ++n) {
      if (!done[n] && (uint32_t)(v[n] >> 32) == tag) {
        val[n] = (uint32_t)v[n];
        done[n] = true;
      }
      all &= done[n];
    }
    if (all) return true;
    if ((spins & 15) == 0 && ld_err(err)) return false;
    if (++spins > kSpinLimit) {
      __hip_atomic_store(const_cast<uint32_t*>(err), 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
      return false;
    }
    __builtin_amdgcn_s_sleep(1);
  }
}

// Wait until the N words p[base + m * stride] (m < N, index < limit) carry
// `tag` and store their values to dst[index]. Each poll issues all pending
// loads before checking any, so it costs one memory round trip; only a
// 64-bit pending mask stays live between polls. Returns false on timeout or
// grid error.
template <int N>
__device__ __forceinline__ bool poll_to_lds(const uint64_t* p, uint32_t base, uint32_t stride,
                                            uint32_t limit, uint32_t tag, float* dst,
                                            const uint32_t* err) {
  static_assert(N <= 64, "pending mask is 64 bits");
  uint64_t pending = 0;
#pragma unroll
  for (int m = 0; m < N; ++m)
    if (base + m * stride < limit) pending |= 1ull << m;
  unsigned spins = 0;
  while (pending) {
    uint64_t v[N];
#pragma unroll
    for (int m = 0; m < N; ++m) v[m] = (pending >> m) & 1 ? ld_tagged(p + base + m * stride) : 0;
#pragma unroll
    for (int m = 0; m < N; ++m)
      if (((pending >> m) & 1) && (uint32_t)(v[m] >> 32) == tag) {
        dst[base + m * stride] = __uint_as_float((uint32_t)v[m]);
        pending &= ~(1ull << m);
      }
    if (!pending) break;
    if ((spins & 15) == 0 && ld_err(err)) return false;
    if (++spins > kSpinLimit) {
      __hip_atomic_store(const_cast<uint32_t*>(err), 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
      return false;
    }
    __builtin_amdgcn_s_sleep(1);
  }
  return true;
}

__device__ __forceinline__ void fail(uint32_t* err, uint32_t code) {
  if (!ld_err(err)) __hip_atomic_store(err, code, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

// Raw chunks are kept as four words; a 3-bit chunk uses the first three.
__device__ __forceinline__ Raw<4> widen(const Raw<4>& r) { return r; }
__device__ __forceinline__ Raw<4> widen(const Raw<3>& r) {
  Raw<4> w;
  w.d[0] = r.d[0];
  w.d[1] = r.d[1];
  w.d[2] = r.d[2];
  w.d[3] = 0;
  return w;
}
template <int BITS>
__device__ __forceinline__ Raw<BITS> narrow(const Raw<4>& r);
template <>
__device__ __forceinline__ Raw<4> narrow<4>(const Raw<4>& r) {
  return r;
}
template <>
__device__ __forceinline__ Raw<3> narrow<3>(const Raw<4>& r) {
  Raw<3> n;
  n.d[0] = r.d[0];
  n.d[1] = r.d[1];
  n.d[2] = r.d[2];
  return n;
}

// Trace layout: worker b, layer l, point p at [(l * nb + b) * 8 + p];
// the coordinator at [n_layers * nb * 8 + l * 2 + p].
__device__ __forceinline__ void trace(const PArgs& a, uint32_t l, uint32_t nb, uint32_t p) {
  if (a.trace && threadIdx.x == 0) a.trace[((size_t)l * nb + blockIdx.x) * 8 + p] = __builtin_amdgcn_s_memrealtime();
}

// ---------------------------------------------------------------------------
// The persistent kernel.
//   H = 32 * CPRH, I = 32 * CPRI; NW waves per block; P logits per lane;
//   MAXI gate/up items per wave; MAXD down passes per wave.
// ---------------------------------------------------------------------------
template <int BITS, int CPRH, int CPRI, int NW, int P, int MAXI, int MAXD>
__global__ __launch_bounds__(NW * 64) void k_decode_persistent(const PArgs a) {
  constexpr int H = CPRH * kChunk;
  constexpr int I = CPRI * kChunk;
  constexpr int NT = NW * 64;
  static_assert(CPRH == 64, "gate/up rows are one wave of 16-byte chunks");
  static_assert(CPRI <= 64 && (64 % CPRI) == 0, "down rows must tile a wave");
  constexpr int LI = CPRI;         // lanes per down row
  constexpr int RPPI = 64 / LI;    // down rows per wave pass
  constexpr int FPT = H / NT;      // router floats per thread
  static_assert(FPT % 4 == 0, "router row split in float4s");
  constexpr int RJ = 2;            // max router rows per block
  constexpr int RBMAX = 16;        // max own output rows per block
  constexpr int HPT = H / NT;      // hidden entries polled per thread
  constexpr int APT = (kKP + 1) * I / NT;  // act entries polled per thread (max)

  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const bool coord = a.idx_out || a.w_out;
  const uint32_t nb = gridDim.x - (coord ? 1u : 0u);
  const uint32_t E = a.E, k = a.k;
  const uint32_t nslots = k + (a.has_shared ? 1u : 0u);
  const uint32_t nrouter = E + (a.has_gate ? 1u : 0u);

  // ------------------------------ coordinator ------------------------------
  // The exact running-minimum slot order of the reference and the weights
  // renormalised in that order, for the caller's idx/w outputs only.
  if (coord && blockIdx.x == nb) {
    if (wave != 0) return;
    __shared__ int32_t cidx[kKP];
    __shared__ float cval[kKP];
    for (uint32_t l = 0; l < a.n_layers; ++l) {
      const uint32_t ep = a.epoch + l;
      uint32_t id[P], bits[P];
      bool valid[P];
#pragma unroll
      for (int e = 0; e < P; ++e) {
        id[e] = lane * P + e;
        valid[e] = id[e] < E;
        bits[e] = 0;
      }
      const bool ok = wait_tagged_n<P>(a.tag_logit, id, valid, ep, bits, a.err);
      if (__ballot(!ok)) return;
      if (a.trace && lane == 0) a.trace[(size_t)a.n_layers * nb * 8 + l * 2 + 0] = __builtin_amdgcn_s_memrealtime();
      float v[P];
#pragma unroll
      for (int e = 0; e < P; ++e) v[e] = valid[e] ? __uint_as_float(bits[e]) : -INFINITY;
      wave_softmax<P>(v, E, lane);
      exact_topk<P>(v, k, lane, cidx, cval);
      __builtin_amdgcn_wave_barrier();
      __builtin_amdgcn_fence(__ATOMIC_SEQ_CST, "workgroup");
      if (lane < (int)k) {
        float w = cval[lane];
        if (a.normalize) {
          float sum = 0.f;
          for (uint32_t i = 0; i < k; ++i) sum += cval[i];
          if (sum > 0.f) w = cval[lane] * (1.0f / sum);
        }
        if (a.idx_out) a.idx_out[(size_t)l * k + lane] = cidx[lane];
        if (a.w_out) a.w_out[(size_t)l * k + lane] = w;
      }
      if (a.trace && lane == 0) a.trace[(size_t)a.n_layers * nb * 8 + l * 2 + 1] = __builtin_amdgcn_s_memrealtime();
    }
    return;
  }

  // ------------------------------ workers ----------------------------------
  __shared__ float sx[H];
  __shared__ float sr[H];
  __shared__ float sact[(kKP + 1) * I];
  __shared__ float sout[(kKP + 1) * RBMAX];
  __shared__ float sred[RJ][NW];
  __shared__ float sinv;
  __shared__ int32_t sset[kKP];
  __shared__ float swt[kKP];
  __shared__ float sgate;
  __shared__ uint32_t sfail;

  const uint32_t b = blockIdx.x;
  const uint32_t RB = (H + nb - 1) / nb;  // own output rows [b*RB, min(b*RB + RB, H))
  const uint32_t NWT = nb * NW;
  const uint32_t gw = b * NW + wave;
  const uint32_t gpr_h = H / a.group, gpr_i = I / a.group;
  const uint32_t cshift = __builtin_ctz(a.group / kChunk);
  const BlobGeom& gR = a.geom_routed;
  const BlobGeom& gS = a.geom_shared;
  if (tid == 0) sfail = 0;

  for (uint32_t l = 0; l < a.n_layers; ++l) {
    const uint32_t ep = a.epoch + l;
    const PLayer L = a.L[l];
    trace(a, l, nb, 0);

    // -------- loads known before any wait: router rows, shared expert --------
    f32x4 rw[RJ][FPT / 4];
#pragma unroll
    for (int j = 0; j < RJ; ++j) {
      const uint32_t e = b + j * nb;
      if (e < nrouter) {
        const float* row = e < E ? L.router + (size_t)e * H : L.gate;
#pragma unroll
        for (int q = 0; q < FPT / 4; ++q)
          rw[j][q] = __builtin_nontemporal_load(reinterpret_cast<const f32x4*>(row) + tid + q * NT);
      }
    }
    // Gate/up items: item i = gw + j * NWT -> slot i / I, row i % I.
    Raw<4> gq[MAXI], uq[MAXI];  // 3-bit rows use words 0..2
    float gs[MAXI], gb[MAXI], us[MAXI], ub[MAXI];
    auto load_item = [&](int j, const uint8_t* blob, bool shared_slot, uint32_t row) {
      const uint32_t c = lane;
      const size_t gi = ((size_t)row * gpr_h + (c >> cshift)) * 2;
      const BlobGeom& g = shared_slot ? gS : gR;
      if (shared_slot || BITS == 4) {
        const size_t off = (size_t)row * (CPRH * 16) + c * 16;
        gq[j] = load_raw<4>(blob + g.w[0] + off);
        uq[j] = load_raw<4>(blob + g.w[1] + off);
      } else {
        const size_t off = (size_t)row * (CPRH * chunk_bytes<BITS>()) + c * chunk_bytes<BITS>();
        gq[j] = widen(load_raw<BITS>(blob + g.w[0] + off));
        uq[j] = widen(load_raw<BITS>(blob + g.w[1] + off));
      }
      gs[j] = bf16f(*reinterpret_cast<const uint16_t*>(blob + g.s[0] + gi));
      gb[j] = bf16f(*reinterpret_cast<const uint16_t*>(blob + g.b[0] + gi));
      us[j] = bf16f(*reinterpret_cast<const uint16_t*>(blob + g.s[1] + gi));
      ub[j] = bf16f(*reinterpret_cast<const uint16_t*>(blob + g.b[1] + gi));
    };
    if (a.has_shared) {
#pragma unroll
      for (int j = 0; j < MAXI; ++j) {
        const uint32_t i = gw + j * NWT;
        if (i < nslots * I && i / I == k) load_item(j, L.shared, true, i % I);
      }
    }
    // Down passes: block item t = (j * NW + wave) * RPPI + lane / LI -> slot
    // t / RB, own row t % RB; lane % LI is the input chunk.
    Raw<4> dq[MAXD];
    float ds[MAXD], db[MAXD];
    const uint32_t dch = lane % LI;
    auto down_item = [&](int j, uint32_t* p, uint32_t* row) {
      const uint32_t t = (j * NW + wave) * RPPI + lane / LI;
      *p = t / RB;
      *row = b * RB + t % RB;
    };
    auto load_down = [&](int j, const uint8_t* blob, bool shared_slot, uint32_t row) {
      const size_t gi = ((size_t)row * gpr_i + (dch >> cshift)) * 2;
      const BlobGeom& g = shared_slot ? gS : gR;
      if (shared_slot || BITS == 4)
        dq[j] = load_raw<4>(blob + g.w[2] + (size_t)row * (CPRI * 16) + dch * 16);
      else
        dq[j] = widen(load_raw<BITS>(blob + g.w[2] + (size_t)row * (CPRI * chunk_bytes<BITS>()) +
                                     dch * chunk_bytes<BITS>()));
      ds[j] = bf16f(*reinterpret_cast<const uint16_t*>(blob + g.s[2] + gi));
      db[j] = bf16f(*reinterpret_cast<const uint16_t*>(blob + g.b[2] + gi));
    };
    if (a.has_shared) {
#pragma unroll
      for (int j = 0; j < MAXD; ++j) {
        uint32_t p, row;
        down_item(j, &p, &row);
        if (p == k && row < H) load_down(j, L.shared, true, row);
      }
    }

    // -------- phase 1: x, router rows --------
    if (l == 0) {
      for (uint32_t i = tid; i < H; i += NT) {
        sx[i] = a.input[i];
        sr[i] = a.resid_in[i];
      }
    } else {
      const bool ok = poll_to_lds<HPT>(a.tag_resid, tid, NT, H, ep - 1, sr, a.err);
      float ss = 0.f;
#pragma unroll
      for (int m = 0; m < HPT; ++m) {
        const float r = sr[tid + m * NT];
        ss += r * r;
      }
      if (!ok) sfail = 1;
      ss = group_sum_last<64>(ss);
      if (lane == 63) sred[0][wave] = ss;
      __syncthreads();
      if (sfail) return;
      if (tid == 0) {
        float t = 0.f;
        for (int w = 0; w < NW; ++w) t += sred[0][w];
        sinv = L.norm ? 1.0f / sqrtf(t / (float)H + a.eps) : 1.0f;
      }
      __syncthreads();
      const float inv = sinv;
      for (uint32_t i = tid; i < H; i += NT) sx[i] = L.norm ? sr[i] * inv * bf16f(L.norm[i]) : sr[i];
    }
    __syncthreads();
    trace(a, l, nb, 1);
#pragma unroll
    for (int j = 0; j < RJ; ++j) {
      const uint32_t e = b + j * nb;
      float acc = 0.f;
      if (e < nrouter) {
#pragma unroll
        for (int q = 0; q < FPT / 4; ++q) {
          const int c = 4 * (tid + q * NT);
          acc = __builtin_fmaf(rw[j][q].x, sx[c + 0], acc);
          acc = __builtin_fmaf(rw[j][q].y, sx[c + 1], acc);
          acc = __builtin_fmaf(rw[j][q].z, sx[c + 2], acc);
          acc = __builtin_fmaf(rw[j][q].w, sx[c + 3], acc);
        }
      }
      acc = group_sum_last<64>(acc);
      if (lane == 63) sred[j][wave] = acc;
    }
    __syncthreads();
    if (tid < RJ) {
      const uint32_t e = b + tid * nb;
      if (e < nrouter) {
        float t = 0.f;
        for (int w = 0; w < NW; ++w) t += sred[tid][w];
        st_tagged(a.tag_logit + e, ep, t);
      }
    }
    trace(a, l, nb, 2);

    // -------- phase 2: top-k set, gate/up --------
    if (wave == 0) {
      uint32_t id[P + 1], bits[P + 1];
      bool valid[P + 1];
#pragma unroll
      for (int e = 0; e < P; ++e) {
        id[e] = lane * P + e;
        valid[e] = id[e] < E;
        bits[e] = 0;
      }
      id[P] = E;
      valid[P] = a.has_gate && lane == 0;
      bits[P] = 0;
      const bool ok = wait_tagged_n<P + 1>(a.tag_logit, id, valid, ep, bits, a.err);
      if (__ballot(!ok)) {
        if (lane == 0) sfail = 1;
      } else {
        if (lane == 0 && a.has_gate) sgate = __uint_as_float(bits[P]);
        float v[P];
#pragma unroll
        for (int e = 0; e < P; ++e) v[e] = valid[e] ? __uint_as_float(bits[e]) : -INFINITY;
        wave_softmax<P>(v, E, lane);
        if (!topk_set<P>(v, E, k, lane, sset)) {
          // Degenerate scores (boundary tie, NaN): the exact scan decides.
          __shared__ int32_t fidx[kKP];
          __shared__ float fval[kKP];
          exact_topk<P>(v, k, lane, fidx, fval);
          __builtin_amdgcn_wave_barrier();
          __builtin_amdgcn_fence(__ATOMIC_SEQ_CST, "workgroup");
          if (lane < (int)k) {
            const int32_t my = fidx[lane];
            uint32_t rank = 0;
            for (uint32_t i = 0; i < k; ++i) rank += fidx[i] < my ? 1u : 0u;
            sset[rank] = my;
          }
        }
        __builtin_amdgcn_wave_barrier();
        __builtin_amdgcn_fence(__ATOMIC_SEQ_CST, "workgroup");
        // Routing weights of the set (ascending expert index), renormalised
        // in that order when the layer renormalises.
        // Gather each set member's probability from its owner lane.
        for (uint32_t s2 = 0; s2 < k; ++s2) {
          const int32_t j = sset[s2];
          const int owner = j / P, slot = j % P;
          float mine = 0.f;
#pragma unroll
          for (int e = 0; e < P; ++e)
            if (e == slot) mine = v[e];
          const float pj = readlane_f(mine, owner);
          if (lane == 0) swt[s2] = pj;
        }
        __builtin_amdgcn_wave_barrier();
        __builtin_amdgcn_fence(__ATOMIC_SEQ_CST, "workgroup");
        if (a.normalize && lane == 0) {
          float sum = 0.f;
          for (uint32_t i = 0; i < k; ++i) sum += swt[i];
          if (sum > 0.f) {
            const float inv = 1.0f / sum;
            for (uint32_t i = 0; i < k; ++i) swt[i] = swt[i] * inv;
          }
        }
      }
    }
    __syncthreads();
    if (sfail) return;
    trace(a, l, nb, 3);
    // Routed gate/up and down loads.
#pragma unroll
    for (int j = 0; j < MAXI; ++j) {
      const uint32_t i = gw + j * NWT;
      if (i < nslots * I && i / I < k)
        load_item(j, L.experts + (size_t)sset[i / I] * L.stride, false, i % I);
    }
#pragma unroll
    for (int j = 0; j < MAXD; ++j) {
      uint32_t p, row;
      down_item(j, &p, &row);
      if (p < k && row < H) load_down(j, L.experts + (size_t)sset[p] * L.stride, false, row);
    }
    trace(a, l, nb, 7);
    {
      float xr[kChunk];
#pragma unroll
      for (int q = 0; q < kChunk; ++q) xr[q] = sx[lane * kChunk + q];
      const float xs = xsum(xr);
#pragma unroll
      for (int j = 0; j < MAXI; ++j) {
        const uint32_t i = gw + j * NWT;
        if (i < nslots * I) {
          const uint32_t p = i / I;
          float pg, pu;
          if (p == k || BITS == 4) {
            pg = chunk_dot<4>(gq[j], xr, xs, gs[j], gb[j]);
            pu = chunk_dot<4>(uq[j], xr, xs, us[j], ub[j]);
          } else {
            pg = chunk_dot<BITS>(narrow<BITS>(gq[j]), xr, xs, gs[j], gb[j]);
            pu = chunk_dot<BITS>(narrow<BITS>(uq[j]), xr, xs, us[j], ub[j]);
          }
          const float g = group_sum_last<64>(pg);
          const float u = group_sum_last<64>(pu);
          if (lane == 63) st_tagged(a.tag_act + i, ep, silu_mul(g, u));
        }
      }
    }
    trace(a, l, nb, 4);

    // -------- phase 3: act, down, combine --------
    {
      const bool ok = poll_to_lds<APT>(a.tag_act, tid, NT, nslots * I, ep, sact, a.err);
      if (!ok) sfail = 1;
    }
    __syncthreads();
    if (sfail) return;
    trace(a, l, nb, 5);
#pragma unroll
    for (int j = 0; j < MAXD; ++j) {
      uint32_t p, row;
      down_item(j, &p, &row);
      float part = 0.f;
      const bool live = p < nslots && row < H;
      if (live) {
        float av[kChunk];
#pragma unroll
        for (int q = 0; q < kChunk; ++q) av[q] = sact[p * I + dch * kChunk + q];
        const float as = xsum(av);
        part = (p == k || BITS == 4) ? chunk_dot<4>(dq[j], av, as, ds[j], db[j])
                                     : chunk_dot<BITS>(narrow<BITS>(dq[j]), av, as, ds[j], db[j]);
      }
      const float o = group_sum_last<LI>(part);
      if (dch == LI - 1 && live) sout[p * RBMAX + (row - b * RB)] = o;
    }
    __syncthreads();
    if (tid < RB && b * RB + tid < H) {
      const uint32_t row = b * RB + tid;
      float moe = 0.f;
      for (uint32_t s2 = 0; s2 < k; ++s2) moe = __builtin_fmaf(sout[s2 * RBMAX + tid], swt[s2], moe);
      float sum = moe;
      if (a.has_shared) {
        const float sh = sout[k * RBMAX + tid];
        sum = a.has_gate ? __builtin_fmaf(sh, sigmoidf_ref(sgate), moe) : moe + sh;
      }
      const float val = sr[row] + sum;
      st_tagged(a.tag_resid + row, ep, val);
      if (l + 1 == a.n_layers) a.out[row] = val;
    }
    trace(a, l, nb, 6);
    __syncthreads();
  }
}

// ---------------------------------------------------------------------------
// Host launcher.
// ---------------------------------------------------------------------------
template <int BITS, int CPRH, int CPRI, int NW, int P, int MAXI, int MAXD>
static hipError_t launch_inst(const PArgs& a, uint32_t grid, hipStream_t st) {
  void* args[] = {(void*)&a};
  return hipLaunchCooperativeKernel(
      reinterpret_cast<const void*>(&k_decode_persistent<BITS, CPRH, CPRI, NW, P, MAXI, MAXD>),
      dim3(grid), dim3(NW * 64), args, 0, st);
}

// Variant table: (inter, max experts) -> NW, P, MAXI, MAXD.
struct PVariant {
  uint32_t inter, max_experts, nw, p, maxi, maxd;
};
static const PVariant kVariants[] = {
    {512, 256, 4, 4, 5, 6},   // Qwen3.6-A3B shape
    {1024, 64, 4, 1, 9, 9},   // OLMoE shape
};

bool persist_plan(uint32_t hidden, uint32_t inter, uint32_t n_experts, uint32_t k, uint32_t bits,
                  bool shared, bool coordinator, PPlan* plan) {
  if (hidden != 2048 || k > (uint32_t)kKP || k < 1) return false;
  if (bits != 4 && bits != 3) return false;
  const uint32_t nslots = k + (shared ? 1 : 0);
  for (uint32_t v = 0; v < sizeof(kVariants) / sizeof(kVariants[0]); ++v) {
    const PVariant& pv = kVariants[v];
    if (inter != pv.inter || n_experts > pv.max_experts || n_experts > 64 * pv.p) continue;
    PPlan p{};
    p.variant = v;
    p.nw = pv.nw;
    p.nb = coordinator ? 255 : 256;  // one block per CU; the coordinator takes the last CU
    const uint32_t nwt = p.nb * p.nw;
    const uint32_t items_per_wave = (nslots * inter + nwt - 1) / nwt;
    const uint32_t rb = (hidden + p.nb - 1) / p.nb;
    const uint32_t rppi = 64 / (inter / 32);
    const uint32_t passes = (nslots * rb + rppi - 1) / rppi;
    const uint32_t passes_per_wave = (passes + p.nw - 1) / p.nw;
    if (items_per_wave > pv.maxi || passes_per_wave > pv.maxd || rb > 16) return false;
    if (n_experts + 1 > 2 * p.nb) return false;
    if ((kKP + 1) * inter / (p.nw * 64) * (p.nw * 64) != (kKP + 1) * inter) return false;
    p.grid = p.nb + (coordinator ? 1 : 0);
    *plan = p;
    return true;
  }
  return false;
}

hipError_t launch_decode_persistent(const PArgs& a, const PPlan& plan, uint32_t bits,
                                    hipStream_t st) {
  if (plan.variant == 0) {
    return bits == 4 ? launch_inst<4, 64, 16, 4, 4, 5, 6>(a, plan.grid, st)
                     : launch_inst<3, 64, 16, 4, 4, 5, 6>(a, plan.grid, st);
  }
  return bits == 4 ? launch_inst<4, 64, 32, 4, 1, 9, 9>(a, plan.grid, st)
                   : launch_inst<3, 64, 32, 4, 1, 9, 9>(a, plan.grid, st);
}

}  // namespace smoe
