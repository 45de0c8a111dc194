// router.hip — noaux_tc routing (DeepSeek-V3 / Cogito-V2) from precomputed
// gate logits, one wave per token.
//
//   k_noaux_topk  sigmoid scores, correction bias, group scores (sum of the
//                 top two biased scores of each group), the reference's
//                 running-minimum top-k over the group scores, the group
//                 mask, the same top-k over the masked biased scores, and
//                 the renormalised, scaled un-biased weights, in the
//                 reference's slot order and summation order
//                 (crates/streammoe/src/riir/moe/moe_router.rs:211-330).
//
// Lane l holds experts l, l + 64, ... Groups of a power-of-two size up to
// 64 take their top two with a lane butterfly (the scan's result: the two
// largest values with multiplicity); other sizes are scanned in lane g for
// group g over an LDS copy strided by group_size + 1 (so the lanes' reads
// fall in different banks), with the reference's compares. Both top-k
// passes use exact_topk_t, the reference's scan order and tie rules.
#include "common.h"
#include "kernels.h"
#include "topk.h"

namespace smoe {

// (largest, second largest) pairs merged with the pair the DPP control
// brings in (lanes outside ROW_MASK merge with (-inf, -inf): unchanged).
template <int CTRL, int ROW_MASK = 0xF, int P>
__device__ __forceinline__ void top2_merge(float (&a1)[P], float (&a2)[P]) {
#pragma unroll
  for (int e = 0; e < P; ++e) {
    const float c1 = __int_as_float(__builtin_amdgcn_update_dpp(__float_as_int(-INFINITY), __float_as_int(a1[e]),
                                                                CTRL, ROW_MASK, 0xF, false));
    const float c2 = __int_as_float(__builtin_amdgcn_update_dpp(__float_as_int(-INFINITY), __float_as_int(a2[e]),
                                                                CTRL, ROW_MASK, 0xF, false));
    const float t2 = fmaxf(fminf(a1[e], c1), fmaxf(a2[e], c2));
    a1[e] = fmaxf(a1[e], c1);
    a2[e] = t2;
  }
}

template <int P>
__global__ __launch_bounds__(64) void k_noaux_topk(const float* logits,
                                                   const float* __restrict__ bias, uint32_t n,
                                                   uint32_t n_group, uint32_t topk_group, uint32_t k,
                                                   float scale, float* scores_out, RouteOut out) {
  __shared__ float s_sig[64 * P];        // un-biased sigmoid scores
  __shared__ float s_bsd[64 * P + 64];   // biased scores, element j at j + j / group_size (scan layout)
  __shared__ float s_gsc[64];            // group scores
  __shared__ int32_t s_idx[kMaxK];
  __shared__ float s_val[kMaxK];
  const uint32_t t = blockIdx.x;
  const int lane = threadIdx.x;
  const uint32_t gs = n / n_group;
  // Power-of-two groups of at most 64 elements lie inside one 64-element
  // chunk: their top two come from a lane butterfly; other sizes are
  // scanned from LDS.
  const bool lanes_path = gs <= 64 && (gs & (gs - 1)) == 0;
  const float* lg = logits + (size_t)t * n;

  // 1-2. s = 1 / (1 + exp(-logit)); biased = s + correction_bias. Lane l
  // holds elements l, l + 64, ... (coalesced loads).
  float b[P];
#pragma unroll
  for (int e = 0; e < P; ++e) {
    const uint32_t j = e * 64 + lane;
    b[e] = -INFINITY;
    if (j < n) {
      const float s = 1.0f / (1.0f + expf(-lg[j]));
      b[e] = s + bias[j];
      s_sig[j] = s;
      if (!lanes_path) s_bsd[j + j / gs] = b[e];
      if (scores_out) scores_out[(size_t)t * n + j] = s;
    }
  }

  // 3. Group score = top1 + top2 of the group's biased scores, as the
  // reference's linear scan (v > top1: shift; else v > top2) leaves them:
  // the two largest values with multiplicity, NaN never taken (here: -inf,
  // which no compare takes either).
  if (lanes_path) {
    // DPP merges of (largest, second) pairs over disjoint lane sets: quad
    // swaps (lane ^ 1, lane ^ 2), the 8-lane half-row mirror, the row
    // mirror (every lane of a group of <= 16 then holds its result), then
    // row 1 (3) takes row 0 (2) and row 3 rows 0-1: for 32 and 64 the
    // result is in the group's last lane.
    float a1[P], a2[P];
#pragma unroll
    for (int e = 0; e < P; ++e) {
      a1[e] = b[e] == b[e] ? b[e] : -INFINITY;
      a2[e] = -INFINITY;
    }
    if (gs >= 2) top2_merge<0xB1>(a1, a2);
    if (gs >= 4) top2_merge<0x4E>(a1, a2);
    if (gs >= 8) top2_merge<0x141>(a1, a2);
    if (gs >= 16) top2_merge<0x140>(a1, a2);
    if (gs >= 32) top2_merge<0x142, 0xA>(a1, a2);
    if (gs >= 64) top2_merge<0x143, 0xC>(a1, a2);
#pragma unroll
    for (int e = 0; e < P; ++e) {
      const uint32_t j = e * 64 + lane;
      if (j < n && j % gs == gs - 1) s_gsc[j / gs] = a1[e] + a2[e];
    }
  } else {
    __syncthreads();
    if ((uint32_t)lane < n_group) {
      const float* p = s_bsd + (size_t)lane * (gs + 1);
      float top1 = -INFINITY, top2 = -INFINITY;
      uint32_t i = 0;
      for (; i + 8 <= gs; i += 8) {
        float v[8];
#pragma unroll
        for (int u = 0; u < 8; ++u) v[u] = p[i + u];
#pragma unroll
        for (int u = 0; u < 8; ++u) {
          const bool gt1 = v[u] > top1, gt2 = v[u] > top2;
          top2 = gt1 ? top1 : (gt2 ? v[u] : top2);
          top1 = gt1 ? v[u] : top1;
        }
      }
      for (; i < gs; ++i) {
        const float v = p[i];
        const bool gt1 = v > top1, gt2 = v > top2;
        top2 = gt1 ? top1 : (gt2 ? v : top2);
        top1 = gt1 ? v : top1;
      }
      s_gsc[lane] = top1 + top2;
    }
  }
  __syncthreads();

  // 4. topk() of the group scores; lanes past n_group hold -inf, which
  // never beats a slot.
  float gsc[1] = {(uint32_t)lane < n_group ? s_gsc[lane] : -INFINITY};
  const int32_t kept = exact_topk_t<1>(gsc, topk_group, lane, nullptr, nullptr);

  // 5. Mask the groups that were not kept (a start slot that was never
  // replaced keeps group 0, as the reference's index set does): the OR of
  // the kept groups' bits over the queue lanes.
  const uint64_t bit = kept >= 0 ? 1ull << kept : 0ull;
  const uint32_t klo = wave_or_last((uint32_t)bit), khi = wave_or_last((uint32_t)(bit >> 32));
  const uint64_t keep = ((uint64_t)(uint32_t)__builtin_amdgcn_readlane((int)khi, 63) << 32) |
                        (uint32_t)__builtin_amdgcn_readlane((int)klo, 63);
#pragma unroll
  for (int e = 0; e < P; ++e) {
    const uint32_t j = e * 64 + lane;
    if (j >= n || !((keep >> (j / gs)) & 1ull)) b[e] = -INFINITY;
  }

  // 6. topk() of the masked biased scores.
  exact_topk_t<P>(b, k, lane, s_idx, s_val);
  __syncthreads();

  // 7. Gather the un-biased scores (lane s: slot s), sum them in slot
  // order, w *= 1 / sum when sum > 0, then w *= routed_scaling_factor.
  const int32_t id = lane < (int)k ? s_idx[lane] : 0;
  float w = s_sig[id];
  float sum = 0.f;
  for (uint32_t s = 0; s < k; ++s) sum += readlane_f(w, (int)s);
  if (lane < (int)k) {
    if (sum > 0.f) {
      const float inv = 1.0f / sum;
      w *= inv;
    }
    w *= scale;
    if (out.idx) out.idx[(size_t)t * k + lane] = id;
    if (out.weight) out.weight[(size_t)t * k + lane] = w;
    if (out.table && t == 0) {
      out.table->blob[lane] = out.experts + (uint64_t)id * out.stride;
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

hipError_t launch_noaux_topk(const float* logits, const float* bias, uint32_t n_tokens, uint32_t n,
                             uint32_t n_group, uint32_t topk_group, uint32_t k, float scale,
                             float* scores_out, const RouteOut& out, hipStream_t st) {
  if (n == 0 || n > kNoauxMaxExperts || n_group == 0 || n_group > kNoauxMaxGroups || n % n_group ||
      topk_group == 0 || topk_group > n_group || k == 0 || k > n || k > (uint32_t)kMaxK)
    return hipErrorInvalidValue;
  const uint32_t p = (n + 63) / 64;
  const dim3 grid(n_tokens), block(64);
  if (p <= 1)
    hipLaunchKernelGGL(k_noaux_topk<1>, grid, block, 0, st, logits, bias, n, n_group, topk_group, k, scale,
                       scores_out, out);
  else if (p <= 2)
    hipLaunchKernelGGL(k_noaux_topk<2>, grid, block, 0, st, logits, bias, n, n_group, topk_group, k, scale,
                       scores_out, out);
  else if (p <= 4)
    hipLaunchKernelGGL(k_noaux_topk<4>, grid, block, 0, st, logits, bias, n, n_group, topk_group, k, scale,
                       scores_out, out);
  else if (p <= 8)
    hipLaunchKernelGGL(k_noaux_topk<8>, grid, block, 0, st, logits, bias, n, n_group, topk_group, k, scale,
                       scores_out, out);
  else
    hipLaunchKernelGGL(k_noaux_topk<16>, grid, block, 0, st, logits, bias, n, n_group, topk_group, k, scale,
                       scores_out, out);
  return hipGetLastError();
}

}  // namespace smoe
