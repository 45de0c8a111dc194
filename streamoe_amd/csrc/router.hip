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
// Lane l holds experts [l*P, l*P + P). The group scan runs in lane g for
// group g over an LDS copy of the biased scores laid out with a stride of
// group_size + 1 (so the lanes' reads of element i fall in different
// banks), with the reference's sequential compares; both top-k passes use
// exact_topk, the reference's scan order and tie rules.
#include "common.h"
#include "kernels.h"
#include "topk.h"

namespace smoe {

template <int P>
__global__ __launch_bounds__(64) void k_noaux_topk(const float* logits,
                                                   const float* __restrict__ bias, uint32_t n,
                                                   uint32_t n_group, uint32_t topk_group, uint32_t k,
                                                   float scale, float* scores_out, RouteOut out) {
  __shared__ float s_sig[64 * P];        // un-biased sigmoid scores
  __shared__ float s_bsd[64 * P + 64];   // biased scores, element j at j + j / group_size
  __shared__ int32_t s_gidx[64], s_idx[kMaxK];
  __shared__ float s_gval[64], s_val[kMaxK];
  const uint32_t t = blockIdx.x;
  const int lane = threadIdx.x;
  const uint32_t gs = n / n_group;
  const float* lg = logits + (size_t)t * n;

  // 1-2. s = 1 / (1 + exp(-logit)); biased = s + correction_bias.
  float b[P];
#pragma unroll
  for (int e = 0; e < P; ++e) {
    const uint32_t j = lane * P + e;
    b[e] = -INFINITY;
    if (j < n) {
      const float s = 1.0f / (1.0f + expf(-lg[j]));
      b[e] = s + bias[j];
      s_sig[j] = s;
      s_bsd[j + j / gs] = b[e];
      if (scores_out) scores_out[(size_t)t * n + j] = s;
    }
  }
  __syncthreads();

  // 3. Group score = top1 + top2 by the reference's linear scan.
  float gsc[1] = {-INFINITY};
  if ((uint32_t)lane < n_group) {
    const float* p = s_bsd + (size_t)lane * (gs + 1);
    float top1 = -INFINITY, top2 = -INFINITY;
    for (uint32_t i = 0; i < gs; ++i) {
      const float v = p[i];
      if (v > top1) {
        top2 = top1;
        top1 = v;
      } else if (v > top2) {
        top2 = v;
      }
    }
    gsc[0] = top1 + top2;
  }

  // 4. topk() of the group scores; lanes past n_group hold -inf, which
  // never beats a slot.
  exact_topk<1>(gsc, topk_group, lane, s_gidx, s_gval);
  __syncthreads();

  // 5. Mask the groups that were not kept (a start slot that was never
  // replaced keeps group 0, as the reference's index set does).
  bool kept = false;
  for (uint32_t s = 0; s < topk_group; ++s) kept |= s_gidx[s] == lane;
  const uint64_t keep = __ballot((uint32_t)lane < n_group && kept);
#pragma unroll
  for (int e = 0; e < P; ++e) {
    const uint32_t j = lane * P + e;
    if (j >= n || !((keep >> (j / gs)) & 1ull)) b[e] = -INFINITY;
  }

  // 6. topk() of the masked biased scores.
  exact_topk<P>(b, k, lane, s_idx, s_val);
  __syncthreads();

  // 7. Gather the un-biased scores in slot order, sum in slot order,
  // w *= 1 / sum when sum > 0, then w *= routed_scaling_factor.
  float sum = 0.f;
  for (uint32_t s = 0; s < k; ++s) sum += s_sig[s_idx[s]];
  if (lane < (int)k) {
    const int32_t id = s_idx[lane];
    float w = s_sig[id];
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
