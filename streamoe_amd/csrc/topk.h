// topk.h — wave-level softmax and top-k of the reference router
// (crates/streammoe/src/riir/moe/moe_router.rs:52-141), shared by the
// decode kernels. One wave holds the n scores, P per lane (lane l owns
// [l*P, l*P + P)).
#pragma once

#include "common.h"

namespace smoe {

// ---------------------------------------------------------------------------
// Softmax over n values held P per lane (lane l owns [l*P, l*P + P)), as the
// reference: max, exp(v - max), sum, * (1 / sum). Invalid entries -> -inf.
// ---------------------------------------------------------------------------
template <int P>
__device__ __forceinline__ void wave_softmax(float (&v)[P], uint32_t n, int lane) {
  float m = -INFINITY;
#pragma unroll
  for (int e = 0; e < P; ++e) m = fmaxf(m, v[e]);
  m = readlane_f(wave_max_last(m), 63);
  float sum = 0.f;
#pragma unroll
  for (int e = 0; e < P; ++e) {
    const uint32_t j = lane * P + e;
    v[e] = j < n ? expf(v[e] - m) : 0.f;
    sum += v[e];
  }
  sum = readlane_f(group_sum_last<64>(sum), 63);
  const float inv = 1.0f / sum;
#pragma unroll
  for (int e = 0; e < P; ++e) {
    const uint32_t j = lane * P + e;
    v[e] = j < n ? v[e] * inv : -INFINITY;
  }
}

// Exact running-minimum top-k of the reference (moe_router.rs:83-124) on
// the values held P per lane. Slots live in lanes 0..k-1 as a queue sorted
// by (value, slot): the head is the slot the next winner replaces. Returns
// in lanes s < k: slot s's index and value.
__device__ __forceinline__ uint32_t orderable(float f) {
  const uint32_t u = __float_as_uint(f);
  return (u & 0x80000000u) ? ~u : (u | 0x80000000u);
}

template <int P>
__device__ void exact_topk(const float (&v)[P], uint32_t k, int lane, int32_t* out_idx,
                           float* out_val) {
  // Queue entry per lane q < k: key (orderable value, slot), element index.
  uint64_t key = lane < (int)k ? (((uint64_t)orderable(-1e30f) << 32) | (uint32_t)lane) : ~0ull;
  int32_t qidx = 0;
  float qval = -1e30f;
  int32_t pos = -1;
  for (uint32_t guard = 0; guard <= 64u * P; ++guard) {
    // Head = lane 0 (smallest key).
    const float hval = __int_as_float(__builtin_amdgcn_readfirstlane(__float_as_int(qval)));
    const uint32_t hslot = (uint32_t)__builtin_amdgcn_readfirstlane((int)(uint32_t)key);
    // Next index > pos whose value beats the head.
    int32_t cand = 0x7FFFFFFF;
#pragma unroll
    for (int e = P - 1; e >= 0; --e) {
      const int32_t j = lane * P + e;
      if (j > pos && v[e] > hval) cand = j;
    }
    const uint64_t ball = __ballot(cand != 0x7FFFFFFF);
    if (ball == 0) break;
    const int first = __ffsll((unsigned long long)ball) - 1;
    const int32_t j = __builtin_amdgcn_readlane(cand, first);
    float pj = 0.f;
#pragma unroll
    for (int e = 0; e < P; ++e)
      if (lane * P + e == j) pj = v[e];
    pj = readlane_f(pj, first);
    // Remove the head and insert (pj, hslot) in order among lanes 1..k-1.
    const uint64_t nkey = ((uint64_t)orderable(pj) << 32) | hslot;
    const bool less = lane >= 1 && lane < (int)k && key < nkey;
    const int p = __popcll(__ballot(less));  // new position among the k
    // Lane q < p takes lane q+1's entry; lane p takes the new one.
    const uint64_t kn = __shfl_down(key, 1, 64);
    const int32_t in = __shfl_down(qidx, 1, 64);
    const float vn = __shfl_down(qval, 1, 64);
    if (lane < p) {
      key = kn;
      qidx = in;
      qval = vn;
    } else if (lane == p) {
      key = nkey;
      qidx = j;
      qval = pj;
    }
    pos = j;
  }
  // Scatter back to slot order: the entry in queue lane q belongs to slot
  // (key & 0xFFFFFFFF).
  if (lane < (int)k) {
    const uint32_t slot = (uint32_t)key;
    out_idx[slot] = qidx;
    out_val[slot] = qval;
  }
}

// Top-k SET: the k largest values (ascending index order in set_ids) when
// the k-th and (k+1)-th largest differ, no value is NaN and the k-th is
// above the -1e30 start value of the reference's slots. Otherwise returns
// false and the caller falls back to exact_topk.
template <int P>
__device__ bool topk_set(const float (&v)[P], uint32_t n, uint32_t k, int lane,
                         int32_t* set_ids) {
  // Each lane sorts its P values descending (stable: lower index first).
  float sv[P];
  int32_t si[P];
#pragma unroll
  for (int e = 0; e < P; ++e) {
    sv[e] = v[e];
    si[e] = lane * P + e;
  }
  bool nan = false;
#pragma unroll
  for (int e = 0; e < P; ++e) nan |= (sv[e] != sv[e]);
  if (__ballot(nan)) return false;
#pragma unroll
  for (int a = 0; a < P; ++a)
#pragma unroll
    for (int b = P - 1; b > a; --b)
      if (sv[b] > sv[b - 1]) {
        const float tv = sv[b];
        sv[b] = sv[b - 1];
        sv[b - 1] = tv;
        const int32_t ti = si[b];
        si[b] = si[b - 1];
        si[b - 1] = ti;
      }
  float kth = 0.f, next = -INFINITY;
  int taken = 0;  // how many of this lane's sorted values are taken
  for (uint32_t r = 0; r <= k; ++r) {
    const float head = taken < P ? sv[0] : -INFINITY;
    const float m = readlane_f(wave_max_last(head), 63);
    if (r == k) {
      next = m;
      break;
    }
    kth = m;
    const uint64_t ball = __ballot(taken < P && head == m);
    const int first = __ffsll((unsigned long long)ball) - 1;
    if (lane == first) {
#pragma unroll
      for (int e = 0; e < P - 1; ++e) {
        sv[e] = sv[e + 1];
        si[e] = si[e + 1];
      }
      sv[P - 1] = -INFINITY;
      ++taken;
    }
  }
  if (!(kth > next) || !(kth > -1e30f)) return false;
  // Set = { j : v_j >= kth } (exactly k elements). Compact in index order.
  int cnt = 0;
#pragma unroll
  for (int e = 0; e < P; ++e) cnt += ((uint32_t)(lane * P + e) < n && v[e] >= kth) ? 1 : 0;
  // Exclusive prefix of cnt over lanes.
  int incl = cnt;
#pragma unroll
  for (int o = 1; o < 64; o <<= 1) {
    const int t = __shfl_up(incl, o, 64);
    if (lane >= o) incl += t;
  }
  int at = incl - cnt;
#pragma unroll
  for (int e = 0; e < P; ++e) {
    const uint32_t j = lane * P + e;
    if (j < n && v[e] >= kth) set_ids[at++] = (int32_t)j;
  }
  return true;
}


// ---------------------------------------------------------------------------
// Top-k SET straight from the logits, for the routed expert kernels.
//
// Softmax is monotone, so the k largest probabilities are the k largest
// logits whenever the reference's running-minimum scan cannot see a tie
// at the boundary. The scan keeps exactly the k largest probabilities when
// the k-th is strictly above the (k+1)-th (moe_router.rs:83-124). With
// e = exp(l - max), every probability is e * (1 / sum) rounded once, and a
// positive common factor with one rounding preserves a strict order when
// the two e values are more than 2^-20 apart relatively. So the set is
// taken from the logits' orderable integer keys with k + 1 rounds of a
// wave-wide unsigned max (one DPP op per level), and accepted only when
// exp(l_k - max) > exp(l_{k+1} - max) * (1 + 2^-20); ties, NaN or an
// infinite max return false and the caller takes the exact scan. Returns
// the set in ascending index order in set_ids[0..k).
// ---------------------------------------------------------------------------
template <int CTRL, int ROW_MASK = 0xF>
__device__ __forceinline__ uint32_t dpp_umax_src(uint32_t v) {
  return (uint32_t)__builtin_amdgcn_update_dpp(0, (int)v, CTRL, ROW_MASK, 0xF, true);
}

// Unsigned max over the wave, valid in lane 63.
__device__ __forceinline__ uint32_t wave_umax_last(uint32_t v) {
  v = max(v, dpp_umax_src<0x111>(v));
  v = max(v, dpp_umax_src<0x112>(v));
  v = max(v, dpp_umax_src<0x114>(v));
  v = max(v, dpp_umax_src<0x118>(v));
  v = max(v, dpp_umax_src<0x142, 0xA>(v));
  v = max(v, dpp_umax_src<0x143, 0xC>(v));
  return v;
}

__device__ __forceinline__ float from_orderable(uint32_t k) {
  return __uint_as_float((k & 0x80000000u) ? (k & 0x7FFFFFFFu) : ~k);
}

template <int P>
__device__ bool topk_set_logits(const float (&l)[P], uint32_t n, uint32_t k, int lane,
                                int32_t* set_ids) {
  uint32_t key[P];
  bool bad = false;
#pragma unroll
  for (int e = 0; e < P; ++e) {
    const uint32_t j = lane * P + e;
    bad |= (l[e] != l[e]);
    key[e] = j < n ? orderable(l[e]) : 0u;
  }
  if (__ballot(bad)) return false;
  uint32_t sk[P];
#pragma unroll
  for (int e = 0; e < P; ++e) sk[e] = key[e];
#pragma unroll
  for (int a = 0; a < P; ++a)
#pragma unroll
    for (int b = P - 1; b > a; --b) {
      const uint32_t hi = max(sk[b - 1], sk[b]), lo = min(sk[b - 1], sk[b]);
      sk[b - 1] = hi;
      sk[b] = lo;
    }
  uint32_t top = 0, kth = 0, next = 0;
  for (uint32_t r = 0; r <= k; ++r) {
    const uint32_t m = (uint32_t)__builtin_amdgcn_readlane((int)wave_umax_last(sk[0]), 63);
    if (r == 0) top = m;
    if (r == k) {
      next = m;
      break;
    }
    kth = m;
    const uint64_t ball = __ballot(sk[0] == m);
    const int first = __builtin_amdgcn_readfirstlane(__ffsll((unsigned long long)ball) - 1);
    if (lane == first) {
#pragma unroll
      for (int e = 0; e < P - 1; ++e) sk[e] = sk[e + 1];
      sk[P - 1] = 0;
    }
  }
  const float fm = from_orderable(top), fk = from_orderable(kth), fn = from_orderable(next);
  if (!(fm < INFINITY) || !(fk > fn)) return false;
  if (!(expf(fk - fm) > expf(fn - fm) * (1.0f + 0x1p-20f))) return false;
  const uint64_t below = lane == 0 ? 0ull : (~0ull >> (64 - lane));
  uint32_t at = 0;
#pragma unroll
  for (int e = 0; e < P; ++e) at += __popcll(__ballot(key[e] >= kth) & below);
#pragma unroll
  for (int e = 0; e < P; ++e)
    if (key[e] >= kth) set_ids[at++] = (int32_t)(lane * P + e);
  return true;
}

}  // namespace smoe
