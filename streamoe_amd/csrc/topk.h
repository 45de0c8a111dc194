// topk.h — wave-level softmax and top-k of the reference router
// (crates/streammoe/src/riir/moe/moe_router.rs:52-141), shared by the
// decode kernels. One wave holds the n scores, P per lane (lane l owns
// [l*P, l*P + P)).
#pragma once

#include "common.h"
#include "expf_ref.h"

namespace smoe {

// ---------------------------------------------------------------------------
// The reference's softmax (moe_router.rs:52-72) bit for bit: max, then
// e_j = expf(v_j - max) with glibc's expf (expf_ref.h), the sum of the e_j
// in index order (one add after another, as the reference's loop), inv =
// 1 / sum correctly rounded, p_j = e_j * inv. n values held P per lane:
// lane l owns [l*P, l*P + P) (TR = false) or l, l + 64, ... (TR = true).
// Positions >= n become -inf. The max is the wave's fmaxf (it differs from
// the reference's strict-> scan only when a NaN is present, and then every
// probability is NaN in both). The sum runs over sbuf (LDS, >= 64 P
// floats, which also receives the probabilities): every lane adds the same
// broadcast values, so all lanes hold the sum. `tab` is this lane's table
// entry (load_exp_tab). Single-wave blocks only (one barrier).
// ---------------------------------------------------------------------------
struct ExpTabReg {
  uint32_t lo, hi;  // kExpTab[lane & 31]
};

__device__ __forceinline__ ExpTabReg load_exp_tab(int lane) {
  const uint64_t t = kExpTabDev[lane & 31];
  return ExpTabReg{(uint32_t)t, (uint32_t)(t >> 32)};
}

// expf_ref with the table entry taken from lane i (every lane must run it).
__device__ __forceinline__ float wave_expf_ref(float x, ExpTabReg tab) {
  return expf_ref(x, [&](uint32_t i) -> uint64_t {
    const int a = (int)(i << 2);
    const uint32_t lo = (uint32_t)__builtin_amdgcn_ds_bpermute(a, (int)tab.lo);
    const uint32_t hi = (uint32_t)__builtin_amdgcn_ds_bpermute(a, (int)tab.hi);
    return ((uint64_t)hi << 32) | lo;
  });
}

template <int P, bool TR = false>
__device__ __forceinline__ void softmax_ref(float (&v)[P], uint32_t n, int lane, float* sbuf, ExpTabReg tab) {
  float m = -INFINITY;
#pragma unroll
  for (int e = 0; e < P; ++e) m = fmaxf(m, v[e]);
  m = readlane_f(wave_max_last(m), 63);
#pragma unroll
  for (int e = 0; e < P; ++e) {
    const uint32_t j = TR ? (uint32_t)(e * 64 + lane) : (uint32_t)(lane * P + e);
    const float ex = wave_expf_ref(v[e] - m, tab);
    v[e] = j < n ? ex : 0.f;
    sbuf[j] = v[e];
  }
  __syncthreads();
  // Sequential sum in index order; the zeros past n change nothing (the sum
  // of non-negative values is never -0).
  float sum = 0.f;
  const f32x4* s4 = reinterpret_cast<const f32x4*>(sbuf);
  for (uint32_t i = 0; i < (n + 3) / 4; ++i) {
    const f32x4 q = s4[i];
    sum += q.x;
    sum += q.y;
    sum += q.z;
    sum += q.w;
  }
  const float inv = __fdiv_rn(1.0f, sum);
#pragma unroll
  for (int e = 0; e < P; ++e) {
    const uint32_t j = TR ? (uint32_t)(e * 64 + lane) : (uint32_t)(lane * P + e);
    v[e] = j < n ? v[e] * inv : -INFINITY;
  }
  __syncthreads();  // every lane has read sbuf
#pragma unroll
  for (int e = 0; e < P; ++e) sbuf[TR ? e * 64 + lane : lane * P + e] = v[e];
  __syncthreads();
}

// The same softmax with a wave-tree sum and the device expf: within a few
// ulps of softmax_ref, and ~0.8 us shorter (no sequential sum). Used only
// for the combine weights of a decode layer whose top-k set is unambiguous
// and whose caller asked for no idx / weights: those weights enter the
// combine, which is compared within a tolerance, and decide nothing.
template <int P>
__device__ __forceinline__ void wave_softmax_fast(float (&v)[P], uint32_t n, int lane) {
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

// Lane i receives lane i + 1's value (DPP wave_shl:1, one VALU op instead
// of an LDS-crossbar permute); lane 63 keeps its own.
__device__ __forceinline__ uint32_t wave_next_u32(uint32_t v) {
  return (uint32_t)__builtin_amdgcn_update_dpp((int)v, (int)v, 0x130, 0xF, 0xF, false);
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
    const uint64_t kn = ((uint64_t)wave_next_u32((uint32_t)(key >> 32)) << 32) | wave_next_u32((uint32_t)key);
    const int32_t in = (int32_t)wave_next_u32((uint32_t)qidx);
    const float vn = __uint_as_float(wave_next_u32(__float_as_uint(qval)));
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

// exact_topk on values held transposed: v[e] of lane l is element e * 64 + l.
// The same scan and result (the reference's running minimum, slot order =
// replacement order): the 64-index chunks are walked in order, and in each
// one a compare and a ballot over the lanes not yet passed find the next
// element that beats the slot minimum, so an event costs a few scalar
// steps instead of a pass over the lane's P values.
// Returns, in lanes < k, the element index the lane's queue entry holds
// (the slots' contents in queue order), -1 elsewhere; out_idx / out_val may
// be null.
template <int P>
__device__ int32_t exact_topk_t(const float (&v)[P], uint32_t k, int lane, int32_t* out_idx, float* out_val) {
  uint64_t key = lane < (int)k ? (((uint64_t)orderable(-1e30f) << 32) | (uint32_t)lane) : ~0ull;
  int32_t qidx = 0;
  float qval = -1e30f;
  // Queue lanes 1 .. k-1 (k <= 64): where a new entry may be placed.
  const uint64_t qmask = (k >= 64 ? ~0ull : ((1ull << k) - 1)) & ~1ull;
#pragma unroll
  for (int e = 0; e < P; ++e) {
    uint64_t pend = ~0ull;  // lanes of chunk e not yet passed
    for (int guard = 0; guard < 64; ++guard) {
      const float hval = __int_as_float(__builtin_amdgcn_readfirstlane(__float_as_int(qval)));
      const uint64_t hit = __ballot(v[e] > hval) & pend;
      if (hit == 0) break;
      const int first = __builtin_ctzll(hit);
      pend = first == 63 ? 0ull : pend & (~0ull << (first + 1));
      const float pj = readlane_f(v[e], first);
      const uint32_t hslot = (uint32_t)__builtin_amdgcn_readfirstlane((int)(uint32_t)key);
      const uint64_t nkey = ((uint64_t)orderable(pj) << 32) | hslot;
      const int p = __popcll(__ballot(key < nkey) & qmask);  // new position among the k
      const uint64_t kn = ((uint64_t)wave_next_u32((uint32_t)(key >> 32)) << 32) | wave_next_u32((uint32_t)key);
      const int32_t in = (int32_t)wave_next_u32((uint32_t)qidx);
      const float vn = __uint_as_float(wave_next_u32(__float_as_uint(qval)));
      // Lane q < p takes lane q+1's entry, lane p the new one (selects).
      const bool sh = lane < p, at = lane == p;
      key = sh ? kn : (at ? nkey : key);
      qidx = sh ? in : (at ? e * 64 + first : qidx);
      qval = sh ? vn : (at ? pj : qval);
    }
  }
  if (lane < (int)k) {
    const uint32_t slot = (uint32_t)key;
    if (out_idx) out_idx[slot] = qidx;
    if (out_val) out_val[slot] = qval;
  }
  return lane < (int)k ? qidx : -1;
}

// Bitwise OR over the wave, valid in lane 63 (DPP row shifts, then the
// row broadcasts).
__device__ __forceinline__ uint32_t wave_or_last(uint32_t v) {
  v |= (uint32_t)__builtin_amdgcn_update_dpp(0, (int)v, 0x111, 0xF, 0xF, false);
  v |= (uint32_t)__builtin_amdgcn_update_dpp(0, (int)v, 0x112, 0xF, 0xF, false);
  v |= (uint32_t)__builtin_amdgcn_update_dpp(0, (int)v, 0x114, 0xF, 0xF, false);
  v |= (uint32_t)__builtin_amdgcn_update_dpp(0, (int)v, 0x118, 0xF, 0xF, false);
  v |= (uint32_t)__builtin_amdgcn_update_dpp(0, (int)v, 0x142, 0xA, 0xF, false);
  v |= (uint32_t)__builtin_amdgcn_update_dpp(0, (int)v, 0x143, 0xC, 0xF, false);
  return v;
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
// taken from the logits' orderable integer keys with at most k + 1 rounds
// of a wave-wide unsigned max (one DPP op per level; every key equal to
// the round's maximum leaves in that round), and accepted only when
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

// Unsigned max over the whole wave, valid in every lane: a butterfly over
// each 16-lane row (DPP row rotations by 8, 4, 2, 1), then across row
// pairs and wave halves with the gfx950 permlane swaps. No scalar register
// is involved, so a chain of these never waits on the scalar unit.
__device__ __forceinline__ uint32_t wave_umax_all(uint32_t v) {
  v = max(v, dpp_umax_src<0x128>(v));
  v = max(v, dpp_umax_src<0x124>(v));
  v = max(v, dpp_umax_src<0x122>(v));
  v = max(v, dpp_umax_src<0x121>(v));
  const auto r = __builtin_amdgcn_permlane16_swap(v, v, false, false);
  v = max(r[0], r[1]);
  const auto h = __builtin_amdgcn_permlane32_swap(v, v, false, false);
  return max(h[0], h[1]);
}

// The k-th largest key of the logits (key = orderable float, 0 for
// positions >= n) when the top-k set is unambiguous, as described above.
// Rounds take the wave maximum of the lanes' heads and pop every head equal
// to it, so equal keys leave together; kth is the key at which the count of
// taken keys first reaches k, next the key at which it first exceeds k
// (equal exactly when a tie straddles the boundary). Returns false for
// NaN, an infinite maximum, a tie at the boundary or a margin below
// 2^-20; the caller then takes the exact scan.
// KC > 0: k is the compile-time constant KC (the rounds unroll: 15% fewer
// cycles at k = 8 than the loop); KC = 0: k at run time.
template <int P, int KC = 0>
__device__ __forceinline__ bool topk_threshold(const float (&l)[P], uint32_t n, uint32_t k_rt, int lane,
                                               uint32_t (&key)[P], uint32_t& kth_out) {
  const uint32_t k = KC > 0 ? (uint32_t)KC : k_rt;
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
  // Round r: m = wave maximum of the heads; every head equal to m pops.
  // Lane r records m and the running count of popped keys; the boundary
  // rounds are found after the loop, so a round is vector work only.
  uint32_t rec_m = 0, rec_c = 0, cnt = 0;
  constexpr int kRounds = KC > 0 ? KC + 1 : 1;  // unroll factor
#pragma unroll kRounds
  for (uint32_t r = 0; r <= k; ++r) {
    const uint32_t m = wave_umax_all(sk[0]);
    const bool pop = sk[0] == m;
    const uint64_t pm = __ballot(pop);
#pragma unroll
    for (int e = 0; e < P - 1; ++e) sk[e] = pop ? sk[e + 1] : sk[e];
    sk[P - 1] = pop ? 0u : sk[P - 1];
    cnt += (uint32_t)__popcll(pm);
    if ((uint32_t)lane == r) {
      rec_m = m;
      rec_c = cnt;
    }
  }
  // kth: the maximum of the round whose count first reaches k; next: of
  // the round whose count first exceeds k (the same round when a tie
  // straddles the boundary).
  const bool live = (uint32_t)lane <= k;
  const uint64_t reach = __ballot(live && rec_c >= k), over = __ballot(live && rec_c > k);
  if (!reach || !over) return false;
  const uint32_t top = (uint32_t)__builtin_amdgcn_readfirstlane((int)rec_m);
  const uint32_t kth = (uint32_t)__builtin_amdgcn_readlane((int)rec_m, (int)__builtin_ctzll(reach));
  const uint32_t next = (uint32_t)__builtin_amdgcn_readlane((int)rec_m, (int)__builtin_ctzll(over));
  const float fm = from_orderable(top), fk = from_orderable(kth), fn = from_orderable(next);
  if (!(fm < INFINITY) || !(fk > fn)) return false;
  if (!(expf(fk - fm) > expf(fn - fm) * (1.0f + 0x1p-20f))) return false;
  kth_out = kth;
  return true;
}

// The top-k set in ascending index order in set_ids[0..k) (LDS), or false
// (see topk_threshold).
template <int P, int KC = 0>
__device__ bool topk_set_logits(const float (&l)[P], uint32_t n, uint32_t k, int lane,
                                int32_t* set_ids) {
  uint32_t key[P], kth;
  if (!topk_threshold<P, KC>(l, n, k, lane, key, kth)) return false;
  uint32_t at = 0;
#pragma unroll
  for (int e = 0; e < P; ++e) {
    const uint64_t b = __ballot(key[e] >= kth);
    at = __builtin_amdgcn_mbcnt_hi((uint32_t)(b >> 32), __builtin_amdgcn_mbcnt_lo((uint32_t)b, at));
  }
#pragma unroll
  for (int e = 0; e < P; ++e)
    if (key[e] >= kth) set_ids[at++] = (int32_t)(lane * P + e);
  return true;
}

// Element `slot` (0 <= slot < k) of the top-k set in ascending index order,
// in every lane, or false (see topk_threshold). No LDS, no barrier.
template <int P, int KC = 0>
__device__ bool topk_slot_logits(const float (&l)[P], uint32_t n, uint32_t k, uint32_t slot,
                                 int lane, int32_t& id) {
  uint32_t key[P], kth;
  if (!topk_threshold<P, KC>(l, n, k, lane, key, kth)) return false;
  uint32_t rank = 0;  // set members in lower lanes
#pragma unroll
  for (int e = 0; e < P; ++e) {
    const uint64_t b = __ballot(key[e] >= kth);
    rank = __builtin_amdgcn_mbcnt_hi((uint32_t)(b >> 32), __builtin_amdgcn_mbcnt_lo((uint32_t)b, rank));
  }
  int32_t hit = -1;
#pragma unroll
  for (int e = 0; e < P; ++e) {
    const bool in = key[e] >= kth;
    if (in && rank == slot) hit = (int32_t)(lane * P + e);
    rank += in ? 1u : 0u;
  }
  const uint64_t hb = __ballot(hit >= 0);
  id = __builtin_amdgcn_readlane(hit, (int)__builtin_ctzll(hb));
  return true;
}

}  // namespace smoe
