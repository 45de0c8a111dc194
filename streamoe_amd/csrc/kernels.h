// kernels.h — host-side interface between the C ABI (api.hip) and the
// kernel translation units. Plain structs shared by host and device.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

namespace smoe {

constexpr int kMaxKHost = 16;
constexpr int kMaxSlotsHost = kMaxKHost + 1;

// One quantized [rows, in_dim] matrix.
struct QView {
  const uint8_t* codes;
  const uint16_t* scales;
  const uint16_t* biases;
  uint32_t bits;   // 4 or 3
  uint32_t group;  // 32, 64, 128
};

// Byte geometry of one expert blob [gate | up | down], each block
// [codes | bf16 scales | bf16 biases] (variants.rs:401-486).
struct BlobGeom {
  uint32_t bits;
  uint32_t hidden, inter, group;
  uint64_t w[3], s[3], b[3];  // offsets of codes / scales / biases per block
};

// What the expert FFN kernels read per decode token: the blob of every
// slot (routed slots 0..k-1, then the shared expert at slot k), the
// routing weights and the shared expert's pre-sigmoid gate score.
struct FfnTable {
  const uint8_t* blob[kMaxSlotsHost];
  float weight[kMaxSlotsHost];
  float shared_gate;  // NaN: add the shared output unscaled
  uint32_t k;
  uint32_t has_shared;
};

// Routing destination for the top-k kernel in layer mode.
struct RouteOut {
  int32_t* idx;            // [n_tokens, k] or null
  float* weight;           // [n_tokens, k] or null
  FfnTable* table;         // device table (token 0) or null
  const uint8_t* experts;  // layer arena
  uint64_t stride;
  const uint8_t* shared_blob;  // null: no shared expert
  const float* gate_scores;    // [n_tokens] pre-sigmoid shared gate, or null (unscaled)
};

BlobGeom blob_geom(uint32_t hidden, uint32_t inter, uint32_t group, uint32_t bits);

// All launchers return hipSuccess or the launch error; `*unsupported`
// is set when no kernel instance exists for the shape.
hipError_t launch_qmv(const QView& w, const float* x, float* y, uint32_t out_dim, uint32_t in_dim,
                      hipStream_t st, bool* unsupported);
hipError_t launch_dequant(const QView& w, uint32_t in_dim, uint32_t row0, uint32_t n_rows,
                          float* out, hipStream_t st);
hipError_t launch_argmax(const float* v, uint32_t n, int32_t* out, hipStream_t st);

// logits[t, e] = W[e] . x[t] for e < n_experts; gate_scores[t] =
// gate_w . x[t] when gate_w is not null.
hipError_t launch_router_logits(const float* W, const float* gate_w, const float* x,
                                uint32_t n_tokens, uint32_t n_experts, uint32_t hidden,
                                float* logits, float* gate_scores, hipStream_t st);
// Softmax (optional) + running-min top-k + optional renorm, one wave per token.
hipError_t launch_topk(const float* scores, uint32_t n_tokens, uint32_t n, uint32_t k,
                       bool softmax, bool normalize, const RouteOut& out, hipStream_t st);

// Expert FFN of every slot in the table: act[slot, r] = silu(gate) * up.
// Exactly one of tab_dev / tab_val is used (tab_dev when not null).
hipError_t launch_gateup(const BlobGeom& routed, const BlobGeom& shared, const FfnTable* tab_dev,
                         const FfnTable& tab_val, uint32_t n_slots, const float* x, float* act,
                         hipStream_t st, bool* unsupported);
// hidden_out = h_mid + sum_k w_k down_k(act_k) (+ shared term).
hipError_t launch_down_combine(const BlobGeom& routed, const BlobGeom& shared,
                               const FfnTable* tab_dev, const FfnTable& tab_val, uint32_t n_slots,
                               const float* act, const float* h_mid, const float* shared_out,
                               float* hidden_out, hipStream_t st, bool* unsupported);
// x_out = RMSNorm(r) * w (bf16), or a copy of r when w is null.
hipError_t launch_rmsnorm(const float* r, const uint16_t* w, float eps, uint32_t dim, float* x_out,
                          hipStream_t st);

// Synthetic data.
hipError_t launch_synth_experts(uint8_t* base, uint32_t n_experts, uint64_t stride,
                                const BlobGeom& g, uint64_t seed, float ssig, float bsig,
                                hipStream_t st);
hipError_t launch_synth_normal_f32(float* out, uint64_t n, uint64_t seed, float sigma,
                                   hipStream_t st);
hipError_t launch_synth_normal_bf16(uint16_t* out, uint64_t n, uint64_t seed, float sigma,
                                    hipStream_t st);

}  // namespace smoe
