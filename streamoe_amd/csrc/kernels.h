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
  uint32_t bits;   // 4, 3, or 8 (one byte per input: smoe_qmv / smoe_qmm only)
  uint32_t group;  // 32, 64, 128
};

// 8-bit affine rows (an 8-bit router or shared-expert gate): input c of row
// r has code q[r * K + c] (byte n of u32 word i: input 4 i + n) and the bf16
// scale / bias s / b[r * (K / group) + c / group]; its weight is
// fma(q, s, b). q null: not used.
struct Q8Rows {
  const uint8_t* q = nullptr;
  const uint16_t* s = nullptr;
  const uint16_t* b = nullptr;
  uint32_t group = 0;  // 32, 64 or 128
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
  float* probs;                // [n_tokens, n] softmax probabilities, or null
};

BlobGeom blob_geom(uint32_t hidden, uint32_t inter, uint32_t group, uint32_t bits);

// y[i] = expf_ref(x[i]) (glibc's expf), i < n.
hipError_t launch_expf(const float* x, float* y, uint64_t n, hipStream_t st);

// One decode layer for the three-kernel path (fused.hip).
struct FusedLayer {
  uint32_t hidden;         // 2048 or 4096
  const float* x_in;       // x given as is, or null: x = RMSNorm(resid) * norm
  const float* resid;      // residual r (when x_in is null)
  const uint16_t* norm;    // bf16 RMSNorm weights, or null: x = r
  float eps;
  uint32_t* xl;            // x as integer limbs for the expert kernel, hidden / 32 chunks
                           // of kXLimbWords dwords (written by the router kernel)
  const float* router;     // f32 [E, hidden]; with an 8-bit router any readable
                           // hidden floats (K_B's table wave loads one row as
                           // a stand-in when there is no gate, and uses none)
  const float* gate;       // f32 [hidden] shared-expert gate, or null (unscaled)
  const uint8_t* experts;  // expert e at experts + e * stride
  uint64_t stride;
  const uint8_t* shared;   // 4-bit shared expert blob, or null
  BlobGeom routed, sgeom;  // routed / shared (4-bit) geometry
  uint32_t E, k, normalize;
  float* logits;           // [E]: router logits (the table wave computes the shared gate score)
  float* act;              // [(k + 1) * inter]: routed slots, shared at slot k
  FfnTable* table;         // route table of this token
  const float* h_mid;      // residual added by the combine
  float* out;              // hidden out (may alias h_mid / resid)
  int32_t* idx_out;        // [k] exact slot order, or null
  float* w_out;            // [k], or null
  uint64_t* trace;         // per-block timestamps of this layer, or null (one token only)
  // Several tokens at once (grid dimension y = token in K_B and K_C; K_A
  // loops over the tokens so each router / shared-expert row is read once).
  // Token t's x_in / resid / h_mid / out rows are at + t * hidden, its
  // logits at + t * lstride, act at + t * astride, limbs at + t * xstride,
  // route table at table + t, idx_out / w_out at + t * k.
  uint32_t n_tokens;
  uint32_t lstride, astride, xstride;
};

constexpr uint32_t kMaxDecodeTokens = 4;  // tokens per multi-token decode call

// Trace layout of the three-kernel path: per layer kFaTraceLayer words;
// kernel q (0 route, 1 gate/up, 2 down), block b at
// [(q * kFaTraceBlocks + b) * 8 + point]. Points: 0 start, 1 routing input
// landed (gate/up: logits; down: expert pointers), 2 top-k set known
// (gate/up), 3 weights landed, 4 arithmetic done, 5 stores acknowledged.
constexpr uint32_t kFaTraceBlocks = 4096;
constexpr uint32_t kFaTracePoints = 8;
constexpr uint64_t kFaTraceLayer = 3ull * kFaTraceBlocks * kFaTracePoints;

// Experts per layer of the three-kernel path: the top-k wave holds 8
// logits per lane, read unguarded from a row of logit_stride(E) floats.
constexpr uint32_t kFaMaxExperts = 512;
inline uint32_t logit_stride(uint32_t E) {
  const uint32_t need = E + 1 > 256 ? (E + 1 > 512 ? E + 1 : 512) : 256;  // >= 64 lanes x P
  return (need + 63) & ~63u;
}
bool fused_supported(uint32_t hidden, uint32_t inter, uint32_t group, uint32_t bits,
                     uint32_t n_experts, uint32_t k);
// K_A (router + shared gate/up), K_B (top-k + routed gate/up), K_C (down +
// combine) on `st`; no allocation, no memset (graph-capturable).
// The 8-bit router and / or shared gate of a three-kernel layer (q null:
// f32): K_A writes the gate's weights as f32 to gate_f32 (hidden floats),
// which the layer's FusedLayer::gate then names.
struct FaQ8 {
  Q8Rows router, gate;
  float* gate_f32 = nullptr;
};
hipError_t launch_fused_layer(const FusedLayer& a, hipStream_t st, const FaQ8& q = FaQ8{});

// Prefill (prefill.hip): limits, arguments and workspace.
constexpr uint32_t kPfMaxTokens = 1024;
constexpr uint32_t kPfMaxExperts = 512;
constexpr uint32_t kPfMaxK = 16;
constexpr uint32_t kPfMaxGroupsK = 128;  // K / group of either GEMM (e.g. 4096 / 32)
constexpr uint32_t kPfMinHidden = 1024;  // the gate/up GEMM's token-id lookahead needs K / 256 >= 3

struct PfArgs {
  BlobGeom g;              // routed expert geometry
  const uint8_t* experts;  // expert e at experts + e * stride
  uint64_t stride;
  uint32_t E, k, n_tokens, max_items;
  const int32_t* idx;      // [n_tokens, k]
  const float* w;          // [n_tokens, k]
  const void* x;           // [n_tokens, hidden], bf16 or f32
  int x_bf16;
  float* out;              // [n_tokens, hidden]
  uint32_t* err;           // device error word (2: invalid routing input)
  // Workspace (prefill_workspace).
  uint32_t* items;         // [max_items, 2]: expert, start | count << 16
  uint32_t* n_items;
  uint32_t* item_tok;      // [max_items, 32]: token of each item row (token 0 past the count)
  uint2* tok_pw;           // [n, k] (entry position, routing weight bits) of each token's
                           // entries in ascending expert order
  float* xsum;             // [n, hidden / group] group sums of each token's x row (as the MFMAs see it)
  float* asum;             // [n*k, inter / group] group sums of the activations
  uint16_t* x_hi;          // [n, hidden] x rows, bf16, MFMA order
  uint16_t* x_lo;          // [n, hidden] low halves (fp32 input only)
  uint16_t* act_hi;        // [n*k, inter] SwiGLU output as fp16, MFMA order (qmm: x as bf16 hi)
  uint16_t* act_lo;        // qmm only: x as bf16 lo (null for the prefill)
  float* down;             // [n*k (+ n), hidden]
  uint64_t* trace;         // k_pf_route timestamps (8 words), or null (diagnostics)
  // The MoE block's tail (linear_attn_forward.rs:3998-4075): an optional
  // shared expert over all n tokens (its entries at positions n*k + t),
  // its pre-sigmoid gate scores gate . x_t, and the residual h_mid.
  const uint8_t* shared;   // shared expert blob (4-bit, routed hidden/inter/group), or null
  BlobGeom sg;             // its geometry
  int shared_in_list;      // 1: its items ride in the routed work list (routed bits 4);
                           // 0: a list of their own (sitems, ...) and 4-bit GEMM launches
  const float* gate;       // [hidden] shared-expert gate vector, or null (unscaled)
  const float* h_mid;      // [n_tokens, hidden] residual, or null (out = the routed sum)
  float* gscore;           // [n] gate . x_t
  uint32_t* xr;            // [9] per-XCD ranges of the work list (null: even split)
  uint32_t* sitems;        // shared-only work list (shared_in_list == 0): items, count, token rows, ranges
  uint32_t* sn_items;
  uint32_t* sitem_tok;
  uint32_t* sxr;
  int gemm_path;           // 0: the 32 x 32 gate/up and down tiles where they apply, 1: k_pf_mm only, 2: down on k_pf_mm
};

// Workspace bytes for these sizes; with `a` and `base`, also points a's
// workspace fields into base.
uint64_t prefill_workspace(uint32_t hidden, uint32_t inter, uint32_t group, uint32_t n_tokens,
                           uint32_t n_experts, uint32_t k, bool shared, PfArgs* a, uint8_t* base);
// Prefill through the per-phase decode kernels, one token at a time, for
// the shapes prefill_supported refuses (decode.hip): workspace bytes and
// launch.
uint64_t prefill_tokens_workspace(uint32_t hidden, uint32_t inter, uint32_t n_tokens, uint32_t k, bool x_bf16);
hipError_t launch_prefill_tokens(const BlobGeom& g, const uint8_t* experts, uint64_t stride, uint32_t E,
                                 const int32_t* idx, const float* w, const void* x, bool x_bf16, uint32_t n,
                                 uint32_t k, float* out, uint8_t* ws, uint32_t* err, hipStream_t st,
                                 bool* unsupported);
bool prefill_supported(uint32_t hidden, uint32_t inter, uint32_t group, uint32_t bits,
                       uint32_t n_tokens, uint32_t n_experts, uint32_t k);
hipError_t launch_prefill(const PfArgs& a, uint32_t n_cu, hipStream_t st);

// Dense quantized GEMM on the prefill GEMM (prefill.hip): workspace, limits
// (in_dim multiple of 256 and <= 16384 / 128 groups, out_dim multiple of
// 256) and launch. PfArgs fields used: g (hidden = out_dim, inter = in_dim,
// w/s/b[2] = the weight offsets from `experts`), experts, stride = 0,
// n_tokens, the workspace fields of qmm_workspace, and down = y.
uint64_t qmm_workspace(uint32_t in_dim, uint32_t group, uint32_t n_tokens, PfArgs* a, uint8_t* base);
bool qmm_supported(uint32_t in_dim, uint32_t out_dim, uint32_t group, uint32_t bits, uint32_t n_tokens);
hipError_t launch_qmm(const PfArgs& a, const float* x, uint32_t n_cu, hipStream_t st);

// All launchers return hipSuccess or the launch error; `*unsupported`
// is set when no kernel instance exists for the shape.
// With arg_out, also the argmax of y (first index on ties): per-wave
// partials in arg_v / arg_i (kQmvMaxWaves entries) and one merge launch.
constexpr uint32_t kQmvMaxWaves = 3072;
hipError_t launch_qmv(const QView& w, const float* x, float* y, uint32_t out_dim, uint32_t in_dim,
                      hipStream_t st, bool* unsupported, float* arg_v = nullptr, uint32_t* arg_i = nullptr,
                      int32_t* arg_out = nullptr);
hipError_t launch_dequant(const QView& w, uint32_t in_dim, uint32_t row0, uint32_t n_rows,
                          float* out, hipStream_t st);
// Argmax (first index on ties); part_v / part_i: 256-entry scratch.
hipError_t launch_argmax(const float* v, uint32_t n, int32_t* out, float* part_v, uint32_t* part_i,
                         hipStream_t st);

// logits[t, e] = W[e] . x[t] for e < n_experts; gate_scores[t] =
// gate_w . x[t] when gate_w is not null. Wq / gq (when their q is set):
// 8-bit rows in place of W / gate_w.
// With norm_w, x is the residual: the kernel applies the bf16-weighted
// RMSNorm itself and writes the normalised rows to x_out.
hipError_t launch_router_logits(const float* W, const float* gate_w, const float* x,
                                uint32_t n_tokens, uint32_t n_experts, uint32_t hidden,
                                float* logits, float* gate_scores, hipStream_t st,
                                const uint16_t* norm_w = nullptr, float eps = 0.f, float* x_out = nullptr,
                                const Q8Rows& Wq = Q8Rows{}, const Q8Rows& gq = Q8Rows{});
// Softmax (optional) + running-min top-k + optional renorm, one wave per token.
hipError_t launch_topk(const float* scores, uint32_t n_tokens, uint32_t n, uint32_t k,
                       bool softmax, bool normalize, const RouteOut& out, hipStream_t st);
// noaux_tc routing from logits [n_tokens, n] (router.hip). scores_out may
// equal logits (each lane reads its scores before writing them) or be null.
constexpr uint32_t kNoauxMaxExperts = 1024, kNoauxMaxGroups = 64;
hipError_t launch_noaux_topk(const float* logits, const float* bias, uint32_t n_tokens, uint32_t n,
                             uint32_t n_group, uint32_t topk_group, uint32_t k, float scale,
                             float* scores_out, const RouteOut& out, hipStream_t st);

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
// Streaming-read diagnostic over `bytes` (multiple of 16) with
// kStreamBlocks blocks; sink: kStreamBlocks u32.
constexpr uint32_t kStreamBlocks = 2048;
hipError_t launch_stream_read(const void* buf, uint64_t bytes, uint32_t* sink, hipStream_t st);

// Synthetic data.
hipError_t launch_synth_experts(uint8_t* base, uint32_t n_experts, uint64_t stride,
                                const BlobGeom& g, uint64_t seed, float ssig, float bsig,
                                hipStream_t st);
hipError_t launch_synth_normal_f32(float* out, uint64_t n, uint64_t seed, float sigma,
                                   hipStream_t st);
hipError_t launch_synth_normal_bf16(uint16_t* out, uint64_t n, uint64_t seed, float sigma,
                                    hipStream_t st);

}  // namespace smoe
