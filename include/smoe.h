/*
 * smoe.h — C ABI of libsmoe, the MI355X (gfx950) routed-expert MoE path.
 *
 * This is the drop-in boundary that replaces the reference's Metal
 * kernel crate (crates/streammoe-metal, `Kernels` + `KernelCall`) and the
 * engine's MoE encoders (crates/streammoe/src/riir/moe/expert_forward.rs)
 * for the routed-expert hot path. Each entry point below cites the
 * reference interface it replaces as path:line, relative to the
 * reference repository root. Short prefixes:
 *   metal/lib.rs      = crates/streammoe-metal/src/lib.rs
 *   expert_forward.rs = crates/streammoe/src/riir/moe/expert_forward.rs
 *   gpu_matvec.rs     = crates/streammoe/src/riir/backend/gpu/gpu_matvec.rs
 *   moe_router.rs     = crates/streammoe/src/riir/moe/moe_router.rs
 *   shaders.metal     = crates/streammoe/shaders/shaders.metal
 *
 * Conventions (the reference's contract, restated for a C caller):
 *   - Every pointer named as device memory is a device address on the
 *     handle's GPU (hipMalloc, or any allocator of that device).
 *     Host-memory arguments are marked "host".
 *   - Every compute entry point only ENQUEUES work on the handle's
 *     stream and returns; nothing is allocated on the hot path
 *     (scratch is reserved at smoe_create / smoe_reserve). Call
 *     smoe_sync (or synchronise the stream) before reading results.
 *   - Argument errors return a status code and enqueue nothing (the
 *     reference panics or returns ExpertForwardError / CpuMatvecError;
 *     here nothing panics).
 *   - A handle is not thread-safe (the reference's Ctx is Send + !Sync,
 *     crates/streammoe/src/lib.rs:23-28): one handle per engine context.
 *   - Quantized weights use the MLX affine layout: 4-bit = 8 codes per
 *     little-endian u32, low nibble first; packed 3-bit = 8 codes per
 *     3 bytes, code i at bits 3i..3i+3 of a little-endian 24-bit pack;
 *     bf16 scale and bias per `group` inputs; w = q * scale + bias
 *     (crates/streammoe/src/riir/variants.rs:401-486).
 */
#ifndef SMOE_H
#define SMOE_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define SMOE_MAX_K 16 /* expert_forward.rs:117 (MAX_K) */
/* smoe_abi_version() of a library built from this header; 2: smoe_layer
 * gained router_q / shared_gate_q. */
#define SMOE_ABI_VERSION 2

typedef enum {
  SMOE_OK = 0,
  SMOE_ERR_INVALID_ARG = 1,         /* null pointer / zero dimension / bad enum */
  SMOE_ERR_BAD_K = 2,               /* k outside 1..=SMOE_MAX_K or > n_experts (ExpertForwardError::BadK) */
  SMOE_ERR_IN_DIM_NOT_MULTIPLE = 3, /* in_dim not a multiple of the group (CpuMatvecError::InDimNotMultiple) */
  SMOE_ERR_UNSUPPORTED_BITS = 4,    /* bits not 4 or 3 */
  SMOE_ERR_UNSUPPORTED_GROUP = 5,   /* group not 32, 64 or 128 */
  SMOE_ERR_UNSUPPORTED_SHAPE = 6,   /* a dimension this build has no kernel for */
  SMOE_ERR_MISALIGNED = 7,          /* weight/scale region not aligned (CpuMatvecError::Misaligned) */
  SMOE_ERR_SCRATCH_TOO_SMALL = 8,   /* shapes exceed the reserved scratch; call smoe_reserve */
  SMOE_ERR_WORKSPACE_TOO_SMALL = 9, /* caller workspace smaller than *_workspace_size */
  SMOE_ERR_HIP = 10,                /* a HIP runtime call failed (launch, memset, sync) */
  SMOE_ERR_NO_DEVICE = 11,          /* no gfx950 device at that ordinal */
  SMOE_ERR_DEVICE_TIMEOUT = 12,     /* reserved (a bounded device-side wait expired); no entry point of this build waits */
  SMOE_ERR_IO = 13                  /* a file could not be opened or read, or is too short (ExpertIoError::Io) */
} smoe_status;

/* Handle options (smoe_set_option). */
typedef enum {
  SMOE_OPT_DECODE_PATH = 1,  /* 0 auto (default: three-kernel where it has an
                                instance, else one kernel per phase), 1 one
                                kernel per phase, 3 three-kernel only (2, the
                                former persistent path, is rejected) */
  SMOE_OPT_TRACE_BUFFER = 2, /* device uint64 buffer for in-kernel timestamps, or 0 =
                                off. Three-kernel decode: per layer 3 * 4096 * 8
                                words (kernel, block, point); prefill: 8 words
                                (phase ends of the bucketing kernel). Diagnostics
                                only. */
  SMOE_OPT_PREFILL_GEMM = 3  /* prefill GEMM tiles: 0 auto (default: for 4-bit
                                group-64 experts, gate/up on 32 x 32 MFMA tiles
                                over 128-column units (bf16 x, hidden a
                                multiple of 512) and down on 32 x 32 tiles over
                                256-column units (inter a multiple of 512),
                                units of <= 16 rows on 16 x 16 tiles; else
                                16 x 16 tiles over 64-column units), 1 the
                                16 x 16 tiles always, 2 as 0 with the down
                                GEMM on the 16 x 16 tiles. All give the same
                                results up to fp32 rounding order. */
} smoe_option;

typedef struct smoe_handle smoe_handle;

/* Human-readable text of a status code (static storage). */
const char* smoe_strerror(int status);

/* Version of this ABI: bumped on any signature change. */
uint32_t smoe_abi_version(void);

/* ------------------------------------------------------------------ */
/* Context                                                             */
/* ------------------------------------------------------------------ */

/* Create a handle on GPU `device`, enqueueing on `stream` (a
 * hipStream_t; NULL = the default stream). Reserves the decode scratch
 * for hidden <= 4096, inter <= 2048, n_experts <= 1024 and one token.
 * Replaces Kernels::new (metal/lib.rs:538-665) together with
 * MoeBuffers::new_for (expert_forward.rs:432-528). */
int smoe_create(int device, void* stream, smoe_handle** out);

/* Release the handle and its scratch. */
int smoe_destroy(smoe_handle* h);

/* Change the stream later launches go to (hipStream_t). */
int smoe_set_stream(smoe_handle* h, void* stream);

/* Grow the decode scratch (allocates; never call on a hot path or under
 * graph capture). Shapes above the reservation return
 * SMOE_ERR_SCRATCH_TOO_SMALL from the compute entry points. */
int smoe_reserve(smoe_handle* h, uint32_t max_hidden, uint32_t max_inter, uint32_t max_experts);

/* Block until all work enqueued on the handle's stream has finished, then
 * report (and clear) a routing error found on the device by smoe_moe_prefill.
 * Replaces MetalContext::commit_and_wait_labeled's wait and its
 * command-buffer error check (backend/gpu/metal.rs:343-440). */
int smoe_sync(smoe_handle* h);

/* Set a handle option (smoe_option). No counterpart in the reference: the
 * decode-path choice and the phase trace are testing and tuning knobs. */
int smoe_set_option(smoe_handle* h, int option, int64_t value);

/* ------------------------------------------------------------------ */
/* Quantized weights and dense quantized matvec (qmv)                  */
/* ------------------------------------------------------------------ */

/* One quantized [out_dim, in_dim] matrix inside a device buffer.
 * Mirrors QuantWeights (metal/lib.rs:339-351), plus the weight width. */
typedef struct {
  const void* base;       /* device */
  uint64_t packed_offset; /* byte offset of the codes, 16-byte aligned (4- and 8-bit) / 4-byte (3-bit) */
  uint64_t scales_offset; /* byte offset of bf16 scales [out_dim, in_dim/group], 2-byte aligned */
  uint64_t biases_offset; /* byte offset of bf16 biases, same shape */
  uint32_t group_size;    /* 32, 64 or 128 */
  uint32_t bits;          /* 4; 3 for the packed 3-bit layout; 8 for one byte per
                             input (byte n of u32 word i = input 4i + n, the
                             reference's 8-bit affine layout, cpu_matvec.rs:
                             205-283; smoe_qmv, smoe_qmv_argmax and smoe_qmm,
                             in_dim <= 8192, and the router / shared gate of
                             smoe_layer) */
} smoe_qweights;

/* y[r] = sum_c (q[r,c] * s[r,c/g] + b[r,c/g]) * x[c] for r < out_dim,
 * fp32 accumulation. x: device f32[in_dim]; y: device f32[out_dim].
 * in_dim: a multiple of the group, up to 8192 (as the reference's qmv,
 * which needs in_dim % 32 == 0, gpu_matvec.rs:94-101).
 * Replaces encode_matvec (gpu_matvec.rs:116-159) and its kernel
 * dequant_matvec_4bit_qmv (shaders.metal:366-423); used for the LM head
 * (crates/streammoe/src/riir/io/gpu_lm_head.rs:130-193). */
int smoe_qmv(smoe_handle* h, const smoe_qweights* w, const float* x, float* y, uint32_t out_dim,
             uint32_t in_dim);

/* Greedy argmax of a device f32[n] (16-byte aligned) into a device int32:
 * the reference's scan `best = 0; if v[i] > v[best] then best = i`
 * (first index wins on ties; a NaN never wins, and a NaN at index 0 is
 * never replaced, so the result is 0 then). The LM head's token pick. Two
 * launches: 256 slice blocks, then one block over the partials. */
int smoe_argmax(smoe_handle* h, const float* v, uint32_t n, int32_t* out_index);

/* smoe_qmv and smoe_argmax of its output in one pass (the LM head with
 * the greedy pick, io/gpu_lm_head.rs:130-193): y as smoe_qmv computes it,
 * *out_index = the first index of max(y) as smoe_argmax gives it, from
 * per-wave partials of the matvec itself (y is not read back). Uses the
 * handle's scratch (allocated by smoe_create). */
int smoe_qmv_argmax(smoe_handle* h, const smoe_qweights* w, const float* x, float* y, uint32_t out_dim,
                    uint32_t in_dim, int32_t* out_index);

/* Device workspace bytes smoe_qmm needs (0 for zero sizes). */
uint64_t smoe_qmm_workspace_size(uint32_t in_dim, uint32_t group, uint32_t n_tokens);

/* Dense quantized matmul y[n_tokens, out_dim] = x[n_tokens, in_dim] .
 * dequant(W)[out_dim, in_dim]^T (f32 in and out, row-major), on bf16 MFMA
 * with exact dequant and fp32 accumulation (x split into bf16 hi + lo):
 * the QmmCall / encode_dense_matmul_n_tokens of metal/lib.rs:357-380,
 * 684-734 and gpu_matvec.rs:256-302 (shared expert and projections at
 * N > 1). The GEMM takes bits 4 or 3, group 32/64/128, in_dim a
 * multiple of 256 (<= 16384), out_dim a multiple of 256; weights, scales,
 * biases, x, y 16-byte aligned, biases after the scales; workspace
 * 256-byte aligned. Other shapes with in_dim <= 8192 (a multiple of the
 * group) run smoe_qmv's kernel once per token row (x rows 16-byte
 * aligned; workspace unused). Enqueue-only, allocates nothing. */
int smoe_qmm(smoe_handle* h, const smoe_qweights* w, const float* x, float* y, uint32_t out_dim,
             uint32_t in_dim, uint32_t n_tokens, void* workspace, uint64_t workspace_bytes);

/* Dequantize rows [row0, row0 + n_rows) of `w` into device
 * f32[n_rows, in_dim]: w = fma(q, s, b), one rounding, exactly the value
 * the reference CPU path forms (crates/streammoe/src/riir/backend/cpu/
 * cpu_matvec.rs:164-165; 8-bit rows: cpu_matvec.rs:205-283). Verification
 * and load-time entry point (bits 4, 3 or 8): the decode kernels use the
 * same code-unpacking routine and never materialise w; a prefill block's
 * f32 shared-expert gate is one 8-bit row dequantized here once. */
int smoe_dequant(smoe_handle* h, const smoe_qweights* w, uint32_t in_dim, uint32_t row0,
                 uint32_t n_rows, float* out);

/* ------------------------------------------------------------------ */
/* Router                                                              */
/* ------------------------------------------------------------------ */

/* Per token t < n_tokens: logits = router_w · x[t] (f32 [n_experts,
 * hidden] router, fp32), softmax, running-minimum top-k (slot order =
 * replacement order, ties to the earlier expert), then the guarded
 * renormalisation when `normalize` (norm_topk_prob).
 * x: device f32[n_tokens, hidden]; idx: device int32[n_tokens, k];
 * weights: device f32[n_tokens, k]; logits_out: device
 * f32[n_tokens, n_experts] or NULL.
 * Replaces the router gate matvec (attn/linear_attn_forward.rs:2093)
 * plus moe_router_cpu_with (moe_router.rs:165-181) on the host, or on
 * the GPU moe_softmax_topk + moe_normalize_weights (shaders.metal:
 * 3556-3690, encoded by moe/gpu_moe_router.rs). */
int smoe_router(smoe_handle* h, const float* router_w, const float* x, uint32_t n_tokens,
                uint32_t n_experts, uint32_t hidden, uint32_t k, int normalize, int32_t* idx,
                float* weights, float* logits_out);

/* Softmax + top-k + optional renorm from precomputed logits
 * (device f32[n_tokens, n_experts]). Replaces Op::MoeSoftmaxTopK +
 * Op::MoeNormalizeWeights (backend/mod.rs:473-497; shaders.metal:
 * 3556-3690). */
int smoe_softmax_topk(smoe_handle* h, const float* logits, uint32_t n_tokens, uint32_t n_experts,
                      uint32_t k, int normalize, int32_t* idx, float* weights);

/* Softmax only: probs[t] = softmax(logits[t]) per token t < n_tokens
 * (device f32[n_tokens, n], n <= 1024), softmax() of moe_router.rs:52-72
 * bit for bit: max, e_j = expf(l_j - max) with glibc's expf (the libm
 * function the reference's f32::exp calls on Linux), the e_j summed one
 * after another in index order, 1 / sum, e_j * (1 / sum). The routers
 * above and the decode layers use the same arithmetic wherever the
 * probabilities decide the routing (the exact scan for ambiguous top-k
 * sets) or are returned (routing weights). */
int smoe_softmax(smoe_handle* h, const float* logits, uint32_t n_tokens, uint32_t n, float* probs);

/* The softmax's exponential alone, y[i] = expf(x[i]) for i < n (device
 * f32): glibc's expf bit for bit (moe_router.rs:64, `(*v - max_val)
 * .exp()`), for callers that check the device routing against a host
 * libm. */
int smoe_expf(smoe_handle* h, const float* x, float* y, uint64_t n);

/* Top-k only, on arbitrary scores (no softmax): topk() of
 * moe_router.rs:83-124 per token. values: device f32[n_tokens, k]. */
int smoe_topk(smoe_handle* h, const float* scores, uint32_t n_tokens, uint32_t n, uint32_t k,
              int32_t* idx, float* values);

/* noaux_tc routing (DeepSeek-V3 / Cogito-V2) per token t < n_tokens from
 * the gate logits (device f32[n_tokens, n_experts]) and the per-expert
 * e_score_correction_bias (device f32[n_experts]): s = sigmoid(logit);
 * group score = sum of the two largest (s + bias) of each of the n_group
 * equal groups; the running-minimum top-k of the group scores keeps
 * topk_group groups; the same top-k over (s + bias) of the kept groups
 * gives idx (slot order = replacement order); weights = s[idx] * (1 / sum
 * over the slots, in slot order, when > 0) * routed_scaling_factor.
 * idx: device int32[n_tokens, k]; weights: device f32[n_tokens, k];
 * scores_out: device f32[n_tokens, n_experts] receiving s, or NULL; it may
 * equal logits (the reference leaves the sigmoid scores in place).
 * Errors: n_experts == 0 -> INVALID_ARG (EmptyScores); n_group == 0 or not
 * dividing n_experts, topk_group outside 1..=n_group, k outside
 * 1..=min(n_experts, SMOE_MAX_K) -> BAD_K; n_experts > 1024 or n_group > 64
 * -> UNSUPPORTED_SHAPE.
 * Replaces noaux_tc_router_cpu (moe_router.rs:211-330), which the Cogito-V2
 * MoE paths call on host-copied logits (moe/cogito_moe_gpu.rs:286-300,
 * moe/moe_cpu.rs:129-140). */
int smoe_noaux_tc_topk(smoe_handle* h, const float* logits, const float* correction_bias,
                       uint32_t n_tokens, uint32_t n_experts, uint32_t n_group, uint32_t topk_group,
                       uint32_t k, float routed_scaling_factor, int32_t* idx, float* weights,
                       float* scores_out);

/* ------------------------------------------------------------------ */
/* Decode: K routed experts + shared expert + combine (one token)      */
/* ------------------------------------------------------------------ */

/* Shape of one packed expert blob [gate | up | down], each block
 * [codes | bf16 scales | bf16 biases] (variants.rs:401-486). The decode
 * entry points take hidden <= 8192 and inter <= 2048, both multiples of
 * the group: every variant of the reference (variants.rs:620-1040, from the
 * 256-wide test models to Cogito-V2's 7168 and Qwen3.8-Flash-Next's 2560 x
 * 640). */
typedef struct {
  uint32_t hidden; /* H: gate/up in_dim, down out_dim */
  uint32_t inter;  /* I: gate/up out_dim, down in_dim */
  uint32_t group;  /* quantization group along the input dim */
  uint32_t bits;   /* 4 or 3 */
} smoe_expert_shape;

/* Bytes of one expert blob of `shape` (variants.rs:519-528). */
uint64_t smoe_expert_bytes(const smoe_expert_shape* shape);

/* One routed slot's expert binding: the blob starts at base + offset
 * (device). Mirrors the engine's (&Buffer, u64) expert bindings
 * (attn/linear_attn_forward.rs:2461-2470; io/expert_io.rs:578-592). */
typedef struct {
  const void* base;
  uint64_t offset;
} smoe_binding;

/* hidden_out = h_mid + sum_k weights[k] * FFN_k(input)
 *              (+ sigmoid(shared_gate_score) * shared_out),
 * with FFN_k = down(silu(gate(x)) * up(x)) on the k bound experts.
 * bindings, weights: host arrays of k; input, h_mid, shared_out,
 * hidden_out: device f32[hidden]. shared_out NULL drops the shared term
 * (moe_combine_residual_flat_noshared); a NaN shared_gate_score adds
 * shared_out unscaled (the DeepSeek combine).
 * Replaces encode_experts_mmap_into (expert_forward.rs:927-986) /
 * gpu_batched_experts_encode_mmap (:880-915) and the kernels they encode
 * (dequant_matvec_{4,3}bit_v3_experts, swiglu_fused,
 * moe_combine_residual_flat[_noshared]; shaders.metal:1091-1388). */
int smoe_experts_decode(smoe_handle* h, const smoe_expert_shape* shape,
                        const smoe_binding* bindings, uint32_t k, const float* weights,
                        const float* input, const float* h_mid, const float* shared_out,
                        float shared_gate_score, float* hidden_out);

/* One resident MoE layer: experts at base + e * stride (device), a router
 * [n_experts, hidden] (f32, or 8-bit affine as the reference's A3B
 * mlp.gate.weight, linear_attn_forward.rs:1300-1301), an optional
 * always-on 4-bit shared expert (same hidden and inter as the routed ones)
 * with an optional gate vector [hidden] (f32 or 8-bit affine; its sigmoid
 * scales the shared output; none = unscaled). Exactly one of router_w /
 * router_q is set, at most one of shared_gate / shared_gate_q. The 8-bit
 * forms are smoe_qweights of bits 8 (host structs read during the call,
 * device data; codes 16-byte aligned, hidden a multiple of the group); every
 * weight is fma(q, s, b) as the reference's CPU matvec forms it. */
typedef struct {
  smoe_expert_shape shape;
  const void* experts;       /* device, n_experts * stride bytes */
  uint64_t stride;           /* bytes between experts (>= smoe_expert_bytes) */
  uint32_t n_experts;
  uint32_t k;                /* routed experts per token */
  int32_t normalize;         /* norm_topk_prob */
  const float* router_w;     /* device f32[n_experts, hidden], or NULL (router_q) */
  const void* shared_expert; /* device 4-bit blob, or NULL */
  const float* shared_gate;  /* device f32[hidden], or NULL */
  const smoe_qweights* router_q;      /* 8-bit router [n_experts, hidden], or NULL */
  const smoe_qweights* shared_gate_q; /* 8-bit shared gate [1, hidden], or NULL */
} smoe_layer;

/* Decode one token through one layer with routing on the device:
 * router -> top-k -> routed + shared expert FFN -> combine. For hidden
 * 2048 or 4096, inter 512 or 1024, <= 512 experts this is three kernels (router +
 * shared gate/up; top-k + routed gate/up; down + combine) that allocate
 * nothing and set no memory, so a caller can capture them in a HIP graph;
 * other shapes take one kernel per phase. See SMOE_OPT_DECODE_PATH.
 * input: device f32[hidden] (the post-attention-norm hidden);
 * h_mid: device f32[hidden] (residual); hidden_out: device f32[hidden];
 * idx_out / w_out: device int32[k] / f32[k], or NULL, in the
 * reference's slot order (the running-minimum replacement order).
 * Combine order: the per-phase path adds the routed terms in that slot
 * order, as the reference does (deferred.rs:462-468); the three-kernel
 * path adds them in ascending expert index (the order its top-k set
 * comes in), so its hidden_out can differ from the reference's by a few
 * ULP (same terms, another summation order), never bit-identical by
 * construction. The renormalisation sum runs in the same order as the
 * combine.
 * Replaces finish_post_attention's routing (attn/linear_attn_forward.rs:
 * 2123-2165) + moe_dispatch_per_token (:2382-2710) without the host
 * round trip. */
int smoe_moe_decode_layer(smoe_handle* h, const smoe_layer* layer, const float* input,
                          const float* h_mid, float* hidden_out, int32_t* idx_out, float* w_out);

/* The same over n_layers layers back to back (the decode layer loop,
 * crates/streammoe/src/riir/mod.rs:~4030-4180, MoE blocks only):
 * layer l reads x_l and writes r_{l+1} = r_l + MoE_l(x_l), where
 * x_0 = input, r_0 = residual and, between layers, x_{l+1} =
 * RMSNorm(r_{l+1}) * norm_w[l+1] (bf16 weights, eps) when norm_w is not
 * NULL, else x_{l+1} = r_{l+1}. layers: host array; norm_w: host array
 * of n_layers device bf16[hidden] pointers, or NULL; residual_io:
 * device f32[hidden], updated in place; work: device f32[hidden] input
 * staging (x_l for l > 0). */
int smoe_moe_decode_layers(smoe_handle* h, const smoe_layer* layers, uint32_t n_layers,
                           const void* const* norm_w, float eps, const float* input,
                           float* residual_io, float* work);

/* smoe_moe_decode_layers without a handle and without any allocation, for
 * callers that cannot allocate device memory: code under HIP graph
 * capture, tight serving loops, harnesses that forbid hipMalloc. No
 * counterpart in the reference. Same arguments and results as
 * smoe_moe_decode_layers (bit for bit), on the CURRENT device, enqueued on
 * `stream` (a hipStream_t; NULL = the default stream). The three-kernel
 * shapes only (hidden 2048 or 4096, inter 512 or 1024, <= 512 experts, k <= 16;
 * else SMOE_ERR_UNSUPPORTED_SHAPE). Its intermediates live in a fixed
 * 128 KiB device array that each GPU the library runs on holds until the
 * process ends; layers needing more return SMOE_ERR_SCRATCH_TOO_SMALL. The
 * first call on a device without a handle (smoe_create does it for its
 * device) looks the array's address up once. Calls that overlap on one GPU
 * share the array and race: serialise them (one stream per GPU). */
int smoe_moe_decode_layers_noalloc(void* stream, const smoe_layer* layers, uint32_t n_layers,
                                   const void* const* norm_w, float eps, const float* input,
                                   float* residual_io);

/* Several decode tokens (1..4) through the same layers at once, each as
 * smoe_moe_decode_layers would decode it alone (own routing, experts,
 * combine and chained RMSNorm; bit-identical to that): input, residual_io
 * and work are [n_tokens, hidden] rows (16-byte aligned). Every layer is
 * still three launches: the router and shared-expert rows are read once
 * for all tokens and each token's routed experts run side by side in the
 * same grids. idx_out / w_out (nullable): [n_tokens, k] of the last layer
 * in the reference's slot order. Replaces the T-token pass of
 * decode_multi.rs (moe_dispatch_multi, 445-654). At hidden 4096, 3 or 4
 * tokens take a fourth launch per layer (the router kernel in two
 * halves). Shapes without a three-kernel instance (and
 * SMOE_OPT_DECODE_PATH = 1) decode each token through the per-phase chain
 * in turn, bit-identical to smoe_moe_decode_layers on that token; with
 * SMOE_OPT_DECODE_PATH = 3 they return SMOE_ERR_UNSUPPORTED_SHAPE. */
int smoe_moe_decode_tokens(smoe_handle* h, const smoe_layer* layers, uint32_t n_layers,
                           const void* const* norm_w, float eps, uint32_t n_tokens, const float* input,
                           float* residual_io, float* work, int32_t* idx_out, float* w_out);

/* ------------------------------------------------------------------ */
/* Prefill: many tokens through one layer's routed experts             */
/* ------------------------------------------------------------------ */

/* Device workspace bytes smoe_moe_prefill needs for these sizes. */
uint64_t smoe_moe_prefill_workspace_size(const smoe_expert_shape* shape, uint32_t n_tokens,
                                         uint32_t n_experts, uint32_t k);

/* out_sum[t] = sum_s weights[t,s] * FFN_{idx[t,s]}(x[t]) for t < n_tokens:
 * tokens sorted by expert on the device, grouped gate/up GEMM with
 * exact in-kernel dequant on bf16 MFMA (fp32 accumulate), SwiGLU into
 * fp16 activations (as the reference's gather GEMM casts them; beyond
 * +-65504 they become inf), down GEMM on fp16 MFMA, then a fixed-order
 * per-token combine (ascending expert, no atomics: bit-identical across
 * runs).
 * x: device, bf16 [n_tokens, hidden] when x_is_bf16 else f32;
 * idx: device int32[n_tokens, k]; weights: device f32[n_tokens, k];
 * out_sum: device f32[n_tokens, hidden] (overwritten); workspace:
 * device, >= smoe_moe_prefill_workspace_size bytes, 256-byte aligned.
 * Grouped GEMMs for bits 4 or 3, group 32/64/128, hidden and inter
 * multiples of 256 with hidden >= 1024, <= 512 experts; every other
 * expert shape of the decode entry points (hidden <= 8192, inter <= 2048,
 * multiples of the group) and more experts go one token at a time
 * through the per-phase decode kernels (f32 activations; the combine
 * again in ascending expert order). 1..1024 tokens, 1 <= k <= min(16,
 * n_experts); else SMOE_ERR_UNSUPPORTED_SHAPE / SMOE_ERR_BAD_K. The
 * workspace size covers either path (bf16 x assumed). An expert id out of
 * range or repeated within a token is found on the device: the call
 * returns SMOE_OK and the next smoe_sync returns SMOE_ERR_INVALID_ARG.
 * Enqueue-only, allocates nothing, capturable in a HIP graph.
 * Replaces encode_moe_gather_id_fuse (expert_forward.rs:1874-2042) with
 * MoeIdMap0Call / MoeGatherIdCall / MoeCombineTopkCall (metal/lib.rs:
 * 932-1189), and its CPU oracle moe_permute_fuse_cpu
 * (crates/streammoe/src/riir/moe/moe_cpu.rs:282-339). */
int smoe_moe_prefill(smoe_handle* h, const smoe_expert_shape* shape, const void* experts,
                     uint64_t stride, uint32_t n_experts, const int32_t* idx,
                     const float* weights, const void* x, int x_is_bf16, uint32_t n_tokens,
                     uint32_t k, float* out_sum, void* workspace, uint64_t workspace_bytes);

/* Device workspace bytes smoe_moe_prefill_block needs (0: a shape
 * without grouped-GEMM tiles, which the block entry does not take). */
uint64_t smoe_moe_prefill_block_workspace_size(const smoe_expert_shape* shape, uint32_t n_tokens,
                                               uint32_t n_experts, uint32_t k, int has_shared);

/* The prefill MoE block of one layer (linear_attn_forward.rs:3998-4075):
 * the routed experts as smoe_moe_prefill, an optional shared expert over
 * all n_tokens (4-bit, the routed hidden / inter / group; its gate/up and
 * down run as further work items of the same grouped GEMMs when the routed
 * experts are 4-bit, so its weights are read once per pass, else through
 * the 4-bit GEMM instances of their own), then per token t
 *   hidden_out[t] = (h_mid[t] + moe_sum[t]) + sigmoid(g_t) * shared_out[t]
 * with g_t = shared_gate . x[t] (f32 [hidden]; NULL: the shared term
 * unscaled), or hidden_out[t] = h_mid[t] + moe_sum[t] without a shared
 * expert: moe_combine_residual_n_tokens_cpu / _noshared_ (backend/cpu/
 * mod.rs:657-695, the Metal moe_combine_residual_n_tokens,
 * shaders.metal:3318-3355), added in that order with no fused
 * multiply-add, the sigmoid with glibc's expf (cpu_ops.rs:22-25). The
 * shared expert's SwiGLU and down projection are the reference's
 * MatvecNTokens + SwigluFusedBatched + MatvecNTokens ops in one pass.
 * h_mid, hidden_out: device f32 [n_tokens, hidden] (hidden_out may alias
 * h_mid). Grouped-GEMM shapes only (see smoe_moe_prefill); others return
 * SMOE_ERR_UNSUPPORTED_SHAPE. Enqueue-only, allocates nothing, capturable
 * in a HIP graph. */
int smoe_moe_prefill_block(smoe_handle* h, const smoe_expert_shape* shape, const void* experts,
                           uint64_t stride, uint32_t n_experts, const int32_t* idx, const float* weights,
                           const void* x, int x_is_bf16, uint32_t n_tokens, uint32_t k,
                           const void* shared_expert, const float* shared_gate, const float* h_mid,
                           float* hidden_out, void* workspace, uint64_t workspace_bytes);

/* ------------------------------------------------------------------ */
/* Expert arena loader: packed_experts/layer_NN.bin -> device memory    */
/* ------------------------------------------------------------------ */

typedef struct {
  uint32_t bits;        /* 4 or 3 */
  uint32_t reserved;
  uint64_t expert_size; /* bytes of one expert blob (smoe_expert_bytes) */
  uint64_t stride;      /* bytes between experts in the file (>= expert_size) */
} smoe_file_layout;

/* Layout and expert stride of a layer file file_bytes long that holds
 * n_experts experts of this hidden/inter/group (host only, no handle).
 * declared_size / declared_stride: packed_experts/layout.json's
 * expert_size / expert_stride, or 0 / 0 without one. The declared padded
 * stride wins when it exceeds the size, the size is a known layout and the
 * file is exactly n_experts strides long; else the layout whose n_experts
 * blobs fill the file exactly (4-bit, then packed 3-bit); else 4-bit with
 * stride = its size (the legacy assumption). Replaces layout_and_stride /
 * layout_of_len / ExpertLayout::from_expert_size (io/expert_io.rs:229-267,
 * variants.rs:442-450). */
int smoe_layer_file_layout(uint64_t file_bytes, uint32_t n_experts, uint32_t hidden, uint32_t inter,
                           uint32_t group, uint64_t declared_size, uint64_t declared_stride,
                           smoe_file_layout* out);

/* Copy bytes [offset, offset + bytes) of the file at path (bytes == 0:
 * from offset to the end) into device memory dst of capacity dst_bytes,
 * through two pinned staging buffers (kept by the handle) and async copies
 * on the handle's stream; returns once the data is on the device.
 * *bytes_read (nullable) = bytes copied. Replaces the resident-layer part
 * of ExpertFiles::open + attach_to_device (io/expert_io.rs:300-420): a
 * layer file becomes one device arena, expert e at dst + e * stride.
 * SMOE_ERR_IO: cannot open or read, or the file ends before offset +
 * bytes; SMOE_ERR_INVALID_ARG: null pointers or dst_bytes too small. */
int smoe_load_file(smoe_handle* h, const char* path, uint64_t offset, uint64_t bytes, void* dst,
                   uint64_t dst_bytes, uint64_t* bytes_read);

/* ------------------------------------------------------------------ */
/* Seeded synthetic data (bench and test inputs)                       */
/* ------------------------------------------------------------------ */
/* Replace the synthetic-data helpers of expert_forward.rs:2257-2347 and
 * the xorshift generators of the reference's kernel tests: fills device
 * memory from a counter-based generator, so a given (seed, size) gives
 * the same bytes on any run. */

/* Diagnostic (no reference counterpart): read every byte of the device
 * buffer `buf` once with 128-bit loads across the whole GPU, the measured
 * HBM read peak the decode is compared against. bytes: multiple of 16;
 * sink: device uint32[2048] (per-block XOR of the data read). */
int smoe_stream_read(smoe_handle* h, const void* buf, uint64_t bytes, uint32_t* sink);

/* n_experts blobs at base + e * stride: codes uniform (4-bit: random
 * u32 words; 3-bit: random 24-bit packs), scales bf16(|N(0, scale_sigma)|),
 * biases bf16(N(0, bias_sigma)). */
int smoe_synth_experts(smoe_handle* h, void* base, uint32_t n_experts, uint64_t stride,
                       const smoe_expert_shape* shape, uint64_t seed, float scale_sigma,
                       float bias_sigma);

/* Device f32[n] ~ N(0, sigma). */
int smoe_synth_normal_f32(smoe_handle* h, float* out, uint64_t n, uint64_t seed, float sigma);

/* Device bf16[n] (RNE of N(0, sigma)). */
int smoe_synth_normal_bf16(smoe_handle* h, uint16_t* out, uint64_t n, uint64_t seed, float sigma);

#ifdef __cplusplus
}
#endif
#endif /* SMOE_H */
