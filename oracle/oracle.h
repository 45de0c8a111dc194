/*
 * oracle.h — CPU restatement of the streamoe routed-expert hot path.
 *
 * TEST INFRASTRUCTURE ONLY. This library is the parity checker and the
 * CPU baseline. Only tests/, __graft_entry__.smoke() and bench.py's
 * cpu_baseline leg may load it; the product path (streamoe_amd/) never
 * links or calls it.
 *
 * Every function restates one function of the reference
 * (/root/reference, Rust) and cites it as path:line. Arithmetic follows
 * Rust semantics exactly: a plain `a * b + c` in Rust is two roundings
 * (Rust never contracts), `x.mul_add(y, z)` is one fused rounding. This
 * file is therefore compiled with -ffp-contract=off and spells every
 * reference `mul_add` as fmaf().
 *
 * Short citation prefixes:
 *   cpu_matvec.rs  = crates/streammoe/src/riir/backend/cpu/cpu_matvec.rs
 *   moe_router.rs  = crates/streammoe/src/riir/moe/moe_router.rs
 *   moe_cpu.rs     = crates/streammoe/src/riir/moe/moe_cpu.rs
 *   deferred.rs    = crates/streammoe/src/riir/moe/deferred.rs
 *   cpu_ops.rs     = crates/streammoe/src/riir/backend/cpu/cpu_ops.rs
 *   cpu_mod.rs     = crates/streammoe/src/riir/backend/cpu/mod.rs
 *   variants.rs    = crates/streammoe/src/riir/variants.rs
 *   lm_head.rs     = crates/streammoe/src/riir/io/lm_head.rs
 *   mlp_cpu.rs     = crates/streammoe/src/riir/moe/mlp_cpu.rs
 */
#ifndef SMOE_ORACLE_H
#define SMOE_ORACLE_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* Status codes (mirror the reference's typed errors as integers). */
enum {
  ORC_OK = 0,
  ORC_ERR_IN_DIM_NOT_MULTIPLE = 1, /* CpuMatvecError::InDimNotMultiple */
  ORC_ERR_BAD_K = 2,               /* MoeRouterError::BadK / ExpertForwardError::BadK */
  ORC_ERR_EMPTY = 3,               /* MoeRouterError::EmptyScores */
  ORC_ERR_BAD_BITS = 4,            /* ExpertLayout has no such width */
  ORC_ERR_BAD_ARG = 5
};

/* ---- bf16 -------------------------------------------------------- */
float orc_bf16_to_f32(uint16_t b);
uint16_t orc_f32_to_bf16(float x);

/* ---- layout ------------------------------------------------------ */
size_t orc_expert_bytes(uint32_t hidden, uint32_t inter, uint32_t bits, uint32_t group);
void orc_expert_offsets(uint32_t hidden, uint32_t inter, uint32_t bits, uint32_t group,
                        uint32_t block, uint64_t out_wsb[3]);

/* ---- dequant / matvec --------------------------------------------- */
void orc_dequant_4bit(const uint32_t* packed, const uint16_t* scales, const uint16_t* biases,
                      uint32_t in_dim, uint32_t out_dim, uint32_t group, float* w_out);
/* 8-bit rows: w = fma(q, s, b), byte n of word i = input 4i + n. */
void orc_dequant_8bit(const uint32_t* packed, const uint16_t* scales, const uint16_t* biases,
                      uint32_t in_dim, uint32_t out_dim, uint32_t group, float* w_out);
int orc_dequant_matvec_4bit_gs(const uint32_t* packed, const uint16_t* scales,
                               const uint16_t* biases, uint32_t in_dim, uint32_t out_dim,
                               uint32_t group, const float* x, float* out, int nthreads);
int orc_lm_head(const uint32_t* packed, const uint16_t* scales, const uint16_t* biases,
                uint32_t hidden, uint32_t vocab, uint32_t group, const float* x, float* out);
/* dequant_matvec_8bit_gs_cpu (cpu_matvec.rs:205-283): one byte per input,
 * byte n of u32 word i = input 4i + n; group a multiple of 4. */
int orc_dequant_matvec_8bit_gs(const uint32_t* packed, const uint16_t* scales,
                               const uint16_t* biases, uint32_t in_dim, uint32_t out_dim,
                               uint32_t group, const float* x, float* out, int nthreads);
void orc_f32_matvec(const float* w, uint32_t in_dim, uint32_t out_dim, const float* x, float* out);
void orc_f32_matvec_mt(const float* w, uint32_t in_dim, uint32_t out_dim, const float* x, float* out,
                       int nthreads);
uint32_t orc_argmax(const float* v, uint32_t n);

/* ---- 3-bit layout ------------------------------------------------- */
void orc_pack_3bit(const uint32_t* words4, size_t nwords, uint8_t* out3);
int orc_q3_expert_to_q4(const uint8_t* blob3, uint32_t hidden, uint32_t inter, uint32_t group,
                        uint8_t* blob4);

/* ---- expert FFN ---------------------------------------------------- */
int orc_expert_swiglu(const uint8_t* blob, uint32_t bits, uint32_t hidden, uint32_t inter,
                      uint32_t group, const float* x, float* out, int nthreads);

/* ---- router -------------------------------------------------------- */
int orc_softmax(float* x, uint32_t n);
int orc_topk(const float* scores, uint32_t n, uint32_t k, int32_t* idx, float* val);
/* orc_softmax over `rows` independent rows of n values, rows in parallel. */
int orc_softmax_rows(float* x, uint32_t rows, uint32_t n, int nthreads);
/* y[i] = expf(x[i]): the host libm's expf, the function moe_router.rs:64 calls. */
int orc_expf_many(const float* x, float* y, uint64_t n, int nthreads);
void orc_normalize_weights(float* w, uint32_t k);
int orc_router(float* scores, uint32_t n, uint32_t k, int normalize, int32_t* idx, float* w);
float orc_sigmoid(float x);
int orc_noaux_tc_router(float* scores, const float* bias, uint32_t n, uint32_t n_group,
                        uint32_t topk_group, uint32_t k, float scale, int32_t* idx, float* w);

/* ---- combine ------------------------------------------------------- */
void orc_combine(const float* expert_out, const float* weights, uint32_t k, const float* h_mid,
                 const float* shared_out, float shared_gate_score, uint32_t dim, float* hidden_out);

/* ---- one decode layer ---------------------------------------------- */
typedef struct {
  uint32_t hidden, inter, n_experts, k, group, bits;
  int normalize;                 /* norm_topk_prob */
  const uint8_t* experts;        /* n_experts * stride bytes */
  uint64_t stride;
  const float* router_w;         /* [n_experts, hidden] f32 */
  const uint8_t* shared_blob;    /* 4-bit expert blob of inter_shared, or NULL */
  uint32_t shared_inter;
  const float* shared_gate_w;    /* [hidden] f32, or NULL = unscaled shared add */
  /* 8-bit affine router and shared gate (the A3B mlp.gate.weight and
   * mlp.shared_expert_gate.weight, linear_attn_forward.rs:1300-1301),
   * used instead of router_w / shared_gate_w when router_q8 / gate_q8 is
   * set: codes [rows, hidden] bytes, bf16 scales and biases [rows,
   * hidden / group8]. */
  const uint8_t* router_q8;
  const uint16_t* router_s8;
  const uint16_t* router_b8;
  const uint8_t* gate_q8;
  const uint16_t* gate_s8;
  const uint16_t* gate_b8;
  uint32_t group8;
} orc_layer;

int orc_moe_decode_layer(const orc_layer* L, const float* x, const float* h_mid,
                         float* hidden_out, int32_t* idx_out, float* w_out, float* logits_out,
                         int nthreads);

/* ---- rms norm -------------------------------------------------------- */
void orc_rms_norm_bf16(const float* x, const uint16_t* w, uint32_t dim, float eps, float* out);

/* ---- prefill --------------------------------------------------------- */
/* moe_combine_residual_n_tokens_cpu (backend/cpu/mod.rs:657-695):     */
/* hidden = (h_mid + moe_sum) + sigmoid(gate[t]) * shared_out, no FMA.  */
void orc_moe_combine_residual_n_tokens(const float* h_mid, const float* moe_sum, const float* shared_out,
                                       const float* shared_gate, float* hidden_out, uint32_t n_tokens,
                                       uint32_t dim);
int orc_build_expert_buckets(const int32_t* idx, const float* w, uint32_t n_tokens, uint32_t k,
                             uint32_t n_experts, int32_t* expert_ids, uint32_t* offsets,
                             int32_t* token_idx, float* weights, uint32_t* n_buckets);
int orc_moe_permute_fuse(const uint8_t* experts, uint64_t stride, uint32_t bits, uint32_t hidden,
                         uint32_t inter, uint32_t group, const float* x /*[n_tokens,H]*/,
                         const int32_t* expert_ids, const uint32_t* offsets, uint32_t n_buckets,
                         const int32_t* token_idx, const float* weights, float* out_sum,
                         int nthreads);

/* ---- test-input generator (xorshift64*) ------------------------------ */
uint64_t orc_xorshift64s(uint64_t state, uint64_t* out, size_t n);

#ifdef __cplusplus
}
#endif
#endif
