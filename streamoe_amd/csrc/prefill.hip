// prefill.hip — many-token expert path (placeholder until the grouped GEMM lands).
#include "../../include/smoe.h"
#include "kernels.h"

extern "C" {
uint64_t smoe_moe_prefill_workspace_size(const smoe_expert_shape* shape, uint32_t n_tokens,
                                         uint32_t n_experts, uint32_t k) {
  (void)shape; (void)n_tokens; (void)n_experts; (void)k;
  return 0;
}
int smoe_moe_prefill(smoe_handle* h, const smoe_expert_shape* shape, const void* experts,
                     uint64_t stride, uint32_t n_experts, const int32_t* idx,
                     const float* weights, const void* x, int x_is_bf16, uint32_t n_tokens,
                     uint32_t k, float* out_sum, void* workspace, uint64_t workspace_bytes) {
  (void)h; (void)shape; (void)experts; (void)stride; (void)n_experts; (void)idx; (void)weights;
  (void)x; (void)x_is_bf16; (void)n_tokens; (void)k; (void)out_sum; (void)workspace;
  (void)workspace_bytes;
  return SMOE_ERR_UNSUPPORTED_SHAPE;
}
}
