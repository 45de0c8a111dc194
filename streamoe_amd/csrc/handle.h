// handle.h — the libsmoe handle (internal; the C ABI sees an opaque
// pointer): device, stream, reserved decode scratch, options, and the file
// loader's staging buffers.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include "../../include/smoe.h"
#include "kernels.h"

struct smoe_handle {
  int device = 0;
  hipStream_t stream = nullptr;
  // Decode scratch (MoeBuffers' flat buffers, expert_forward.rs:379-528).
  void* mem = nullptr;
  float* act = nullptr;       // [kMaxSlots, max_inter]
  float* logits = nullptr;    // [max_experts + 1]
  float* gate = nullptr;      // [1] shared-expert gate score
  smoe::FfnTable* table = nullptr;  // routing table of the current token
  uint32_t* xl = nullptr;     // [max_hidden / 32 * kXLimbWords] x as integer limbs
  float* arg_v = nullptr;     // [kQmvMaxWaves] argmax partial values
  uint32_t* arg_i = nullptr;  // [kQmvMaxWaves] argmax partial indices
  uint32_t* err = nullptr;        // device error word (prefill routing errors)
  float* gate_row = nullptr;  // [max_hidden] f32 weights of an 8-bit shared gate (three-kernel decode)
  uint32_t max_hidden = 0, max_inter = 0, max_experts = 0;
  // Per-token strides (elements) of logits, act and limbs in the scratch.
  uint32_t lstride = 0, astride = 0, xstride = 0;
  // Options.
  int decode_path = 0;  // 0 auto, 1 per-phase kernels, 3 three-kernel
  uint64_t* trace = nullptr;
  int prefill_gemm = 0;  // SMOE_OPT_PREFILL_GEMM: 0 the 32 x 32 tiles where they apply, 1 k_pf_mm only, 2 down on k_pf_mm
  // File loader: two pinned host staging buffers (allocated on first use,
  // freed by smoe_destroy) and the events that say when a copy out of
  // each has finished.
  void* stage[2] = {nullptr, nullptr};
  hipEvent_t stage_done[2] = {nullptr, nullptr};
  uint64_t stage_bytes = 0;
};

// Frees the loader's staging buffers and events (loader.hip).
void release_staging(smoe_handle* h);
