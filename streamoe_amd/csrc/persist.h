// persist.h — arguments of the persistent multi-layer decode kernel.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include "kernels.h"

namespace smoe {

constexpr int kMaxPLayers = 48;

struct PLayer {
  const uint8_t* experts;  // layer arena: n_experts * stride
  const float* router;     // [E, H] f32
  const uint8_t* shared;   // shared expert blob (4-bit) or null
  const float* gate;       // shared-expert gate vector [H] or null
  const uint16_t* norm;    // bf16 RMSNorm weights for this layer's input, or null (layers > 0)
  uint64_t stride;
};

struct PArgs {
  PLayer L[kMaxPLayers];
  BlobGeom geom_routed, geom_shared;
  uint32_t n_layers, E, k, group;
  uint32_t normalize, has_shared, has_gate;
  float eps;
  const float* input;     // x_0
  const float* resid_in;  // r_0
  float* out;             // r_n
  int32_t* idx_out;       // [n_layers, k] or null
  float* w_out;           // [n_layers, k] or null
  uint64_t* tag_resid;    // [H]
  uint64_t* tag_logit;    // [E + 1]
  uint64_t* tag_act;      // [(k + 1) * I]
  uint32_t epoch;         // epoch of layer 0 (never 0)
  uint32_t* err;          // device error word
  uint64_t* trace;        // optional per-phase timestamps, or null
};

struct PPlan {
  uint32_t nb;       // worker blocks
  uint32_t grid;     // nb, plus the coordinator block when idx/w are requested
  uint32_t nw;       // waves per block
  uint32_t variant;  // kernel instance
};

bool persist_plan(uint32_t hidden, uint32_t inter, uint32_t n_experts, uint32_t k, uint32_t bits,
                  bool shared, bool coordinator, PPlan* plan);
hipError_t launch_decode_persistent(const PArgs& a, const PPlan& plan, uint32_t bits,
                                    hipStream_t st);

}  // namespace smoe
