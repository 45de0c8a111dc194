// synth.hip — seeded synthetic inputs, generated on the device.
//
// A counter-based generator (splitmix64 of seed and element index) makes
// every element independent of the launch shape, so a (seed, size) pair
// always gives the same bytes. Normals come from Box-Muller on two
// 32-bit uniforms.
#include "common.h"
#include "kernels.h"

namespace smoe {

__device__ __forceinline__ uint64_t splitmix64(uint64_t z) {
  z += 0x9E3779B97F4A7C15ull;
  z = (z ^ (z >> 30)) * 0xBF58476D1CE4E5B9ull;
  z = (z ^ (z >> 27)) * 0x94D049BB133111EBull;
  return z ^ (z >> 31);
}

__device__ __forceinline__ uint64_t rand64(uint64_t seed, uint64_t i) {
  return splitmix64(seed * 0xD1B54A32D192ED03ull + splitmix64(i));
}

__device__ __forceinline__ float normal01(uint64_t seed, uint64_t i) {
  const uint64_t r = rand64(seed, i);
  // u1 in (0, 1], u2 in [0, 1).
  const float u1 = ((float)(uint32_t)(r >> 40) + 1.0f) * (1.0f / 16777216.0f);
  const float u2 = (float)((uint32_t)r >> 8) * (1.0f / 16777216.0f);
  return sqrtf(-2.0f * logf(u1)) * cospif(2.0f * u2);
}

__device__ __forceinline__ uint16_t to_bf16_rne(float x) {
  const uint32_t b = __float_as_uint(x);
  return (uint16_t)((b + (((b >> 16) & 1u) + 0x7fffu)) >> 16);
}

// Region ids inside one expert: block * 4 + {0: codes, 1: scales, 2: biases}.
__global__ void k_synth_experts(uint8_t* __restrict__ base, uint32_t n_experts, uint64_t stride,
                                BlobGeom g, uint64_t seed, float ssig, float bsig) {
  const uint64_t wb = g.s[0] - g.w[0];  // code bytes per block
  const uint64_t sb = g.b[0] - g.s[0];  // scale bytes per block
  const uint64_t words = wb / 4, halves = sb / 2;
  const uint64_t per_block = words + 2 * halves;
  const uint64_t per_expert = 3 * per_block;
  const uint64_t total = per_expert * n_experts;
  for (uint64_t t = (uint64_t)blockIdx.x * blockDim.x + threadIdx.x; t < total;
       t += (uint64_t)gridDim.x * blockDim.x) {
    const uint64_t e = t / per_expert, r = t % per_expert;
    const uint32_t blk = (uint32_t)(r / per_block);
    uint64_t o = r % per_block;
    uint8_t* blob = base + e * stride;
    const uint64_t key = ((e * 3 + blk) << 2);
    if (o < words) {
      const uint32_t u = (uint32_t)rand64(seed ^ key, o);
      // 3-bit: one random 24-bit pack per 3 bytes (uniform codes 0..7).
      if (g.bits == 4) {
        reinterpret_cast<uint32_t*>(blob + g.w[blk])[o] = u;
      } else {
        uint8_t* p = blob + g.w[blk] + 4 * o;
        p[0] = (uint8_t)u;
        p[1] = (uint8_t)(u >> 8);
        p[2] = (uint8_t)(u >> 16);
        p[3] = (uint8_t)(u >> 24);
      }
      continue;
    }
    o -= words;
    if (o < halves) {
      const float v = fabsf(normal01(seed ^ (key | 1), o)) * ssig;
      reinterpret_cast<uint16_t*>(blob + g.s[blk])[o] = to_bf16_rne(v);
      continue;
    }
    o -= halves;
    const float v = normal01(seed ^ (key | 2), o) * bsig;
    reinterpret_cast<uint16_t*>(blob + g.b[blk])[o] = to_bf16_rne(v);
  }
}

hipError_t launch_synth_experts(uint8_t* base, uint32_t n_experts, uint64_t stride,
                                const BlobGeom& g, uint64_t seed, float ssig, float bsig,
                                hipStream_t st) {
  hipLaunchKernelGGL(k_synth_experts, dim3(4096), dim3(256), 0, st, base, n_experts, stride, g,
                     seed, ssig, bsig);
  return hipGetLastError();
}

__global__ void k_synth_f32(float* __restrict__ out, uint64_t n, uint64_t seed, float sigma) {
  for (uint64_t i = (uint64_t)blockIdx.x * blockDim.x + threadIdx.x; i < n;
       i += (uint64_t)gridDim.x * blockDim.x)
    out[i] = normal01(seed, i) * sigma;
}

__global__ void k_synth_bf16(uint16_t* __restrict__ out, uint64_t n, uint64_t seed, float sigma) {
  for (uint64_t i = (uint64_t)blockIdx.x * blockDim.x + threadIdx.x; i < n;
       i += (uint64_t)gridDim.x * blockDim.x)
    out[i] = to_bf16_rne(normal01(seed, i) * sigma);
}

hipError_t launch_synth_normal_f32(float* out, uint64_t n, uint64_t seed, float sigma,
                                   hipStream_t st) {
  hipLaunchKernelGGL(k_synth_f32, dim3(2048), dim3(256), 0, st, out, n, seed, sigma);
  return hipGetLastError();
}

hipError_t launch_synth_normal_bf16(uint16_t* out, uint64_t n, uint64_t seed, float sigma,
                                    hipStream_t st) {
  hipLaunchKernelGGL(k_synth_bf16, dim3(2048), dim3(256), 0, st, out, n, seed, sigma);
  return hipGetLastError();
}

}  // namespace smoe

namespace smoe {

// ---------------------------------------------------------------------------
// Streaming-read diagnostic: every byte of `buf` is read once with 128-bit
// loads (grid-stride, 4 loads in flight per thread); each block writes the
// XOR of what it read to sink[block] so the loads cannot be dropped.
// ---------------------------------------------------------------------------
__global__ __launch_bounds__(256) void k_stream_read(const u32x4* __restrict__ p, uint64_t n16,
                                                     uint32_t* __restrict__ sink) {
  __shared__ uint32_t red[4];
  uint32_t acc = 0;
  const uint64_t stride = (uint64_t)gridDim.x * blockDim.x;
  uint64_t i = (uint64_t)blockIdx.x * blockDim.x + threadIdx.x;
  for (; i + 3 * stride < n16; i += 4 * stride) {
    const u32x4 a = __builtin_nontemporal_load(p + i);
    const u32x4 b = __builtin_nontemporal_load(p + i + stride);
    const u32x4 c = __builtin_nontemporal_load(p + i + 2 * stride);
    const u32x4 d = __builtin_nontemporal_load(p + i + 3 * stride);
    acc ^= a.x ^ a.y ^ a.z ^ a.w ^ b.x ^ b.y ^ b.z ^ b.w ^ c.x ^ c.y ^ c.z ^ c.w ^ d.x ^ d.y ^ d.z ^ d.w;
  }
  for (; i < n16; i += stride) {
    const u32x4 a = __builtin_nontemporal_load(p + i);
    acc ^= a.x ^ a.y ^ a.z ^ a.w;
  }
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) acc ^= __shfl_xor(acc, o, 64);
  if ((threadIdx.x & 63) == 0) red[threadIdx.x >> 6] = acc;
  __syncthreads();
  if (threadIdx.x == 0) sink[blockIdx.x] = red[0] ^ red[1] ^ red[2] ^ red[3];
}

hipError_t launch_stream_read(const void* buf, uint64_t bytes, uint32_t* sink, hipStream_t st) {
  hipLaunchKernelGGL(k_stream_read, dim3(kStreamBlocks), dim3(256), 0, st,
                     reinterpret_cast<const u32x4*>(buf), bytes / 16, sink);
  return hipGetLastError();
}

}  // namespace smoe
