// api.hip — the C ABI of libsmoe (include/smoe.h): argument validation,
// the handle's reserved scratch, and dispatch to the kernel launchers.
#include <math.h>
#include <string.h>

#include <mutex>
#include <new>

#include "../../include/smoe.h"
#include "handle.h"
#include "kernels.h"

using namespace smoe;


namespace {

constexpr uint32_t kAbiVersion = SMOE_ABI_VERSION;

int hip_status(hipError_t e) { return e == hipSuccess ? SMOE_OK : SMOE_ERR_HIP; }

bool aligned(const void* p, uint64_t off, uint64_t a) {
  return (((uintptr_t)p + off) % a) == 0;
}

int check_group(uint32_t group) {
  return (group == 32 || group == 64 || group == 128) ? SMOE_OK : SMOE_ERR_UNSUPPORTED_GROUP;
}

int check_shape(const smoe_expert_shape* s) {
  if (!s || !s->hidden || !s->inter) return SMOE_ERR_INVALID_ARG;
  if (s->bits != 4 && s->bits != 3) return SMOE_ERR_UNSUPPORTED_BITS;
  if (int rc = check_group(s->group)) return rc;
  if (s->hidden % s->group || s->inter % s->group) return SMOE_ERR_IN_DIM_NOT_MULTIPLE;
  // Kernel instances: any hidden up to 8192 and inter up to 2048 (both
  // multiples of the group, so of 32).
  if (s->hidden > 8192 || s->inter > 2048) return SMOE_ERR_UNSUPPORTED_SHAPE;
  return SMOE_OK;
}

// A blob's codes must allow the chunk loads: 16 bytes (4-bit), 4 (3-bit).
bool blob_aligned(const void* p, uint32_t bits) { return aligned(p, 0, bits == 4 ? 16 : 4); }

int reserve(smoe_handle* h, uint32_t H, uint32_t I, uint32_t E) {
  if (h->mem && H <= h->max_hidden && I <= h->max_inter && E <= h->max_experts) return SMOE_OK;
  H = H > h->max_hidden ? H : h->max_hidden;
  I = I > h->max_inter ? I : h->max_inter;
  E = E > h->max_experts ? E : h->max_experts;
  auto al = [](size_t n) { return (n + 255) & ~(size_t)255; };
  // act, logits, route table and limbs hold kMaxDecodeTokens tokens
  // (multi-token decode); single-token paths use token 0's.
  const size_t T = kMaxDecodeTokens;
  // Per token at least E + 1 logits, and a whole number of 64 lanes x P
  // (the three-kernel decode reads them unguarded).
  const size_t lstride = logit_stride(E);
  const size_t act_b = al(T * kMaxSlotsHost * I * sizeof(float));
  const size_t log_b = al(T * lstride * sizeof(float));
  const size_t tab_b = al(T * sizeof(FfnTable));
  const size_t xl_b = al(T * (size_t)H / 32 * 32 * sizeof(uint32_t));
  const size_t arg_b = 2 * (size_t)kQmvMaxWaves * sizeof(uint32_t);
  const size_t grow_b = al((size_t)H * sizeof(float));  // an 8-bit shared gate's f32 weights
  const size_t total = act_b + log_b + 256 + tab_b + xl_b + arg_b + 256 + grow_b;
  void* mem = nullptr;
  if (hipSetDevice(h->device) != hipSuccess) return SMOE_ERR_HIP;
  if (hipMalloc(&mem, total) != hipSuccess) return SMOE_ERR_HIP;
  if (hipMemset(mem, 0, total) != hipSuccess) {
    (void)hipFree(mem);
    return SMOE_ERR_HIP;
  }
  if (h->mem) {
    (void)hipDeviceSynchronize();
    (void)hipFree(h->mem);
  }
  char* p = (char*)mem;
  h->mem = mem;
  h->act = (float*)p;
  h->logits = (float*)(p + act_b);
  h->gate = (float*)(p + act_b + log_b);
  h->table = (FfnTable*)(p + act_b + log_b + 256);
  char* q = p + act_b + log_b + 256 + tab_b;
  h->xl = (uint32_t*)q;
  q += xl_b;
  h->arg_v = (float*)q;
  h->arg_i = (uint32_t*)(q + kQmvMaxWaves * sizeof(float));
  q += arg_b;
  h->err = (uint32_t*)q;
  h->gate_row = (float*)(q + 256);
  h->lstride = (uint32_t)lstride;
  h->astride = (uint32_t)(kMaxSlotsHost * I);
  h->xstride = H / 32 * 32;
  h->max_hidden = H;
  h->max_inter = I;
  h->max_experts = E;
  return SMOE_OK;
}

int use_device(smoe_handle* h) { return hipSetDevice(h->device) == hipSuccess ? SMOE_OK : SMOE_ERR_HIP; }

// ---------------------------------------------------------------------------
// Fixed scratch of the no-allocation decode (smoe_moe_decode_layers_noalloc):
// one file-scope device array, which every GPU the library runs on holds
// until the process ends. In host code `scratch` only names the symbol; its
// address on a device comes from hipGetSymbolAddress with that device
// current, kept per device in g_noalloc below, and only that address is
// ever passed to a kernel. Calls that overlap on one GPU share the array
// and race; nothing in it has to start at zero (every kernel writes what it
// later reads within the same layer).
// ---------------------------------------------------------------------------
constexpr size_t kNoAllocScratchBytes = 128 * 1024;
static __device__ __align__(256) uint8_t scratch[kNoAllocScratchBytes];

constexpr int kNoAllocMaxDevices = 64;
std::mutex g_noalloc_mu;
void* g_noalloc[kNoAllocMaxDevices];  // device address of `scratch`, per device

// The device address of `scratch` on the current device `dev`, looked up
// once per device (smoe_create does it for its device; the entry point for
// any other).
int noalloc_scratch(int dev, uint8_t** out) {
  if (dev < 0 || dev >= kNoAllocMaxDevices) return SMOE_ERR_NO_DEVICE;
  std::lock_guard<std::mutex> lock(g_noalloc_mu);
  if (!g_noalloc[dev]) {
    void* p = nullptr;
    if (hipGetSymbolAddress(&p, HIP_SYMBOL(scratch)) != hipSuccess || !p) return SMOE_ERR_HIP;
    g_noalloc[dev] = p;
  }
  *out = (uint8_t*)g_noalloc[dev];
  return SMOE_OK;
}

}  // namespace

extern "C" {

const char* smoe_strerror(int status) {
  switch (status) {
    case SMOE_OK: return "ok";
    case SMOE_ERR_INVALID_ARG: return "invalid argument (null pointer, zero size or bad enum)";
    case SMOE_ERR_BAD_K: return "k out of range: must be 1..=16 and <= n_experts";
    case SMOE_ERR_IN_DIM_NOT_MULTIPLE: return "input dimension is not a multiple of the group size";
    case SMOE_ERR_UNSUPPORTED_BITS: return "unsupported weight width (4 or 3 bits)";
    case SMOE_ERR_UNSUPPORTED_GROUP: return "unsupported group size (32, 64 or 128)";
    case SMOE_ERR_UNSUPPORTED_SHAPE: return "no kernel instance for this shape";
    case SMOE_ERR_MISALIGNED: return "weight, scale or activation pointer misaligned";
    case SMOE_ERR_SCRATCH_TOO_SMALL:
      return "shape exceeds the reserved scratch (smoe_reserve), or the fixed 128 KiB scratch of "
             "smoe_moe_decode_layers_noalloc";
    case SMOE_ERR_WORKSPACE_TOO_SMALL: return "workspace smaller than the required size";
    case SMOE_ERR_HIP: return "HIP runtime error";
    case SMOE_ERR_NO_DEVICE: return "no gfx950 device at that ordinal";
    case SMOE_ERR_DEVICE_TIMEOUT: return "a bounded device-side wait expired (reserved: no entry point of this build waits)";
    case SMOE_ERR_IO: return "file could not be opened or read, or is shorter than asked";
    default: return "unknown status";
  }
}

uint32_t smoe_abi_version(void) { return kAbiVersion; }

int smoe_create(int device, void* stream, smoe_handle** out) {
  if (!out) return SMOE_ERR_INVALID_ARG;
  *out = nullptr;
  int n = 0;
  if (hipGetDeviceCount(&n) != hipSuccess || device < 0 || device >= n) return SMOE_ERR_NO_DEVICE;
  hipDeviceProp_t prop;
  if (hipGetDeviceProperties(&prop, device) != hipSuccess) return SMOE_ERR_HIP;
  if (strncmp(prop.gcnArchName, "gfx950", 6) != 0) return SMOE_ERR_NO_DEVICE;
  smoe_handle* h = new (std::nothrow) smoe_handle;
  if (!h) return SMOE_ERR_HIP;
  h->device = device;
  h->stream = (hipStream_t)stream;
  int rc = reserve(h, 4096, 2048, 1024);
  uint8_t* fixed = nullptr;
  if (!rc) rc = noalloc_scratch(device, &fixed);  // set-up of the no-allocation decode on this device
  if (rc) {
    if (h->mem) (void)hipFree(h->mem);
    delete h;
    return rc;
  }
  *out = h;
  return SMOE_OK;
}

int smoe_destroy(smoe_handle* h) {
  if (!h) return SMOE_ERR_INVALID_ARG;
  (void)hipSetDevice(h->device);
  if (h->mem) {
    (void)hipStreamSynchronize(h->stream);
    (void)hipFree(h->mem);
  }
  release_staging(h);
  delete h;
  return SMOE_OK;
}

int smoe_set_stream(smoe_handle* h, void* stream) {
  if (!h) return SMOE_ERR_INVALID_ARG;
  h->stream = (hipStream_t)stream;
  return SMOE_OK;
}

int smoe_reserve(smoe_handle* h, uint32_t max_hidden, uint32_t max_inter, uint32_t max_experts) {
  if (!h) return SMOE_ERR_INVALID_ARG;
  return reserve(h, max_hidden, max_inter, max_experts);
}

int smoe_sync(smoe_handle* h) {
  if (!h) return SMOE_ERR_INVALID_ARG;
  if (int rc = use_device(h)) return rc;
  if (hipStreamSynchronize(h->stream) != hipSuccess) return SMOE_ERR_HIP;
  uint32_t e = 0;
  if (hipMemcpy(&e, h->err, sizeof(e), hipMemcpyDeviceToHost) != hipSuccess) return SMOE_ERR_HIP;
  if (e) {
    if (hipMemset(h->err, 0, sizeof(e)) != hipSuccess) return SMOE_ERR_HIP;
    return e == 2u ? SMOE_ERR_INVALID_ARG : SMOE_ERR_DEVICE_TIMEOUT;
  }
  return SMOE_OK;
}

int smoe_set_option(smoe_handle* h, int option, int64_t value) {
  if (!h) return SMOE_ERR_INVALID_ARG;
  switch (option) {
    case SMOE_OPT_DECODE_PATH:
      // 2 was the persistent cooperative decode, removed (slower than the
      // three-kernel path on every shape it covered).
      if (value < 0 || value > 3 || value == 2) return SMOE_ERR_INVALID_ARG;
      h->decode_path = (int)value;
      return SMOE_OK;
    case SMOE_OPT_TRACE_BUFFER:
      h->trace = (uint64_t*)(uintptr_t)value;
      return SMOE_OK;
    case SMOE_OPT_PREFILL_GEMM:
      if (value < 0 || value > 2) return SMOE_ERR_INVALID_ARG;
      h->prefill_gemm = (int)value;
      return SMOE_OK;
    default:
      return SMOE_ERR_INVALID_ARG;
  }
}

// allow8: the entry point takes 8-bit weights (one byte per input).
static int qview(const smoe_qweights* w, uint32_t in_dim, QView* v, bool allow8 = false) {
  if (!w || !w->base || !in_dim) return SMOE_ERR_INVALID_ARG;
  if (w->bits != 4 && w->bits != 3 && !(allow8 && w->bits == 8)) return SMOE_ERR_UNSUPPORTED_BITS;
  if (int rc = check_group(w->group_size)) return rc;
  if (in_dim % w->group_size) return SMOE_ERR_IN_DIM_NOT_MULTIPLE;
  if (!aligned(w->base, w->packed_offset, w->bits == 3 ? 4 : 16) ||
      !aligned(w->base, w->scales_offset, 2) || !aligned(w->base, w->biases_offset, 2))
    return SMOE_ERR_MISALIGNED;
  const uint8_t* b = (const uint8_t*)w->base;
  v->codes = b + w->packed_offset;
  v->scales = (const uint16_t*)(b + w->scales_offset);
  v->biases = (const uint16_t*)(b + w->biases_offset);
  v->bits = w->bits;
  v->group = w->group_size;
  return SMOE_OK;
}

int smoe_qmv(smoe_handle* h, const smoe_qweights* w, const float* x, float* y, uint32_t out_dim,
             uint32_t in_dim) {
  if (!h || !x || !y || !out_dim) return SMOE_ERR_INVALID_ARG;
  QView v;
  if (int rc = qview(w, in_dim, &v, true)) return rc;
  if (!aligned(x, 0, 16)) return SMOE_ERR_MISALIGNED;
  if (int rc = use_device(h)) return rc;
  bool unsupported = false;
  const hipError_t e = launch_qmv(v, x, y, out_dim, in_dim, h->stream, &unsupported);
  if (unsupported) return SMOE_ERR_UNSUPPORTED_SHAPE;
  return hip_status(e);
}

uint64_t smoe_qmm_workspace_size(uint32_t in_dim, uint32_t group, uint32_t n_tokens) {
  if (!in_dim || !group || !n_tokens) return 0;
  return qmm_workspace(in_dim, group, n_tokens, nullptr, nullptr);
}

int smoe_qmm(smoe_handle* h, const smoe_qweights* w, const float* x, float* y, uint32_t out_dim,
             uint32_t in_dim, uint32_t n_tokens, void* workspace, uint64_t workspace_bytes) {
  if (!h || !x || !y || !out_dim || !n_tokens || !workspace) return SMOE_ERR_INVALID_ARG;
  QView v;
  if (int rc = qview(w, in_dim, &v, true)) return rc;
  if (!qmm_supported(in_dim, out_dim, w->group_size, w->bits, n_tokens)) {
    // Shapes without GEMM tiles (in_dim or out_dim not a multiple of 256,
    // in_dim up to 8192): one k_qmv per token row, as smoe_qmv computes it.
    if (in_dim > 8192) return SMOE_ERR_UNSUPPORTED_SHAPE;
    if (!aligned(x, 0, 16)) return SMOE_ERR_MISALIGNED;
    if (int rc = use_device(h)) return rc;
    for (uint32_t t = 0; t < n_tokens; ++t) {
      bool unsupported = false;
      const hipError_t e = launch_qmv(v, x + (size_t)t * in_dim, y + (size_t)t * out_dim, out_dim, in_dim,
                                      h->stream, &unsupported);
      if (unsupported) return SMOE_ERR_UNSUPPORTED_SHAPE;
      if (e != hipSuccess) return SMOE_ERR_HIP;
    }
    return SMOE_OK;
  }
  // The GEMM copies weights, scales and biases with 16-byte LDS DMA and
  // addresses biases from the scales (biases after them).
  if (!aligned(w->base, w->packed_offset, 16) || !aligned(w->base, w->scales_offset, 16) ||
      !aligned(w->base, w->biases_offset, 16) || !aligned(x, 0, 16) || !aligned(y, 0, 16) ||
      !aligned(workspace, 0, 256))
    return SMOE_ERR_MISALIGNED;
  if (w->biases_offset <= w->scales_offset || w->biases_offset - w->scales_offset >= (1ull << 31))
    return SMOE_ERR_UNSUPPORTED_SHAPE;
  if (workspace_bytes < qmm_workspace(in_dim, w->group_size, n_tokens, nullptr, nullptr))
    return SMOE_ERR_WORKSPACE_TOO_SMALL;
  if (int rc = use_device(h)) return rc;
  PfArgs a{};
  qmm_workspace(in_dim, w->group_size, n_tokens, &a, (uint8_t*)workspace);
  a.g.bits = w->bits;
  a.g.hidden = out_dim;
  a.g.inter = in_dim;
  a.g.group = w->group_size;
  a.g.w[2] = w->packed_offset;
  a.g.s[2] = w->scales_offset;
  a.g.b[2] = w->biases_offset;
  a.experts = (const uint8_t*)w->base;
  a.stride = 0;
  a.n_tokens = n_tokens;
  a.k = 1;
  a.down = y;
  int n_cu = 0;
  if (hipDeviceGetAttribute(&n_cu, hipDeviceAttributeMultiprocessorCount, h->device) != hipSuccess || n_cu <= 0)
    return SMOE_ERR_HIP;
  return hip_status(launch_qmm(a, x, (uint32_t)n_cu, h->stream));
}

int smoe_qmv_argmax(smoe_handle* h, const smoe_qweights* w, const float* x, float* y, uint32_t out_dim,
                    uint32_t in_dim, int32_t* out_index) {
  if (!h || !x || !y || !out_dim || !out_index) return SMOE_ERR_INVALID_ARG;
  QView v;
  if (int rc = qview(w, in_dim, &v, true)) return rc;
  if (!aligned(x, 0, 16)) return SMOE_ERR_MISALIGNED;
  // 8-bit: the argmax reads y back (16-byte loads).
  if (v.bits == 8 && !aligned(y, 0, 16)) return SMOE_ERR_MISALIGNED;
  if (!h->arg_v) return SMOE_ERR_SCRATCH_TOO_SMALL;
  if (int rc = use_device(h)) return rc;
  bool unsupported = false;
  const hipError_t e = launch_qmv(v, x, y, out_dim, in_dim, h->stream, &unsupported, h->arg_v, h->arg_i, out_index);
  if (unsupported) return SMOE_ERR_UNSUPPORTED_SHAPE;
  return hip_status(e);
}

int smoe_argmax(smoe_handle* h, const float* v, uint32_t n, int32_t* out_index) {
  if (!h || !v || !n || !out_index) return SMOE_ERR_INVALID_ARG;
  if (!aligned(v, 0, 16)) return SMOE_ERR_MISALIGNED;
  if (int rc = use_device(h)) return rc;
  return hip_status(launch_argmax(v, n, out_index, h->arg_v, h->arg_i, h->stream));
}

int smoe_dequant(smoe_handle* h, const smoe_qweights* w, uint32_t in_dim, uint32_t row0,
                 uint32_t n_rows, float* out) {
  if (!h || !out || !n_rows) return SMOE_ERR_INVALID_ARG;
  QView v;
  if (int rc = qview(w, in_dim, &v, true)) return rc;
  if (in_dim % 32) return SMOE_ERR_UNSUPPORTED_SHAPE;
  if (int rc = use_device(h)) return rc;
  return hip_status(launch_dequant(v, in_dim, row0, n_rows, out, h->stream));
}

static int check_router(uint32_t n_tokens, uint32_t n_experts, uint32_t k) {
  if (!n_tokens || !n_experts) return SMOE_ERR_INVALID_ARG;
  if (k < 1 || k > SMOE_MAX_K || k > n_experts) return SMOE_ERR_BAD_K;
  if (n_experts > 1024) return SMOE_ERR_UNSUPPORTED_SHAPE;
  return SMOE_OK;
}

int smoe_router(smoe_handle* h, const float* router_w, const float* x, uint32_t n_tokens,
                uint32_t n_experts, uint32_t hidden, uint32_t k, int normalize, int32_t* idx,
                float* weights, float* logits_out) {
  if (!h || !router_w || !x || !idx || !weights || !hidden) return SMOE_ERR_INVALID_ARG;
  if (int rc = check_router(n_tokens, n_experts, k)) return rc;
  if (hidden % 4) return SMOE_ERR_UNSUPPORTED_SHAPE;
  if (!aligned(router_w, 0, 16) || !aligned(x, 0, 16)) return SMOE_ERR_MISALIGNED;
  float* logits = logits_out;
  if (!logits) {
    if ((uint64_t)n_tokens * n_experts > h->max_experts) return SMOE_ERR_SCRATCH_TOO_SMALL;
    logits = h->logits;
  }
  if (int rc = use_device(h)) return rc;
  hipError_t e = launch_router_logits(router_w, nullptr, x, n_tokens, n_experts, hidden, logits,
                                      nullptr, h->stream);
  if (e != hipSuccess) return SMOE_ERR_HIP;
  RouteOut ro{};
  ro.idx = idx;
  ro.weight = weights;
  return hip_status(launch_topk(logits, n_tokens, n_experts, k, true, normalize != 0, ro, h->stream));
}

int smoe_softmax_topk(smoe_handle* h, const float* logits, uint32_t n_tokens, uint32_t n_experts,
                      uint32_t k, int normalize, int32_t* idx, float* weights) {
  if (!h || !logits || !idx || !weights) return SMOE_ERR_INVALID_ARG;
  if (int rc = check_router(n_tokens, n_experts, k)) return rc;
  if (int rc = use_device(h)) return rc;
  RouteOut ro{};
  ro.idx = idx;
  ro.weight = weights;
  return hip_status(launch_topk(logits, n_tokens, n_experts, k, true, normalize != 0, ro, h->stream));
}

int smoe_softmax(smoe_handle* h, const float* logits, uint32_t n_tokens, uint32_t n, float* probs) {
  if (!h || !logits || !probs) return SMOE_ERR_INVALID_ARG;
  if (int rc = check_router(n_tokens, n, 1)) return rc;
  if (int rc = use_device(h)) return rc;
  RouteOut ro{};
  ro.probs = probs;
  return hip_status(launch_topk(logits, n_tokens, n, 1, true, false, ro, h->stream));
}

int smoe_expf(smoe_handle* h, const float* x, float* y, uint64_t n) {
  if (!h || ((!x || !y) && n)) return SMOE_ERR_INVALID_ARG;
  if (int rc = use_device(h)) return rc;
  return hip_status(launch_expf(x, y, n, h->stream));
}

int smoe_topk(smoe_handle* h, const float* scores, uint32_t n_tokens, uint32_t n, uint32_t k,
              int32_t* idx, float* values) {
  if (!h || !scores || !idx || !values) return SMOE_ERR_INVALID_ARG;
  if (int rc = check_router(n_tokens, n, k)) return rc;
  if (int rc = use_device(h)) return rc;
  RouteOut ro{};
  ro.idx = idx;
  ro.weight = values;
  return hip_status(launch_topk(scores, n_tokens, n, k, false, false, ro, h->stream));
}

int smoe_noaux_tc_topk(smoe_handle* h, const float* logits, const float* correction_bias,
                       uint32_t n_tokens, uint32_t n_experts, uint32_t n_group, uint32_t topk_group,
                       uint32_t k, float routed_scaling_factor, int32_t* idx, float* weights,
                       float* scores_out) {
  if (!h || !logits || !correction_bias || !idx || !weights || !n_tokens || !n_experts)
    return SMOE_ERR_INVALID_ARG;
  if (n_group == 0 || n_experts % n_group) return SMOE_ERR_BAD_K;
  if (topk_group == 0 || topk_group > n_group) return SMOE_ERR_BAD_K;
  if (k < 1 || k > n_experts || k > SMOE_MAX_K) return SMOE_ERR_BAD_K;
  if (n_experts > kNoauxMaxExperts || n_group > kNoauxMaxGroups) return SMOE_ERR_UNSUPPORTED_SHAPE;
  if (int rc = use_device(h)) return rc;
  RouteOut ro{};
  ro.idx = idx;
  ro.weight = weights;
  return hip_status(launch_noaux_topk(logits, correction_bias, n_tokens, n_experts, n_group, topk_group,
                                      k, routed_scaling_factor, scores_out, ro, h->stream));
}

uint64_t smoe_expert_bytes(const smoe_expert_shape* s) {
  if (!s || !s->group) return 0;
  const uint64_t w = (uint64_t)s->inter * s->hidden * s->bits / 8;
  const uint64_t sc = (uint64_t)s->inter * (s->hidden / s->group) * 2;
  return 3 * (w + 2 * sc);
}

int smoe_experts_decode(smoe_handle* h, const smoe_expert_shape* shape,
                        const smoe_binding* bindings, uint32_t k, const float* weights,
                        const float* input, const float* h_mid, const float* shared_out,
                        float shared_gate_score, float* hidden_out) {
  if (!h || !bindings || !weights || !input || !h_mid || !hidden_out) return SMOE_ERR_INVALID_ARG;
  if (int rc = check_shape(shape)) return rc;
  if (k < 1 || k > SMOE_MAX_K) return SMOE_ERR_BAD_K;
  if (shape->hidden > h->max_hidden || shape->inter > h->max_inter)
    return SMOE_ERR_SCRATCH_TOO_SMALL;
  if (!aligned(input, 0, 16)) return SMOE_ERR_MISALIGNED;
  FfnTable tab{};
  for (uint32_t s = 0; s < k; ++s) {
    if (!bindings[s].base) return SMOE_ERR_INVALID_ARG;
    const uint8_t* p = (const uint8_t*)bindings[s].base + bindings[s].offset;
    if (!blob_aligned(p, shape->bits)) return SMOE_ERR_MISALIGNED;
    tab.blob[s] = p;
    tab.weight[s] = weights[s];
  }
  tab.k = k;
  tab.has_shared = 0;
  tab.shared_gate = shared_gate_score;
  if (int rc = use_device(h)) return rc;
  const BlobGeom g = blob_geom(shape->hidden, shape->inter, shape->group, shape->bits);
  bool uns = false;
  hipError_t e = launch_gateup(g, g, nullptr, tab, k, input, h->act, h->stream, &uns);
  if (uns) return SMOE_ERR_UNSUPPORTED_SHAPE;
  if (e != hipSuccess) return SMOE_ERR_HIP;
  e = launch_down_combine(g, g, nullptr, tab, k, h->act, h_mid, shared_out, hidden_out, h->stream,
                          &uns);
  if (uns) return SMOE_ERR_UNSUPPORTED_SHAPE;
  return hip_status(e);
}

// An 8-bit router or shared gate of a layer (bits 8, rows of `hidden`
// inputs); null: r stays unused.
static int q8_rows(const smoe_qweights* w, uint32_t hidden, Q8Rows* r) {
  *r = Q8Rows{};
  if (!w) return SMOE_OK;
  if (w->bits != 8) return SMOE_ERR_UNSUPPORTED_BITS;
  QView v;
  if (int rc = qview(w, hidden, &v, true)) return rc;
  r->q = v.codes;
  r->s = v.scales;
  r->b = v.biases;
  r->group = v.group;
  return SMOE_OK;
}

// The layer's router and (with a shared expert) shared gate in 8-bit form.
static void layer_q8(const smoe_layer* L, Q8Rows* router, Q8Rows* gate) {
  q8_rows(L->router_q, L->shape.hidden, router);
  q8_rows(L->shared_expert ? L->shared_gate_q : nullptr, L->shape.hidden, gate);
}

// Arguments of one resident layer, independent of any reservation.
static int check_layer_args(const smoe_layer* L) {
  if (!L || !L->experts) return SMOE_ERR_INVALID_ARG;
  // Exactly one router form, at most one gate form.
  if ((L->router_w != nullptr) == (L->router_q != nullptr)) return SMOE_ERR_INVALID_ARG;
  if (L->shared_gate && L->shared_gate_q) return SMOE_ERR_INVALID_ARG;
  if (int rc = check_shape(&L->shape)) return rc;
  if (int rc = check_router(1, L->n_experts, L->k)) return rc;
  if (L->stride < smoe_expert_bytes(&L->shape)) return SMOE_ERR_INVALID_ARG;
  if (!blob_aligned(L->experts, L->shape.bits) || L->stride % (L->shape.bits == 4 ? 16 : 4))
    return SMOE_ERR_MISALIGNED;
  if (L->shared_expert && !blob_aligned(L->shared_expert, 4)) return SMOE_ERR_MISALIGNED;
  if ((L->router_w && !aligned(L->router_w, 0, 16)) || (L->shared_gate && !aligned(L->shared_gate, 0, 16)))
    return SMOE_ERR_MISALIGNED;
  if (L->shape.hidden % 4) return SMOE_ERR_UNSUPPORTED_SHAPE;
  Q8Rows q;
  if (int rc = q8_rows(L->router_q, L->shape.hidden, &q)) return rc;
  if (int rc = q8_rows(L->shared_gate_q, L->shape.hidden, &q)) return rc;
  return SMOE_OK;
}

static int check_layer(smoe_handle* h, const smoe_layer* L) {
  if (int rc = check_layer_args(L)) return rc;
  if (L->shape.hidden > h->max_hidden || L->shape.inter > h->max_inter ||
      L->n_experts > h->max_experts)
    return SMOE_ERR_SCRATCH_TOO_SMALL;
  return SMOE_OK;
}

// With norm_w, `input` is the residual: the router kernel normalises it
// (bf16 weights norm_w, eps) and stores the normalised row in x_norm, which
// the expert kernels then read.
static int decode_layer(smoe_handle* h, const smoe_layer* L, const float* input,
                        const float* h_mid, float* hidden_out, int32_t* idx_out, float* w_out,
                        const uint16_t* norm_w = nullptr, float eps = 0.f, float* x_norm = nullptr) {
  const smoe_expert_shape& s = L->shape;
  Q8Rows rq, gq;
  layer_q8(L, &rq, &gq);
  hipError_t e = launch_router_logits(L->router_w, L->shared_expert ? L->shared_gate : nullptr,
                                      input, 1, L->n_experts, s.hidden, h->logits, h->gate,
                                      h->stream, norm_w, eps, x_norm, rq, gq);
  if (norm_w) input = x_norm;
  if (e != hipSuccess) return SMOE_ERR_HIP;
  RouteOut ro{};
  ro.idx = idx_out;
  ro.weight = w_out;
  ro.table = h->table;
  ro.experts = (const uint8_t*)L->experts;
  ro.stride = L->stride;
  ro.shared_blob = (const uint8_t*)L->shared_expert;
  ro.gate_scores = (L->shared_expert && (L->shared_gate || L->shared_gate_q)) ? h->gate : nullptr;
  e = launch_topk(h->logits, 1, L->n_experts, L->k, true, L->normalize != 0, ro, h->stream);
  if (e != hipSuccess) return SMOE_ERR_HIP;
  const BlobGeom g = blob_geom(s.hidden, s.inter, s.group, s.bits);
  const BlobGeom gs = blob_geom(s.hidden, s.inter, s.group, 4);
  FfnTable tv{};
  tv.k = L->k;
  const uint32_t n_slots = L->k + (L->shared_expert ? 1 : 0);
  bool uns = false;
  e = launch_gateup(g, gs, h->table, tv, n_slots, input, h->act, h->stream, &uns);
  if (uns) return SMOE_ERR_UNSUPPORTED_SHAPE;
  if (e != hipSuccess) return SMOE_ERR_HIP;
  e = launch_down_combine(g, gs, h->table, tv, n_slots, h->act, h_mid, nullptr, hidden_out,
                          h->stream, &uns);
  if (uns) return SMOE_ERR_UNSUPPORTED_SHAPE;
  return hip_status(e);
}

// The three-kernel layer (fused.hip). Returns SMOE_ERR_UNSUPPORTED_SHAPE
// when it has no instance for the layer.
static bool fused_ok(const smoe_layer* L) {
  const smoe_expert_shape& s = L->shape;
  return fused_supported(s.hidden, s.inter, s.group, s.bits, L->n_experts, L->k);
}

// Where the three-kernel decode keeps its per-token intermediates (router
// logits, activations, route table, x limbs) and the stream it runs on.
struct FaScratch {
  uint32_t* xl;
  float* logits;
  float* act;
  FfnTable* table;
  uint32_t lstride, astride, xstride;  // per-token strides (elements)
  uint64_t* trace;
  hipStream_t stream;
  float* gate_row;  // [hidden] f32 weights of an 8-bit shared gate
};

static FaScratch handle_scratch(const smoe_handle* h) {
  return FaScratch{h->xl,      h->logits,  h->act,   h->table,  h->lstride,
                   h->astride, h->xstride, h->trace, h->stream, h->gate_row};
}

static int decode_fused(const FaScratch& sc, const smoe_layer* L, const float* x_in, const float* resid,
                        const uint16_t* norm, float eps, const float* h_mid, float* out, int32_t* idx_out,
                        float* w_out, uint32_t layer_index, uint32_t n_tokens = 1) {
  if (!fused_ok(L)) return SMOE_ERR_UNSUPPORTED_SHAPE;
  const smoe_expert_shape& s = L->shape;
  FusedLayer a{};
  a.hidden = s.hidden;
  a.x_in = x_in;
  a.resid = resid;
  a.norm = norm;
  a.eps = eps;
  a.xl = sc.xl;
  FaQ8 q;
  layer_q8(L, &q.router, &q.gate);
  // An 8-bit router: the limbs stand in for K_B's unused gate row.
  a.router = L->router_w ? L->router_w : reinterpret_cast<const float*>(sc.xl);
  a.shared = (const uint8_t*)L->shared_expert;
  a.gate = L->shared_expert ? L->shared_gate : nullptr;
  if (q.gate.q) {
    q.gate_f32 = sc.gate_row;
    a.gate = sc.gate_row;
  }
  a.experts = (const uint8_t*)L->experts;
  a.stride = L->stride;
  a.routed = blob_geom(s.hidden, s.inter, s.group, s.bits);
  a.sgeom = blob_geom(s.hidden, s.inter, s.group, 4);
  a.E = L->n_experts;
  a.k = L->k;
  a.normalize = L->normalize != 0;
  a.logits = sc.logits;
  a.act = sc.act;
  a.table = sc.table;
  a.h_mid = h_mid;
  a.out = out;
  a.idx_out = idx_out;
  a.w_out = w_out;
  a.trace = (sc.trace && n_tokens == 1) ? sc.trace + (uint64_t)layer_index * kFaTraceLayer : nullptr;
  a.n_tokens = n_tokens;
  a.lstride = sc.lstride;
  a.astride = sc.astride;
  a.xstride = sc.xstride;
  return hip_status(launch_fused_layer(a, sc.stream, q));
}

// n_layers layers of one token on the three-kernel path: layer l reads x_l
// (input, or RMSNorm(residual) * norm_w[l] inside the router kernel) and
// adds its MoE output to residual_io.
static int decode_chain_fused(const FaScratch& sc, const smoe_layer* layers, uint32_t n_layers,
                              const void* const* norm_w, float eps, const float* input, float* residual_io) {
  for (uint32_t l = 0; l < n_layers; ++l) {
    const uint16_t* nw = (norm_w && l > 0) ? (const uint16_t*)norm_w[l] : nullptr;
    if (int rc = decode_fused(sc, &layers[l], l == 0 ? input : nullptr, residual_io, nw, eps, residual_io,
                              residual_io, nullptr, nullptr, l))
      return rc;
  }
  return SMOE_OK;
}

int smoe_moe_decode_layer(smoe_handle* h, const smoe_layer* layer, const float* input,
                          const float* h_mid, float* hidden_out, int32_t* idx_out, float* w_out) {
  if (!h || !input || !h_mid || !hidden_out) return SMOE_ERR_INVALID_ARG;
  if (int rc = check_layer(h, layer)) return rc;
  if (!aligned(input, 0, 16)) return SMOE_ERR_MISALIGNED;
  if (int rc = use_device(h)) return rc;
  if (h->decode_path != 1) {
    const int rc = decode_fused(handle_scratch(h), layer, input, nullptr, nullptr, 0.f, h_mid, hidden_out,
                                idx_out, w_out, 0);
    if (rc != SMOE_ERR_UNSUPPORTED_SHAPE || h->decode_path == 3) return rc;
  }
  return decode_layer(h, layer, input, h_mid, hidden_out, idx_out, w_out);
}

// One token through the layers on the per-phase kernels (RMSNorm launch,
// then one layer), with the last layer's idx / w when asked.
static int decode_chain_phases(smoe_handle* h, const smoe_layer* layers, uint32_t n_layers,
                               const void* const* norm_w, float eps, const float* input, float* residual_io,
                               float* work, int32_t* idx_out, float* w_out) {
  for (uint32_t l = 0; l < n_layers; ++l) {
    const bool last = l + 1 == n_layers;
    // Layers after the first read the residual; with norm weights their
    // router kernel applies the RMSNorm and leaves the normalised row in work.
    const float* x = l > 0 ? residual_io : input;
    const uint16_t* nw = (l > 0 && norm_w) ? (const uint16_t*)norm_w[l] : nullptr;
    if (int rc = decode_layer(h, &layers[l], x, residual_io, residual_io, last ? idx_out : nullptr,
                              last ? w_out : nullptr, nw, eps, work))
      return rc;
  }
  return SMOE_OK;
}

int smoe_moe_decode_layers(smoe_handle* h, const smoe_layer* layers, uint32_t n_layers,
                           const void* const* norm_w, float eps, const float* input,
                           float* residual_io, float* work) {
  if (!h || !layers || !n_layers || !input || !residual_io || !work) return SMOE_ERR_INVALID_ARG;
  for (uint32_t l = 0; l < n_layers; ++l) {
    if (int rc = check_layer(h, &layers[l])) return rc;
    if (layers[l].shape.hidden != layers[0].shape.hidden) return SMOE_ERR_INVALID_ARG;
    if (norm_w && l > 0 && !norm_w[l]) return SMOE_ERR_INVALID_ARG;
  }
  if (!aligned(input, 0, 16) || !aligned(residual_io, 0, 16) || !aligned(work, 0, 16))
    return SMOE_ERR_MISALIGNED;
  if (int rc = use_device(h)) return rc;
  if (h->decode_path == 0 || h->decode_path == 3) {
    bool all = true;
    for (uint32_t l = 0; l < n_layers; ++l) all = all && fused_ok(&layers[l]);
    if (all) return decode_chain_fused(handle_scratch(h), layers, n_layers, norm_w, eps, input, residual_io);
    if (h->decode_path == 3) return SMOE_ERR_UNSUPPORTED_SHAPE;
  }
  return decode_chain_phases(h, layers, n_layers, norm_w, eps, input, residual_io, work, nullptr, nullptr);
}

int smoe_moe_decode_layers_noalloc(void* stream, const smoe_layer* layers, uint32_t n_layers,
                                   const void* const* norm_w, float eps, const float* input, float* residual_io) {
  if (!layers || !n_layers || !input || !residual_io) return SMOE_ERR_INVALID_ARG;
  uint32_t max_e = 0, max_i = 0;
  for (uint32_t l = 0; l < n_layers; ++l) {
    if (int rc = check_layer_args(&layers[l])) return rc;
    if (layers[l].shape.hidden != layers[0].shape.hidden) return SMOE_ERR_INVALID_ARG;
    if (norm_w && l > 0 && !norm_w[l]) return SMOE_ERR_INVALID_ARG;
    if (!fused_ok(&layers[l])) return SMOE_ERR_UNSUPPORTED_SHAPE;
    max_e = layers[l].n_experts > max_e ? layers[l].n_experts : max_e;
    max_i = layers[l].shape.inter > max_i ? layers[l].shape.inter : max_i;
  }
  if (!aligned(input, 0, 16) || !aligned(residual_io, 0, 16)) return SMOE_ERR_MISALIGNED;
  // Layout of the fixed scratch for one token (the handle's layout, sized
  // to these layers): logits, activations of the k + 1 slots, route table,
  // x limbs, each 256-byte aligned.
  auto al = [](size_t n) { return (n + 255) & ~(size_t)255; };
  const uint32_t H = layers[0].shape.hidden;
  const size_t lstride = logit_stride(max_e);
  const size_t log_b = al(lstride * sizeof(float));
  const size_t act_b = al((size_t)kMaxSlotsHost * max_i * sizeof(float));
  const size_t tab_b = al(sizeof(FfnTable));
  const size_t xl_b = al((size_t)H / 32 * 32 * sizeof(uint32_t));
  const size_t grow_b = al((size_t)H * sizeof(float));  // an 8-bit shared gate's f32 weights
  if (log_b + act_b + tab_b + xl_b + grow_b > kNoAllocScratchBytes) return SMOE_ERR_SCRATCH_TOO_SMALL;
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess) return SMOE_ERR_HIP;
  uint8_t* base = nullptr;
  if (int rc = noalloc_scratch(dev, &base)) return rc;
  FaScratch sc{};
  sc.logits = (float*)base;
  sc.act = (float*)(base + log_b);
  sc.table = (FfnTable*)(base + log_b + act_b);
  sc.xl = (uint32_t*)(base + log_b + act_b + tab_b);
  sc.gate_row = (float*)(base + log_b + act_b + tab_b + xl_b);
  sc.lstride = (uint32_t)lstride;
  sc.astride = (uint32_t)(kMaxSlotsHost * max_i);
  sc.xstride = H / 32 * 32;
  sc.trace = nullptr;
  sc.stream = (hipStream_t)stream;
  return decode_chain_fused(sc, layers, n_layers, norm_w, eps, input, residual_io);
}

int smoe_moe_decode_tokens(smoe_handle* h, const smoe_layer* layers, uint32_t n_layers,
                           const void* const* norm_w, float eps, uint32_t n_tokens, const float* input,
                           float* residual_io, float* work, int32_t* idx_out, float* w_out) {
  if (!h || !layers || !n_layers || !input || !residual_io || !work) return SMOE_ERR_INVALID_ARG;
  if (n_tokens < 1 || n_tokens > kMaxDecodeTokens) return SMOE_ERR_INVALID_ARG;
  bool all = h->decode_path != 1;
  for (uint32_t l = 0; l < n_layers; ++l) {
    if (int rc = check_layer(h, &layers[l])) return rc;
    if (layers[l].shape.hidden != layers[0].shape.hidden) return SMOE_ERR_INVALID_ARG;
    if (norm_w && l > 0 && !norm_w[l]) return SMOE_ERR_INVALID_ARG;
    all = all && fused_ok(&layers[l]);
  }
  if (!all && h->decode_path == 3) return SMOE_ERR_UNSUPPORTED_SHAPE;
  if (!aligned(input, 0, 16) || !aligned(residual_io, 0, 16) || !aligned(work, 0, 16))
    return SMOE_ERR_MISALIGNED;
  if (int rc = use_device(h)) return rc;
  if (!all) {
    // Shapes without a three-kernel instance (or the per-phase path asked
    // for): each token through the per-phase chain in turn.
    const uint32_t H = layers[0].shape.hidden, K = layers[n_layers - 1].k;
    for (uint32_t t = 0; t < n_tokens; ++t)
      if (int rc = decode_chain_phases(h, layers, n_layers, norm_w, eps, input + (size_t)t * H,
                                       residual_io + (size_t)t * H, work + (size_t)t * H,
                                       idx_out ? idx_out + (size_t)t * K : nullptr,
                                       w_out ? w_out + (size_t)t * K : nullptr))
        return rc;
    return SMOE_OK;
  }
  for (uint32_t l = 0; l < n_layers; ++l) {
    const uint16_t* nw = (norm_w && l > 0) ? (const uint16_t*)norm_w[l] : nullptr;
    const bool last = l + 1 == n_layers;
    if (int rc = decode_fused(handle_scratch(h), &layers[l], l == 0 ? input : nullptr, residual_io, nw, eps,
                              residual_io, residual_io, last ? idx_out : nullptr, last ? w_out : nullptr, l,
                              n_tokens))
      return rc;
  }
  return SMOE_OK;
}

uint64_t smoe_moe_prefill_workspace_size(const smoe_expert_shape* shape, uint32_t n_tokens,
                                         uint32_t n_experts, uint32_t k) {
  if (!shape || !shape->group || !n_tokens || !n_experts || !k) return 0;
  if (!prefill_supported(shape->hidden, shape->inter, shape->group, shape->bits, n_tokens, n_experts, k))
    return prefill_tokens_workspace(shape->hidden, shape->inter, n_tokens, k, true);
  return prefill_workspace(shape->hidden, shape->inter, shape->group, n_tokens, n_experts, k, false, nullptr,
                           nullptr);
}

uint64_t smoe_moe_prefill_block_workspace_size(const smoe_expert_shape* shape, uint32_t n_tokens,
                                               uint32_t n_experts, uint32_t k, int has_shared) {
  if (!shape || !shape->group || !n_tokens || !n_experts || !k) return 0;
  if (!prefill_supported(shape->hidden, shape->inter, shape->group, shape->bits, n_tokens, n_experts, k)) return 0;
  return prefill_workspace(shape->hidden, shape->inter, shape->group, n_tokens, n_experts, k, has_shared != 0,
                           nullptr, nullptr);
}

int smoe_moe_prefill(smoe_handle* h, const smoe_expert_shape* shape, const void* experts,
                     uint64_t stride, uint32_t n_experts, const int32_t* idx,
                     const float* weights, const void* x, int x_is_bf16, uint32_t n_tokens,
                     uint32_t k, float* out_sum, void* workspace, uint64_t workspace_bytes) {
  if (!h || !experts || !idx || !weights || !x || !out_sum || !workspace || !n_tokens || !n_experts)
    return SMOE_ERR_INVALID_ARG;
  if (int rc = check_shape(shape)) return rc;
  if (k < 1 || k > SMOE_MAX_K || k > n_experts) return SMOE_ERR_BAD_K;
  if (stride < smoe_expert_bytes(shape)) return SMOE_ERR_INVALID_ARG;
  if (n_tokens > kPfMaxTokens) return SMOE_ERR_UNSUPPORTED_SHAPE;
  if (!blob_aligned(experts, shape->bits) || stride % 16 || !aligned(x, 0, 16) ||
      !aligned(out_sum, 0, 16) || !aligned(workspace, 0, 256))
    return SMOE_ERR_MISALIGNED;
  if (!prefill_supported(shape->hidden, shape->inter, shape->group, shape->bits, n_tokens, n_experts, k)) {
    // Shapes without grouped-GEMM tiles: one token at a time through the
    // per-phase decode kernels.
    if (workspace_bytes < prefill_tokens_workspace(shape->hidden, shape->inter, n_tokens, k, x_is_bf16 != 0))
      return SMOE_ERR_WORKSPACE_TOO_SMALL;
    if (int rc = use_device(h)) return rc;
    bool unsupported = false;
    const hipError_t e = launch_prefill_tokens(
        blob_geom(shape->hidden, shape->inter, shape->group, shape->bits), (const uint8_t*)experts, stride,
        n_experts, idx, weights, x, x_is_bf16 != 0, n_tokens, k, out_sum, (uint8_t*)workspace, h->err, h->stream,
        &unsupported);
    if (unsupported) return SMOE_ERR_UNSUPPORTED_SHAPE;
    return hip_status(e);
  }
  PfArgs a{};
  const uint64_t need = prefill_workspace(shape->hidden, shape->inter, shape->group, n_tokens,
                                          n_experts, k, false, &a, (uint8_t*)workspace);
  if (workspace_bytes < need) return SMOE_ERR_WORKSPACE_TOO_SMALL;
  if (int rc = use_device(h)) return rc;
  a.g = blob_geom(shape->hidden, shape->inter, shape->group, shape->bits);
  a.experts = (const uint8_t*)experts;
  a.stride = stride;
  a.E = n_experts;
  a.k = k;
  a.n_tokens = n_tokens;
  a.idx = idx;
  a.w = weights;
  a.x = x;
  a.x_bf16 = x_is_bf16 != 0;
  a.out = out_sum;
  a.err = h->err;
  a.trace = h->trace;
  a.gemm_path = h->prefill_gemm;
  int n_cu = 0;
  if (hipDeviceGetAttribute(&n_cu, hipDeviceAttributeMultiprocessorCount, h->device) != hipSuccess || n_cu <= 0)
    return SMOE_ERR_HIP;
  return hip_status(launch_prefill(a, (uint32_t)n_cu, h->stream));
}

int smoe_moe_prefill_block(smoe_handle* h, const smoe_expert_shape* shape, const void* experts,
                           uint64_t stride, uint32_t n_experts, const int32_t* idx, const float* weights,
                           const void* x, int x_is_bf16, uint32_t n_tokens, uint32_t k,
                           const void* shared_expert, const float* shared_gate, const float* h_mid,
                           float* hidden_out, void* workspace, uint64_t workspace_bytes) {
  if (!h || !experts || !idx || !weights || !x || !h_mid || !hidden_out || !workspace || !n_tokens || !n_experts)
    return SMOE_ERR_INVALID_ARG;
  if (shared_gate && !shared_expert) return SMOE_ERR_INVALID_ARG;
  if (int rc = check_shape(shape)) return rc;
  if (k < 1 || k > SMOE_MAX_K || k > n_experts) return SMOE_ERR_BAD_K;
  if (stride < smoe_expert_bytes(shape)) return SMOE_ERR_INVALID_ARG;
  if (n_tokens > kPfMaxTokens) return SMOE_ERR_UNSUPPORTED_SHAPE;
  if (!prefill_supported(shape->hidden, shape->inter, shape->group, shape->bits, n_tokens, n_experts, k))
    return SMOE_ERR_UNSUPPORTED_SHAPE;
  if (!blob_aligned(experts, shape->bits) || stride % 16 || !aligned(x, 0, 16) || !aligned(h_mid, 0, 16) ||
      !aligned(hidden_out, 0, 16) || !aligned(workspace, 0, 256) || (shared_expert && !blob_aligned(shared_expert, 4)) ||
      (shared_gate && !aligned(shared_gate, 0, 16)))
    return SMOE_ERR_MISALIGNED;
  PfArgs a{};
  const uint64_t need = prefill_workspace(shape->hidden, shape->inter, shape->group, n_tokens, n_experts, k,
                                          shared_expert != nullptr, &a, (uint8_t*)workspace);
  if (workspace_bytes < need) return SMOE_ERR_WORKSPACE_TOO_SMALL;
  if (int rc = use_device(h)) return rc;
  a.g = blob_geom(shape->hidden, shape->inter, shape->group, shape->bits);
  a.experts = (const uint8_t*)experts;
  a.stride = stride;
  a.E = n_experts;
  a.k = k;
  a.n_tokens = n_tokens;
  a.idx = idx;
  a.w = weights;
  a.x = x;
  a.x_bf16 = x_is_bf16 != 0;
  a.out = hidden_out;
  a.err = h->err;
  a.trace = h->trace;
  a.gemm_path = h->prefill_gemm;
  a.shared = (const uint8_t*)shared_expert;
  a.sg = blob_geom(shape->hidden, shape->inter, shape->group, 4);
  a.shared_in_list = shared_expert && shape->bits == 4;
  a.gate = shared_expert ? shared_gate : nullptr;
  a.h_mid = h_mid;
  int n_cu = 0;
  if (hipDeviceGetAttribute(&n_cu, hipDeviceAttributeMultiprocessorCount, h->device) != hipSuccess || n_cu <= 0)
    return SMOE_ERR_HIP;
  return hip_status(launch_prefill(a, (uint32_t)n_cu, h->stream));
}

int smoe_synth_experts(smoe_handle* h, void* base, uint32_t n_experts, uint64_t stride,
                       const smoe_expert_shape* shape, uint64_t seed, float scale_sigma,
                       float bias_sigma) {
  if (!h || !base || !n_experts || !shape) return SMOE_ERR_INVALID_ARG;
  if (shape->bits != 4 && shape->bits != 3) return SMOE_ERR_UNSUPPORTED_BITS;
  if (!shape->group || shape->hidden % shape->group || shape->inter % shape->group)
    return SMOE_ERR_IN_DIM_NOT_MULTIPLE;
  if (stride < smoe_expert_bytes(shape)) return SMOE_ERR_INVALID_ARG;
  if (int rc = use_device(h)) return rc;
  const BlobGeom g = blob_geom(shape->hidden, shape->inter, shape->group, shape->bits);
  return hip_status(launch_synth_experts((uint8_t*)base, n_experts, stride, g, seed, scale_sigma,
                                         bias_sigma, h->stream));
}

int smoe_stream_read(smoe_handle* h, const void* buf, uint64_t bytes, uint32_t* sink) {
  if (!h || !buf || !bytes || !sink) return SMOE_ERR_INVALID_ARG;
  if (bytes % 16 || !aligned(buf, 0, 16)) return SMOE_ERR_MISALIGNED;
  if (int rc = use_device(h)) return rc;
  return hip_status(launch_stream_read(buf, bytes, sink, h->stream));
}

int smoe_synth_normal_f32(smoe_handle* h, float* out, uint64_t n, uint64_t seed, float sigma) {
  if (!h || !out || !n) return SMOE_ERR_INVALID_ARG;
  if (int rc = use_device(h)) return rc;
  return hip_status(launch_synth_normal_f32(out, n, seed, sigma, h->stream));
}

int smoe_synth_normal_bf16(smoe_handle* h, uint16_t* out, uint64_t n, uint64_t seed, float sigma) {
  if (!h || !out || !n) return SMOE_ERR_INVALID_ARG;
  if (int rc = use_device(h)) return rc;
  return hip_status(launch_synth_normal_bf16(out, n, seed, sigma, h->stream));
}

}  // extern "C"
