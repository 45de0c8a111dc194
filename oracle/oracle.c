/*
 * oracle.c — CPU restatement of the streamoe routed-expert hot path.
 *
 * TEST INFRASTRUCTURE ONLY (the parity checker and the CPU baseline);
 * never linked into the product. Built with -ffp-contract=off so that
 * every Rust `a * b + c` stays two roundings and every Rust `mul_add`
 * is the explicit fmaf() below. Citations: see oracle.h.
 *
 * Pinning (what checks each function against something other than
 * itself) is listed in tests/test_oracle.py; every function here has at
 * least one known-answer test, closed form or brute-force check.
 */
#include "oracle.h"

#include <math.h>
#include <pthread.h>
#include <stdlib.h>
#include <string.h>
#include <unistd.h>

/* ------------------------------------------------------------------ */
/* bf16: cpu_matvec.rs uses io/embedding.rs bf16_to_f32 (bits << 16);  */
/* the generators round to nearest even as                            */
/* crates/streammoe/tests/matvec_decode_bench.rs:36-39.               */
/* ------------------------------------------------------------------ */
float orc_bf16_to_f32(uint16_t b) {
  uint32_t u = (uint32_t)b << 16;
  float f;
  memcpy(&f, &u, 4);
  return f;
}

uint16_t orc_f32_to_bf16(float x) {
  uint32_t b;
  memcpy(&b, &x, 4);
  return (uint16_t)((b + (((b >> 16) & 1u) + 0x7fffu)) >> 16);
}

/* ------------------------------------------------------------------ */
/* Layout: variants.rs:401-486 (ExpertLayout) and :519-528            */
/* (expert_bytes). [gate | up | down], each [W | bf16 s | bf16 b].    */
/* ------------------------------------------------------------------ */
size_t orc_expert_bytes(uint32_t hidden, uint32_t inter, uint32_t bits, uint32_t group) {
  size_t weights = (size_t)inter * hidden * bits / 8;
  size_t scales = (size_t)inter * (hidden / group) * 2;
  return 3 * (weights + 2 * scales);
}

void orc_expert_offsets(uint32_t hidden, uint32_t inter, uint32_t bits, uint32_t group,
                        uint32_t block, uint64_t out_wsb[3]) {
  uint64_t weights = (uint64_t)inter * hidden * bits / 8;
  uint64_t scales = (uint64_t)inter * (hidden / group) * 2;
  uint64_t w = block * (weights + 2 * scales);
  out_wsb[0] = w;
  out_wsb[1] = w + weights;
  out_wsb[2] = w + weights + scales;
}

/* ------------------------------------------------------------------ */
/* Dequantized value: cpu_matvec.rs:164-165,                          */
/* `w = nibble.mul_add(scale, bias)` — one rounding.                  */
/* ------------------------------------------------------------------ */
void orc_dequant_4bit(const uint32_t* packed, const uint16_t* scales, const uint16_t* biases,
                      uint32_t in_dim, uint32_t out_dim, uint32_t group, float* w_out) {
  uint32_t in_packed = in_dim / 8, in_groups = in_dim / group;
  for (uint32_t r = 0; r < out_dim; ++r) {
    for (uint32_t c = 0; c < in_dim; ++c) {
      uint32_t word = packed[(size_t)r * in_packed + c / 8];
      float q = (float)((word >> ((c % 8) * 4)) & 0xFu);
      float s = orc_bf16_to_f32(scales[(size_t)r * in_groups + c / group]);
      float b = orc_bf16_to_f32(biases[(size_t)r * in_groups + c / group]);
      w_out[(size_t)r * in_dim + c] = fmaf(q, s, b);
    }
  }
}

/* 8-bit rows (cpu_matvec.rs:205-283's weight, before the multiply by x):
 * byte n of u32 word i is input 4i + n; w = fma(q, s, b). */
void orc_dequant_8bit(const uint32_t* packed, const uint16_t* scales, const uint16_t* biases,
                      uint32_t in_dim, uint32_t out_dim, uint32_t group, float* w_out) {
  uint32_t in_packed = in_dim / 4, in_groups = in_dim / group;
  for (uint32_t r = 0; r < out_dim; ++r) {
    for (uint32_t c = 0; c < in_dim; ++c) {
      uint32_t word = packed[(size_t)r * in_packed + c / 4];
      float q = (float)((word >> ((c % 4) * 8)) & 0xFFu);
      float s = orc_bf16_to_f32(scales[(size_t)r * in_groups + c / group]);
      float b = orc_bf16_to_f32(biases[(size_t)r * in_groups + c / group]);
      w_out[(size_t)r * in_dim + c] = fmaf(q, s, b);
    }
  }
}

/* ------------------------------------------------------------------ */
/* Row-parallel worker pool (rayon's par_iter_mut over output rows,    */
/* cpu_matvec.rs:150). Rows are independent, so the result does not   */
/* depend on the thread count.                                         */
/* ------------------------------------------------------------------ */
typedef void (*row_fn)(void* ctx, uint32_t r0, uint32_t r1);
typedef struct {
  row_fn fn;
  void* ctx;
  uint32_t r0, r1;
} row_job;

static int default_threads(void) {
  long n = sysconf(_SC_NPROCESSORS_ONLN);
  return n > 0 ? (int)n : 1;
}

/* A persistent pool (rayon keeps its workers alive between parallel     */
/* iterators): workers sleep on a condition variable between jobs; job  */
/* share t of `nthreads` goes to worker t - 1, share 0 to the caller.    */
typedef struct {
  row_fn fn;
  void* ctx;
  uint32_t rows;
  int nthreads;
} pool_job;

static pthread_mutex_t pool_call_mu = PTHREAD_MUTEX_INITIALIZER; /* one job at a time */
static pthread_mutex_t pool_mu = PTHREAD_MUTEX_INITIALIZER;
static pthread_cond_t pool_go = PTHREAD_COND_INITIALIZER;
static pthread_cond_t pool_done = PTHREAD_COND_INITIALIZER;
static int pool_workers = 0;
static uint64_t pool_gen = 0;
static int pool_pending = 0;
static pool_job pool_cur;

static void run_share(const pool_job* j, int t) {
  uint32_t per = (j->rows + j->nthreads - 1) / j->nthreads;
  uint32_t a = (uint32_t)t * per, b = a + per > j->rows ? j->rows : a + per;
  if (a < b) j->fn(j->ctx, a, b);
}

static void* pool_worker(void* arg) {
  int id = (int)(intptr_t)arg; /* runs share id + 1 */
  uint64_t seen = 0;
  for (;;) {
    pthread_mutex_lock(&pool_mu);
    while (pool_gen == seen) pthread_cond_wait(&pool_go, &pool_mu);
    seen = pool_gen;
    pool_job j = pool_cur;
    pthread_mutex_unlock(&pool_mu);
    if (id + 1 < j.nthreads) run_share(&j, id + 1);
    pthread_mutex_lock(&pool_mu);
    if (--pool_pending == 0) pthread_cond_signal(&pool_done);
    pthread_mutex_unlock(&pool_mu);
  }
  return NULL;
}

static void parallel_rows(row_fn fn, void* ctx, uint32_t rows, int nthreads) {
  if (nthreads <= 0) nthreads = default_threads();
  if ((uint32_t)nthreads > rows) nthreads = rows ? (int)rows : 1;
  if (nthreads <= 1) {
    fn(ctx, 0, rows);
    return;
  }
  pthread_mutex_lock(&pool_call_mu);
  pthread_mutex_lock(&pool_mu);
  while (pool_workers < nthreads - 1) {
    pthread_t th;
    if (pthread_create(&th, NULL, pool_worker, (void*)(intptr_t)pool_workers) != 0) break;
    pthread_detach(th);
    ++pool_workers;
  }
  if (nthreads - 1 > pool_workers) nthreads = pool_workers + 1;
  pool_cur.fn = fn;
  pool_cur.ctx = ctx;
  pool_cur.rows = rows;
  pool_cur.nthreads = nthreads;
  pool_pending = pool_workers;
  ++pool_gen;
  pthread_cond_broadcast(&pool_go);
  pthread_mutex_unlock(&pool_mu);
  run_share(&pool_cur, 0);
  pthread_mutex_lock(&pool_mu);
  while (pool_pending > 0) pthread_cond_wait(&pool_done, &pool_mu);
  pthread_mutex_unlock(&pool_mu);
  pthread_mutex_unlock(&pool_call_mu);
}

/* ------------------------------------------------------------------ */
/* dequant_matvec_4bit_gs_cpu: cpu_matvec.rs:95-173.                   */
/* Per row: acc = fma(fma(q, s, b), x, acc), input order, group by     */
/* group, word by word, nibble by nibble (low nibble first).           */
/* ------------------------------------------------------------------ */
typedef struct {
  const uint32_t* packed;
  const uint16_t* scales;
  const uint16_t* biases;
  uint32_t in_dim, group;
  const float* x;
  float* out;
} mv4_ctx;

static void mv4_rows(void* p, uint32_t r0, uint32_t r1) {
  const mv4_ctx* c = (const mv4_ctx*)p;
  uint32_t in_packed = c->in_dim / 8, in_groups = c->in_dim / c->group;
  uint32_t ppg = c->group / 8;
  for (uint32_t r = r0; r < r1; ++r) {
    const uint32_t* prow = c->packed + (size_t)r * in_packed;
    const uint16_t* srow = c->scales + (size_t)r * in_groups;
    const uint16_t* brow = c->biases + (size_t)r * in_groups;
    float acc = 0.0f;
    for (uint32_t g = 0; g < in_groups; ++g) {
      float scale = orc_bf16_to_f32(srow[g]);
      float bias = orc_bf16_to_f32(brow[g]);
      const uint32_t* gp = prow + (size_t)g * ppg;
      const float* xg = c->x + (size_t)g * c->group;
      for (uint32_t pp = 0; pp < ppg; ++pp) {
        uint32_t word = gp[pp];
        const float* xc = xg + pp * 8;
        for (uint32_t n = 0; n < 8; ++n) {
          float nib = (float)((word >> (n * 4)) & 0xFu);
          float w = fmaf(nib, scale, bias);
          acc = fmaf(w, xc[n], acc);
        }
      }
    }
    c->out[r] = acc;
  }
}

int orc_dequant_matvec_4bit_gs(const uint32_t* packed, const uint16_t* scales,
                               const uint16_t* biases, uint32_t in_dim, uint32_t out_dim,
                               uint32_t group, const float* x, float* out, int nthreads) {
  if (group == 0 || group % 8 != 0 || in_dim % group != 0) return ORC_ERR_IN_DIM_NOT_MULTIPLE;
  mv4_ctx c = {packed, scales, biases, in_dim, group, x, out};
  parallel_rows(mv4_rows, &c, out_dim, nthreads);
  return ORC_OK;
}

/* ------------------------------------------------------------------ */
/* dequant_matvec_8bit_gs_cpu: cpu_matvec.rs:205-283.                   */
/* Per row: acc = fma(fma(q, s, b), x, acc), input order, group by     */
/* group, word by word, byte by byte (byte n of word i = input 4i + n). */
/* ------------------------------------------------------------------ */
static void mv8_rows(void* p, uint32_t r0, uint32_t r1) {
  const mv4_ctx* c = (const mv4_ctx*)p;
  uint32_t in_packed = c->in_dim / 4, in_groups = c->in_dim / c->group;
  uint32_t ppg = c->group / 4;
  for (uint32_t r = r0; r < r1; ++r) {
    const uint32_t* prow = c->packed + (size_t)r * in_packed;
    const uint16_t* srow = c->scales + (size_t)r * in_groups;
    const uint16_t* brow = c->biases + (size_t)r * in_groups;
    float acc = 0.0f;
    for (uint32_t g = 0; g < in_groups; ++g) {
      float scale = orc_bf16_to_f32(srow[g]);
      float bias = orc_bf16_to_f32(brow[g]);
      const uint32_t* gp = prow + (size_t)g * ppg;
      const float* xg = c->x + (size_t)g * c->group;
      for (uint32_t pp = 0; pp < ppg; ++pp) {
        uint32_t word = gp[pp];
        const float* xc = xg + pp * 4;
        for (uint32_t n = 0; n < 4; ++n) {
          float byte = (float)((word >> (n * 8)) & 0xFFu);
          float w = fmaf(byte, scale, bias);
          acc = fmaf(w, xc[n], acc);
        }
      }
    }
    c->out[r] = acc;
  }
}

int orc_dequant_matvec_8bit_gs(const uint32_t* packed, const uint16_t* scales,
                               const uint16_t* biases, uint32_t in_dim, uint32_t out_dim,
                               uint32_t group, const float* x, float* out, int nthreads) {
  if (group == 0 || group % 4 != 0 || in_dim % group != 0) return ORC_ERR_IN_DIM_NOT_MULTIPLE;
  mv4_ctx c = {packed, scales, biases, in_dim, group, x, out};
  parallel_rows(mv8_rows, &c, out_dim, nthreads);
  return ORC_OK;
}

/* ------------------------------------------------------------------ */
/* lm_head_cpu: lm_head.rs:66-122 — the same arithmetic and order as   */
/* cpu_matvec.rs:150-171, single-threaded over rows.                   */
/* ------------------------------------------------------------------ */
int orc_lm_head(const uint32_t* packed, const uint16_t* scales, const uint16_t* biases,
                uint32_t hidden, uint32_t vocab, uint32_t group, const float* x, float* out) {
  if (group == 0 || group % 8 != 0 || hidden % group != 0) return ORC_ERR_IN_DIM_NOT_MULTIPLE;
  mv4_ctx c = {packed, scales, biases, hidden, group, x, out};
  mv4_rows(&c, 0, vocab);
  return ORC_OK;
}

/* ------------------------------------------------------------------ */
/* Router logits for an f32 router matrix: the arithmetic of           */
/* bf16_matvec_cpu (cpu_matvec.rs:318-357, `acc = w.mul_add(x[c], acc)` */
/* in column order) with f32 weights in place of bf16 ones.            */
/* ------------------------------------------------------------------ */
typedef struct {
  const float* w;
  uint32_t in_dim;
  const float* x;
  float* out;
} f32mv_ctx;

static void f32mv_rows(void* p, uint32_t r0, uint32_t r1) {
  const f32mv_ctx* c = (const f32mv_ctx*)p;
  for (uint32_t r = r0; r < r1; ++r) {
    const float* row = c->w + (size_t)r * c->in_dim;
    float acc = 0.0f;
    for (uint32_t i = 0; i < c->in_dim; ++i) acc = fmaf(row[i], c->x[i], acc);
    c->out[r] = acc;
  }
}

/* The same, rows in parallel (the reference's row-parallel matvecs,   */
/* cpu_matvec.rs:150); per-row arithmetic and order are unchanged.     */
void orc_f32_matvec_mt(const float* w, uint32_t in_dim, uint32_t out_dim, const float* x, float* out,
                       int nthreads) {
  f32mv_ctx c = {w, in_dim, x, out};
  parallel_rows(f32mv_rows, &c, out_dim, nthreads);
}

void orc_f32_matvec(const float* w, uint32_t in_dim, uint32_t out_dim, const float* x, float* out) {
  for (uint32_t r = 0; r < out_dim; ++r) {
    const float* row = w + (size_t)r * in_dim;
    float acc = 0.0f;
    for (uint32_t c = 0; c < in_dim; ++c) acc = fmaf(row[c], x[c], acc);
    out[r] = acc;
  }
}

/* Greedy argmax, first index wins on ties (strict >). */
uint32_t orc_argmax(const float* v, uint32_t n) {
  uint32_t best = 0;
  for (uint32_t i = 1; i < n; ++i)
    if (v[i] > v[best]) best = i;
  return best;
}

/* ------------------------------------------------------------------ */
/* 3-bit layout. pack_weights: tools/pack_experts.py:41-54 (8 codes per */
/* 3 bytes, code i at bits 3i..3i+3 of a little-endian 24-bit pack).   */
/* Returns nothing; codes above 7 are masked by the caller's contract.  */
/* ------------------------------------------------------------------ */
void orc_pack_3bit(const uint32_t* words4, size_t nwords, uint8_t* out3) {
  for (size_t i = 0; i < nwords; ++i) {
    uint32_t w = words4[i], p = 0;
    for (uint32_t j = 0; j < 8; ++j) p |= ((w >> (4 * j)) & 0xFu) << (3 * j);
    out3[3 * i + 0] = (uint8_t)(p & 0xFF);
    out3[3 * i + 1] = (uint8_t)((p >> 8) & 0xFF);
    out3[3 * i + 2] = (uint8_t)((p >> 16) & 0xFF);
  }
}

/* q3_expert_to_q4: moe_cpu.rs:227-245. Rewrites a packed 3-bit expert  */
/* into the 4-bit layout (same codes), scales and biases copied.         */
int orc_q3_expert_to_q4(const uint8_t* blob3, uint32_t hidden, uint32_t inter, uint32_t group,
                        uint8_t* blob4) {
  if (group == 0 || hidden % group != 0 || inter % group != 0) return ORC_ERR_IN_DIM_NOT_MULTIPLE;
  size_t w3 = (size_t)inter * hidden * 3 / 8, sb = (size_t)inter * (hidden / group) * 2;
  size_t blk3 = w3 + 2 * sb, w4 = (size_t)inter * hidden / 2, blk4 = w4 + 2 * sb;
  for (int block = 0; block < 3; ++block) {
    const uint8_t* src = blob3 + block * blk3;
    uint8_t* dst = blob4 + block * blk4;
    for (size_t p = 0; p < w3 / 3; ++p) {
      uint32_t v = (uint32_t)src[3 * p] | (uint32_t)src[3 * p + 1] << 8 |
                   (uint32_t)src[3 * p + 2] << 16;
      uint32_t w = 0;
      for (uint32_t i = 0; i < 8; ++i) w |= ((v >> (3 * i)) & 7u) << (4 * i);
      dst[4 * p + 0] = (uint8_t)(w & 0xFF);
      dst[4 * p + 1] = (uint8_t)((w >> 8) & 0xFF);
      dst[4 * p + 2] = (uint8_t)((w >> 16) & 0xFF);
      dst[4 * p + 3] = (uint8_t)((w >> 24) & 0xFF);
    }
    memcpy(dst + w4, src + w3, 2 * sb);
  }
  return ORC_OK;
}

/* ------------------------------------------------------------------ */
/* run_packed_expert_swiglu: moe_cpu.rs:178-220 (and the shared expert */
/* swiglu_ffn_4bit_cpu, mlp_cpu.rs:78-117): gate, up via the 4-bit      */
/* matvec; `silu = g / (1.0 + (-g).exp()); gate = silu * up`; down.     */
/* A 3-bit blob is first rewritten by q3_expert_to_q4, as the CPU       */
/* backend does (cpu_mod.rs:1147-1157).                                 */
/* ------------------------------------------------------------------ */
int orc_expert_swiglu(const uint8_t* blob, uint32_t bits, uint32_t hidden, uint32_t inter,
                      uint32_t group, const float* x, float* out, int nthreads) {
  if (bits != 4 && bits != 3) return ORC_ERR_BAD_BITS;
  if (group == 0 || group % 8 != 0 || hidden % group != 0 || inter % group != 0)
    return ORC_ERR_IN_DIM_NOT_MULTIPLE;
  uint8_t* tmp = NULL;
  if (bits == 3) {
    tmp = (uint8_t*)malloc(orc_expert_bytes(hidden, inter, 4, group));
    orc_q3_expert_to_q4(blob, hidden, inter, group, tmp);
    blob = tmp;
  }
  uint64_t o[3][3];
  for (uint32_t b = 0; b < 3; ++b) orc_expert_offsets(hidden, inter, 4, group, b, o[b]);
  float* gate = (float*)malloc(sizeof(float) * inter);
  float* up = (float*)malloc(sizeof(float) * inter);
#define W32(off) ((const uint32_t*)(blob + (off)))
#define B16(off) ((const uint16_t*)(blob + (off)))
  orc_dequant_matvec_4bit_gs(W32(o[0][0]), B16(o[0][1]), B16(o[0][2]), hidden, inter, group, x,
                             gate, nthreads);
  orc_dequant_matvec_4bit_gs(W32(o[1][0]), B16(o[1][1]), B16(o[1][2]), hidden, inter, group, x,
                             up, nthreads);
  for (uint32_t i = 0; i < inter; ++i) {
    float g = gate[i];
    float silu = g / (1.0f + expf(-g));
    gate[i] = silu * up[i];
  }
  orc_dequant_matvec_4bit_gs(W32(o[2][0]), B16(o[2][1]), B16(o[2][2]), inter, hidden, group, gate,
                             out, nthreads);
#undef W32
#undef B16
  free(gate);
  free(up);
  free(tmp);
  return ORC_OK;
}

/* ------------------------------------------------------------------ */
/* Router: moe_router.rs:52-181.                                       */
/* ------------------------------------------------------------------ */
/* softmax, moe_router.rs:52-72: max (strict >) -> exp(v - max) with a */
/* running sum in index order -> multiply by 1/sum.                     */
int orc_softmax(float* x, uint32_t n) {
  if (n == 0) return ORC_ERR_EMPTY;
  float max_val = x[0];
  for (uint32_t i = 1; i < n; ++i)
    if (x[i] > max_val) max_val = x[i];
  float sum = 0.0f;
  for (uint32_t i = 0; i < n; ++i) {
    x[i] = expf(x[i] - max_val);
    sum += x[i];
  }
  float inv_sum = 1.0f / sum;
  for (uint32_t i = 0; i < n; ++i) x[i] *= inv_sum;
  return ORC_OK;
}

/* Many independent softmax rows (x: rows x n), rows split over threads. */
typedef struct {
  float* x;
  uint32_t n;
} softmax_rows_ctx;

static void softmax_rows_fn(void* c, uint32_t a, uint32_t b) {
  softmax_rows_ctx* s = (softmax_rows_ctx*)c;
  for (uint32_t r = a; r < b; ++r) orc_softmax(s->x + (size_t)r * s->n, s->n);
}

int orc_softmax_rows(float* x, uint32_t rows, uint32_t n, int nthreads) {
  if (n == 0) return ORC_ERR_EMPTY;
  softmax_rows_ctx c = {x, n};
  parallel_rows(softmax_rows_fn, &c, rows, nthreads);
  return ORC_OK;
}

/* The libm expf the softmax calls (moe_router.rs:64), over a buffer in  */
/* blocks of 4096 values split over threads.                             */
typedef struct {
  const float* x;
  float* y;
  uint64_t n;
} expf_ctx;

static void expf_fn(void* c, uint32_t a, uint32_t b) {
  expf_ctx* e = (expf_ctx*)c;
  uint64_t lo = (uint64_t)a * 4096u, hi = (uint64_t)b * 4096u;
  if (hi > e->n) hi = e->n;
  for (uint64_t i = lo; i < hi; ++i) e->y[i] = expf(e->x[i]);
}

int orc_expf_many(const float* x, float* y, uint64_t n, int nthreads) {
  expf_ctx c = {x, y, n};
  parallel_rows(expf_fn, &c, (uint32_t)((n + 4095u) / 4096u), nthreads);
  return ORC_OK;
}

/* topk, moe_router.rs:83-124: slots start at (-1e30, 0); each score    */
/* replaces the running-minimum slot (lowest slot on ties) when strictly */
/* greater. Slot order is the replacement order.                         */
int orc_topk(const float* scores, uint32_t n, uint32_t k, int32_t* idx, float* val) {
  if (k == 0 || k > n) return ORC_ERR_BAD_K;
  for (uint32_t s = 0; s < k; ++s) {
    val[s] = -1e30f;
    idx[s] = 0;
  }
  for (uint32_t i = 0; i < n; ++i) {
    uint32_t min_k = 0;
    for (uint32_t s = 1; s < k; ++s)
      if (val[s] < val[min_k]) min_k = s;
    if (scores[i] > val[min_k]) {
      val[min_k] = scores[i];
      idx[min_k] = (int32_t)i;
    }
  }
  return ORC_OK;
}

/* normalize_weights, moe_router.rs:130-141: guarded w *= 1/sum.         */
void orc_normalize_weights(float* w, uint32_t k) {
  float sum = 0.0f;
  for (uint32_t i = 0; i < k; ++i) sum += w[i];
  if (sum > 0.0f) {
    float inv = 1.0f / sum;
    for (uint32_t i = 0; i < k; ++i) w[i] *= inv;
  }
}

/* moe_router_cpu_with, moe_router.rs:165-181.                           */
int orc_router(float* scores, uint32_t n, uint32_t k, int normalize, int32_t* idx, float* w) {
  int rc = orc_softmax(scores, n);
  if (rc) return rc;
  rc = orc_topk(scores, n, k, idx, w);
  if (rc) return rc;
  if (normalize) orc_normalize_weights(w, k);
  return ORC_OK;
}

/* cpu_sigmoid_scalar, cpu_ops.rs:22-25.                                 */
float orc_sigmoid(float x) { return 1.0f / (1.0f + expf(-x)); }

/* noaux_tc_router_cpu, moe_router.rs:211-330 (DeepSeek-V3 / Cogito-V2):  */
/*  1. scores = 1 / (1 + exp(-logit)) in place (the un-biased scores);    */
/*  2. biased = score + correction_bias (selection only);                 */
/*  3. group score = top1 + top2 of each group's biased values, by a      */
/*     linear scan (v > top1: shift; else v > top2);                      */
/*  4. topk() of the group scores picks topk_group groups;                */
/*  5. the other groups' biased values become -inf;                       */
/*  6. topk() of the masked biased values gives idx in slot order;        */
/*  7. w[s] = scores[idx[s]], summed in slot order, w *= 1/sum when       */
/*     sum > 0, then w *= routed_scaling_factor.                           */
int orc_noaux_tc_router(float* scores, const float* bias, uint32_t n, uint32_t n_group,
                        uint32_t topk_group, uint32_t k, float scale, int32_t* idx, float* w) {
  if (n == 0) return ORC_ERR_EMPTY;
  if (n_group == 0 || n % n_group) return ORC_ERR_BAD_K;
  if (topk_group == 0 || topk_group > n_group) return ORC_ERR_BAD_K;
  if (k == 0 || k > n) return ORC_ERR_BAD_K;
  for (uint32_t i = 0; i < n; ++i) scores[i] = 1.0f / (1.0f + expf(-scores[i]));
  float* biased = (float*)malloc((size_t)n * sizeof(float));
  float* gscore = (float*)malloc((size_t)n_group * sizeof(float));
  int32_t* gidx = (int32_t*)malloc((size_t)topk_group * sizeof(int32_t));
  float* gval = (float*)malloc((size_t)topk_group * sizeof(float));
  float* tval = (float*)malloc((size_t)k * sizeof(float));
  unsigned char* keep = (unsigned char*)calloc(n_group, 1);
  if (!biased || !gscore || !gidx || !gval || !tval || !keep) {
    free(biased), free(gscore), free(gidx), free(gval), free(tval), free(keep);
    return ORC_ERR_BAD_ARG;
  }
  for (uint32_t i = 0; i < n; ++i) biased[i] = scores[i] + bias[i];
  const uint32_t gs = n / n_group;
  for (uint32_t g = 0; g < n_group; ++g) {
    float top1 = -INFINITY, top2 = -INFINITY;
    for (uint32_t i = g * gs; i < (g + 1) * gs; ++i) {
      const float v = biased[i];
      if (v > top1) {
        top2 = top1;
        top1 = v;
      } else if (v > top2) {
        top2 = v;
      }
    }
    gscore[g] = top1 + top2;
  }
  int rc = orc_topk(gscore, n_group, topk_group, gidx, gval);
  if (rc == ORC_OK) {
    for (uint32_t s = 0; s < topk_group; ++s) keep[gidx[s]] = 1;
    for (uint32_t g = 0; g < n_group; ++g)
      if (!keep[g])
        for (uint32_t i = g * gs; i < (g + 1) * gs; ++i) biased[i] = -INFINITY;
    rc = orc_topk(biased, n, k, idx, tval);
  }
  if (rc == ORC_OK) {
    float sum = 0.0f;
    for (uint32_t s = 0; s < k; ++s) {
      w[s] = scores[idx[s]];
      sum += w[s];
    }
    if (sum > 0.0f) {
      const float inv = 1.0f / sum;
      for (uint32_t s = 0; s < k; ++s) w[s] *= inv;
    }
    for (uint32_t s = 0; s < k; ++s) w[s] *= scale;
  }
  free(biased), free(gscore), free(gidx), free(gval), free(tval), free(keep);
  return rc;
}

/* ------------------------------------------------------------------ */
/* cpu_combine: deferred.rs:441-490 (cpu_vec_madd, cpu_ops.rs:12-17):   */
/*   moe[i] = fma(out_k[i], w_k, moe[i])  for k in slot order;          */
/*   shared (sigmoid gate): s = fma(shared[i], sigmoid(score), moe[i]); */
/*   hidden = h_mid + s.   No shared expert: hidden = h_mid + moe.      */
/* A negative-infinity score is not special. An unscaled shared expert  */
/* (deepseek_moe_cpu, moe_cpu.rs:146-160: out += shared) is requested   */
/* with isnan(shared_gate_score).                                        */
/* ------------------------------------------------------------------ */
void orc_combine(const float* expert_out, const float* weights, uint32_t k, const float* h_mid,
                 const float* shared_out, float shared_gate_score, uint32_t dim,
                 float* hidden_out) {
  float* moe = (float*)calloc(dim, sizeof(float));
  for (uint32_t s = 0; s < k; ++s) {
    const float* e = expert_out + (size_t)s * dim;
    for (uint32_t i = 0; i < dim; ++i) moe[i] = fmaf(e[i], weights[s], moe[i]);
  }
  if (!shared_out) {
    for (uint32_t i = 0; i < dim; ++i) hidden_out[i] = h_mid[i] + moe[i];
  } else if (isnan(shared_gate_score)) {
    for (uint32_t i = 0; i < dim; ++i) hidden_out[i] = h_mid[i] + (moe[i] + shared_out[i]);
  } else {
    float sw = orc_sigmoid(shared_gate_score);
    for (uint32_t i = 0; i < dim; ++i) {
      float s = fmaf(shared_out[i], sw, moe[i]);
      hidden_out[i] = h_mid[i] + s;
    }
  }
  free(moe);
}

/* moe_combine_residual_n_tokens_cpu, backend/cpu/mod.rs:657-680, and   */
/* its no-shared sibling (682-695): per token t, g = sigmoid(gate[t])    */
/* (cpu_ops.rs:22-25), hidden = h_mid + moe_sum + g * shared_out,       */
/* evaluated left to right as Rust does: (h_mid + moe_sum) + (g * s),   */
/* no fused multiply-add. shared_out NULL: hidden = h_mid + moe_sum.    */
/* shared_gate NULL with shared_out: the shared term unscaled (g = 1).  */
void orc_moe_combine_residual_n_tokens(const float* h_mid, const float* moe_sum, const float* shared_out,
                                       const float* shared_gate, float* hidden_out, uint32_t n_tokens,
                                       uint32_t dim) {
  for (uint32_t t = 0; t < n_tokens; ++t) {
    const float g = shared_gate ? orc_sigmoid(shared_gate[t]) : 1.0f;
    for (uint32_t i = 0; i < dim; ++i) {
      const size_t idx = (size_t)t * dim + i;
      float v = h_mid[idx] + moe_sum[idx];
      if (shared_out) {
        const float gs = g * shared_out[idx];
        v = v + gs;
      }
      hidden_out[idx] = v;
    }
  }
}

/* ------------------------------------------------------------------ */
/* One decode layer, the per-token path (attn/linear_attn_forward.rs:  */
/* 2123-2170 then moe_dispatch_per_token) restated on the CPU — router */
/* logits (f32 matvec, or the 8-bit affine matvec of cpu_matvec.rs:    */
/* 205-283 for an 8-bit router), moe_router_cpu_with, the routed        */
/* experts (run_packed_expert_swiglu per slot), the shared expert and   */
/* its sigmoid gate (mlp_cpu.rs:78-117; gate logit = f32 dot or the     */
/* 8-bit matvec), then cpu_combine.                                     */
/* ------------------------------------------------------------------ */
int orc_moe_decode_layer(const orc_layer* L, const float* x, const float* h_mid,
                         float* hidden_out, int32_t* idx_out, float* w_out, float* logits_out,
                         int nthreads) {
  if (L->k == 0 || L->k > L->n_experts || L->k > 16) return ORC_ERR_BAD_K;
  uint32_t H = L->hidden;
  int rc0;
  float* scores = (float*)malloc(sizeof(float) * L->n_experts);
  if (L->router_q8) {
    rc0 = orc_dequant_matvec_8bit_gs((const uint32_t*)L->router_q8, L->router_s8, L->router_b8, H,
                                     L->n_experts, L->group8, x, scores, nthreads);
    if (rc0) {
      free(scores);
      return rc0;
    }
  } else {
    orc_f32_matvec_mt(L->router_w, H, L->n_experts, x, scores, nthreads);
  }
  if (logits_out) memcpy(logits_out, scores, sizeof(float) * L->n_experts);
  int rc = orc_router(scores, L->n_experts, L->k, L->normalize, idx_out, w_out);
  free(scores);
  if (rc) return rc;
  float* outs = (float*)malloc(sizeof(float) * H * L->k);
  for (uint32_t s = 0; s < L->k; ++s) {
    const uint8_t* blob = L->experts + (uint64_t)idx_out[s] * L->stride;
    rc = orc_expert_swiglu(blob, L->bits, H, L->inter, L->group, x, outs + (size_t)s * H,
                           nthreads);
    if (rc) {
      free(outs);
      return rc;
    }
  }
  float* shared = NULL;
  float score = NAN;
  if (L->shared_blob) {
    shared = (float*)malloc(sizeof(float) * H);
    orc_expert_swiglu(L->shared_blob, 4, H, L->shared_inter, L->group, x, shared, nthreads);
    if (L->gate_q8)
      orc_dequant_matvec_8bit_gs((const uint32_t*)L->gate_q8, L->gate_s8, L->gate_b8, H, 1, L->group8, x,
                                 &score, 1);
    else if (L->shared_gate_w)
      orc_f32_matvec(L->shared_gate_w, H, 1, x, &score);
  }
  orc_combine(outs, w_out, L->k, h_mid, shared, score, H, hidden_out);
  free(outs);
  free(shared);
  return ORC_OK;
}

/* ------------------------------------------------------------------ */
/* rms_norm_bf16_n_tokens_cpu, cpu_mod.rs:406-430 (one token):          */
/* sum_sq += x*x (two roundings), inv = 1/sqrt(sum_sq/dim + eps),       */
/* out = x * inv * w.                                                   */
/* ------------------------------------------------------------------ */
void orc_rms_norm_bf16(const float* x, const uint16_t* w, uint32_t dim, float eps, float* out) {
  float sum_sq = 0.0f;
  for (uint32_t i = 0; i < dim; ++i) sum_sq += x[i] * x[i];
  float inv_rms = 1.0f / sqrtf(sum_sq / (float)dim + eps);
  for (uint32_t i = 0; i < dim; ++i) out[i] = x[i] * inv_rms * orc_bf16_to_f32(w[i]);
}

/* ------------------------------------------------------------------ */
/* build_expert_buckets: moe_router.rs:374-436. CSR by expert: buckets */
/* ascending by expert id, empty ones omitted, tokens within a bucket  */
/* in (token, slot) order.                                              */
/* ------------------------------------------------------------------ */
int orc_build_expert_buckets(const int32_t* idx, const float* w, uint32_t n_tokens, uint32_t k,
                             uint32_t n_experts, int32_t* expert_ids, uint32_t* offsets,
                             int32_t* token_idx, float* weights, uint32_t* n_buckets) {
  uint32_t total = n_tokens * k;
  uint32_t* counts = (uint32_t*)calloc(n_experts ? n_experts : 1, sizeof(uint32_t));
  int32_t* e2b = (int32_t*)malloc(sizeof(int32_t) * (n_experts ? n_experts : 1));
  for (uint32_t i = 0; i < total; ++i) {
    if (idx[i] < 0 || (uint32_t)idx[i] >= n_experts) {
      free(counts);
      free(e2b);
      return ORC_ERR_BAD_ARG;
    }
    counts[idx[i]]++;
  }
  uint32_t nb = 0, running = 0;
  offsets[0] = 0;
  for (uint32_t e = 0; e < n_experts; ++e) {
    e2b[e] = -1;
    if (!counts[e]) continue;
    e2b[e] = (int32_t)nb;
    expert_ids[nb] = (int32_t)e;
    running += counts[e];
    offsets[++nb] = running;
  }
  uint32_t* cursors = (uint32_t*)malloc(sizeof(uint32_t) * (nb ? nb : 1));
  for (uint32_t b = 0; b < nb; ++b) cursors[b] = offsets[b];
  for (uint32_t t = 0; t < n_tokens; ++t) {
    for (uint32_t s = 0; s < k; ++s) {
      uint32_t flat = t * k + s;
      uint32_t b = (uint32_t)e2b[idx[flat]];
      uint32_t pos = cursors[b]++;
      token_idx[pos] = (int32_t)t;
      weights[pos] = w[flat];
    }
  }
  *n_buckets = nb;
  free(counts);
  free(e2b);
  free(cursors);
  return ORC_OK;
}

/* ------------------------------------------------------------------ */
/* moe_permute_fuse_cpu: moe_cpu.rs:282-339. For each bucket in order,  */
/* for each assignment: tmp = expert(x[token]); out[token][i] =         */
/* fma(tmp[i], w, out[token][i]). The caller zeroes out_sum. The expert */
/* FFNs are independent and computed in parallel first; the scatter-add */
/* then runs in the reference's bucket order.                           */
/* ------------------------------------------------------------------ */
typedef struct {
  const uint8_t* experts;
  uint64_t stride;
  uint32_t bits, hidden, inter, group;
  const float* x;
  const int32_t* slot_expert;
  const int32_t* token_idx;
  float* tmp;
} pf_ctx;

static void pf_rows(void* p, uint32_t a0, uint32_t a1) {
  const pf_ctx* c = (const pf_ctx*)p;
  for (uint32_t a = a0; a < a1; ++a) {
    const uint8_t* blob = c->experts + (uint64_t)c->slot_expert[a] * c->stride;
    orc_expert_swiglu(blob, c->bits, c->hidden, c->inter, c->group,
                      c->x + (size_t)c->token_idx[a] * c->hidden, c->tmp + (size_t)a * c->hidden,
                      1);
  }
}

int orc_moe_permute_fuse(const uint8_t* experts, uint64_t stride, uint32_t bits, uint32_t hidden,
                         uint32_t inter, uint32_t group, const float* x,
                         const int32_t* expert_ids, const uint32_t* offsets, uint32_t n_buckets,
                         const int32_t* token_idx, const float* weights, float* out_sum,
                         int nthreads) {
  if (bits != 4 && bits != 3) return ORC_ERR_BAD_BITS;
  uint32_t total = offsets[n_buckets];
  int32_t* slot_expert = (int32_t*)malloc(sizeof(int32_t) * (total ? total : 1));
  for (uint32_t b = 0; b < n_buckets; ++b)
    for (uint32_t s = offsets[b]; s < offsets[b + 1]; ++s) slot_expert[s] = expert_ids[b];
  float* tmp = (float*)malloc(sizeof(float) * (size_t)(total ? total : 1) * hidden);
  pf_ctx c = {experts, stride, bits, hidden, inter, group, x, slot_expert, token_idx, tmp};
  parallel_rows(pf_rows, &c, total, nthreads);
  for (uint32_t s = 0; s < total; ++s) {
    float* o = out_sum + (size_t)token_idx[s] * hidden;
    const float* t = tmp + (size_t)s * hidden;
    float wt = weights[s];
    for (uint32_t i = 0; i < hidden; ++i) o[i] = fmaf(t[i], wt, o[i]);
  }
  free(slot_expert);
  free(tmp);
  return ORC_OK;
}

/* ------------------------------------------------------------------ */
/* Test-input generator: the xorshift64* stream of the reference's     */
/* kernel tests (crates/streammoe/tests/packed_3bit.rs:21-31; identical */
/* in crates/streammoe-metal/tests/gather_mm_id_diff.rs:40-57). Writes  */
/* n outputs and returns the next state.                                */
/* ------------------------------------------------------------------ */
uint64_t orc_xorshift64s(uint64_t state, uint64_t* out, size_t n) {
  for (size_t i = 0; i < n; ++i) {
    state ^= state >> 12;
    state ^= state << 25;
    state ^= state >> 27;
    out[i] = state * 0x2545F4914F6CDD1Dull;
  }
  return state;
}
