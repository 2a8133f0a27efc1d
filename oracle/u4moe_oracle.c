/*
 * CPU oracle for the U4 MoE expert hot path -- TEST INFRASTRUCTURE ONLY.
 *
 * This file restates, in plain C, the reference engine's CPU arithmetic for
 * the quantized expert path so that the HIP kernels can be checked against
 * it.  Only tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg
 * may load it, and only as a checker / baseline: the product library never
 * calls into it and has no CPU fallback.
 *
 * Every function cites the reference file:line it follows.  Parity pinning:
 *   - f16 <-> f32 conversion, U4 unpack, U4 dequant: exhaustive tests.
 *   - softmax / top-k / normalize / select_router_topk / sigmoid / SwiGLU /
 *     expert weighting / aggregation / RMSNorm / F32 matvec / full MoE FFN
 *     layer: bit-exact against the reference's own gguf_loader.cpp compiled
 *     into oracle/_ref, plus the reference self-test known-answer values.
 *   - grouped schedule: invariants + brute force on small inputs.
 *
 * Floating point follows the reference build: ISO C, no FMA contraction
 * (the reference builds with -std=c++17 and CMAKE_CXX_EXTENSIONS OFF,
 * engine/CMakeLists.txt:9-11), sequential f32 sums, f64 softmax/sigmoid.
 */
#include <math.h>
#include <pthread.h>
#include <stdint.h>
#include <stdlib.h>
#include <string.h>

#define ORC_OK 0
#define ORC_EINVAL (-1)
#define ORC_ERANGE (-2)
#define ORC_ERUNTIME (-3)

/* ------------------------------------------------------------------------ */
/* half precision                                                            */
/* ------------------------------------------------------------------------ */

float orc_half_to_float(uint16_t h) {
  uint32_t sign = ((uint32_t)h & 0x8000u) << 16;
  uint32_t exp = ((uint32_t)h >> 10) & 0x1fu;
  uint32_t man = (uint32_t)h & 0x3ffu;
  uint32_t bits;
  if (exp == 0) {
    if (man == 0) {
      bits = sign;
    } else {
      int e = -1;
      do {
        ++e;
        man <<= 1;
      } while ((man & 0x400u) == 0);
      bits = sign | ((uint32_t)(127 - 15 - e) << 23) | ((man & 0x3ffu) << 13);
    }
  } else if (exp == 31) {
    bits = sign | 0x7f800000u | (man << 13);
  } else {
    bits = sign | ((exp + 112u) << 23) | (man << 13);
  }
  float f;
  memcpy(&f, &bits, sizeof(f));
  return f;
}

/* Round-to-nearest-even f32 -> f16 (the OpenCL convert_half_rte the reference
 * uses for its f16 outputs, iq36_fixed_fc_multi_output.cl:128,194). */
uint16_t orc_float_to_half(float f) {
  uint32_t x;
  memcpy(&x, &f, sizeof(x));
  uint32_t sign = (x >> 16) & 0x8000u;
  uint32_t ax = x & 0x7fffffffu;
  if (ax >= 0x7f800000u) {
    return (uint16_t)(sign | 0x7c00u | (ax > 0x7f800000u ? 0x200u : 0u));
  }
  if (ax >= 0x477ff000u) return (uint16_t)(sign | 0x7c00u);
  if (ax < 0x38800000u) {
    uint32_t e = ax >> 23;
    if (e < 102u) return (uint16_t)sign;
    uint32_t m = (ax & 0x7fffffu) | 0x800000u;
    uint32_t s = 126u - e;
    uint32_t q = m >> s;
    uint32_t rem = m & ((1u << s) - 1u);
    uint32_t half = 1u << (s - 1u);
    if (rem > half || (rem == half && (q & 1u))) ++q;
    return (uint16_t)(sign | q);
  }
  uint32_t q = (((ax >> 23) - 112u) << 10) | ((ax & 0x7fffffu) >> 13);
  uint32_t rem = ax & 0x1fffu;
  if (rem > 0x1000u || (rem == 0x1000u && (q & 1u))) ++q;
  return (uint16_t)(sign | q);
}

void orc_half_to_float_array(const uint16_t* in, int64_t n, float* out) {
  for (int64_t i = 0; i < n; ++i) out[i] = orc_half_to_float(in[i]);
}

void orc_float_to_half_array(const float* in, int64_t n, uint16_t* out) {
  for (int64_t i = 0; i < n; ++i) out[i] = orc_float_to_half(in[i]);
}

/* ------------------------------------------------------------------------ */
/* U4 group-quantized layout                                                 */
/*   qweight u8[N][K/2], low nibble = even k                                 */
/*   scale   f16[N][G], G = K/group                                          */
/*   zp      u4 packed over the flat [N*G] index, low nibble = even          */
/* Source: tools/intel_qwen36_openvino_fixed_fc.py:107-144,241-265 and       */
/* engine/openvino/custom/iq36_fixed_fc_multi_output.cl:118-127.             */
/* ------------------------------------------------------------------------ */

/* Nibble split: tools/intel_qwen36_openvino_fixed_fc.py:250-251. */
void orc_u4_unpack(const uint8_t* packed, int64_t byte_count, uint8_t* codes) {
  for (int64_t i = 0; i < byte_count; ++i) {
    codes[2 * i] = (uint8_t)(packed[i] & 0x0fu);
    codes[2 * i + 1] = (uint8_t)(packed[i] >> 4);
  }
}

static inline uint32_t u4_code(const uint8_t* packed, int64_t index) {
  uint8_t b = packed[index >> 1];
  return (index & 1) ? (uint32_t)(b >> 4) : (uint32_t)(b & 0x0fu);
}

/* Dequant w = f32(q - z) * f32(s): iq36_fixed_fc_multi_output.cl:125-127
 * (Convert -> Subtract(zp) -> Multiply(scale), fixed_fc.py:111-119). */
static inline float u4_weight(const uint8_t* qweight, const uint16_t* scale,
                              const uint8_t* zp, int64_t row, int64_t k,
                              int64_t K, int64_t groups, int64_t group) {
  const int64_t g = k / group;
  const uint32_t q = u4_code(qweight, row * K + k);
  const uint32_t z = u4_code(zp, row * groups + g);
  return (float)((int)q - (int)z) * orc_half_to_float(scale[row * groups + g]);
}

int orc_u4_dequant(const uint8_t* qweight, const uint16_t* scale,
                   const uint8_t* zp, int64_t n, int64_t k, int64_t group,
                   float* out) {
  if (n <= 0 || k <= 0 || group <= 0 || k % group != 0 || k % 2 != 0) {
    return ORC_EINVAL;
  }
  const int64_t groups = k / group;
  for (int64_t r = 0; r < n; ++r) {
    for (int64_t c = 0; c < k; ++c) {
      out[r * k + c] = u4_weight(qweight, scale, zp, r, c, k, groups, group);
    }
  }
  return ORC_OK;
}

/* ------------------------------------------------------------------------ */
/* Row-parallel driver: gguf_loader.cpp:513-544 parallel_for_rows (static    */
/* contiguous shards, one thread per shard).                                 */
/* ------------------------------------------------------------------------ */

typedef void (*orc_range_fn)(void* ctx, int64_t begin, int64_t end);

typedef struct {
  orc_range_fn fn;
  void* ctx;
  int64_t begin;
  int64_t end;
} orc_shard;

static void* orc_shard_main(void* arg) {
  orc_shard* s = (orc_shard*)arg;
  s->fn(s->ctx, s->begin, s->end);
  return NULL;
}

static void orc_parallel_for_rows(int64_t rows, int64_t threads,
                                  orc_range_fn fn, void* ctx) {
  if (rows <= 0) return;
  int64_t t = threads < 1 ? 1 : threads;
  if (t > rows) t = rows;
  if (t <= 1) {
    fn(ctx, 0, rows);
    return;
  }
  pthread_t* tid = (pthread_t*)malloc(sizeof(pthread_t) * (size_t)t);
  orc_shard* sh = (orc_shard*)malloc(sizeof(orc_shard) * (size_t)t);
  int64_t launched = 0;
  for (int64_t i = 0; i < t; ++i) {
    sh[i].fn = fn;
    sh[i].ctx = ctx;
    sh[i].begin = rows * i / t;
    sh[i].end = rows * (i + 1) / t;
    if (pthread_create(&tid[i], NULL, orc_shard_main, &sh[i]) == 0) {
      ++launched;
    } else {
      orc_shard_main(&sh[i]);
      tid[i] = 0;
    }
  }
  for (int64_t i = 0; i < t; ++i) {
    if (tid[i]) pthread_join(tid[i], NULL);
  }
  (void)launched;
  free(tid);
  free(sh);
}

/* ------------------------------------------------------------------------ */
/* U4 matvec: y[n] = sum_k w[n][k] * x[k], sequential f32 sum of products,   */
/* the F32 row dot of gguf_loader.cpp:2240-2246,2283-2293 applied to the     */
/* exact dequantized row.                                                    */
/* ------------------------------------------------------------------------ */

static float u4_row_dot(const uint8_t* qweight, const uint16_t* scale,
                        const uint8_t* zp, int64_t row, int64_t K,
                        int64_t group, const float* x) {
  const int64_t groups = K / group;
  float sum = 0.0f;
  for (int64_t k = 0; k < K; ++k) {
    const float w = u4_weight(qweight, scale, zp, row, k, K, groups, group);
    sum += w * x[k];
  }
  return sum;
}

typedef struct {
  const uint8_t* qweight;
  const uint16_t* scale;
  const uint8_t* zp;
  int64_t k;
  int64_t group;
  const float* x;
  float* y;
} matvec_ctx;

static void matvec_range(void* p, int64_t begin, int64_t end) {
  matvec_ctx* c = (matvec_ctx*)p;
  for (int64_t r = begin; r < end; ++r) {
    c->y[r] = u4_row_dot(c->qweight, c->scale, c->zp, r, c->k, c->group, c->x);
  }
}

int orc_u4_matvec(const uint8_t* qweight, const uint16_t* scale,
                  const uint8_t* zp, int64_t n, int64_t k, int64_t group,
                  const float* x, float* y, int64_t threads) {
  if (n <= 0 || k <= 0 || group <= 0 || k % group != 0 || k % 2 != 0) {
    return ORC_EINVAL;
  }
  matvec_ctx c = {qweight, scale, zp, k, group, x, y};
  orc_parallel_for_rows(n, threads, matvec_range, &c);
  return ORC_OK;
}

/* ------------------------------------------------------------------------ */
/* Router and MoE glue (gguf_loader.cpp:3368-3391, 3638-3819)                */
/* ------------------------------------------------------------------------ */

/* gguf_loader.cpp:3638-3644 */
float orc_sigmoid_scalar(float value) {
  const double x = value;
  const double r = x >= 0.0 ? 1.0 / (1.0 + exp(-x)) : exp(x) / (1.0 + exp(x));
  return (float)r;
}

/* gguf_loader.cpp:3646-3670: f64 exponentials against the max, f32 output. */
int orc_softmax(const float* logits, int64_t n, float* probs) {
  if (n <= 0) return ORC_EINVAL;
  int64_t max_i = 0;
  for (int64_t i = 1; i < n; ++i) {
    if (logits[i] > logits[max_i]) max_i = i; /* std::max_element: first max */
  }
  double* e = (double*)malloc(sizeof(double) * (size_t)n);
  double sum = 0.0;
  for (int64_t i = 0; i < n; ++i) {
    e[i] = exp((double)logits[i] - (double)logits[max_i]);
    sum += e[i];
  }
  if (sum == 0.0 || !isfinite(sum)) {
    free(e);
    return ORC_ERUNTIME;
  }
  for (int64_t i = 0; i < n; ++i) probs[i] = (float)(e[i] / sum);
  free(e);
  return ORC_OK;
}

/* gguf_loader.cpp:3672-3697: descending value, lower index on ties.  The
 * comparator is a strict weak order on (value desc, index asc), so the first
 * k of partial_sort are unique: a selection pass reproduces them. */
int orc_top_k(const float* values, int64_t n, int64_t k, int32_t* out) {
  if (k <= 0 || k > n) return ORC_EINVAL;
  unsigned char* used = (unsigned char*)calloc((size_t)n, 1);
  for (int64_t r = 0; r < k; ++r) {
    int64_t best = -1;
    for (int64_t i = 0; i < n; ++i) {
      if (used[i]) continue;
      if (best < 0) {
        best = i;
        continue;
      }
      const float v = values[i];
      const float b = values[best];
      /* comp(i, best): v == b ? i < best : v > b  (i > best here) */
      if (!(v == b) && v > b) best = i;
    }
    used[best] = 1;
    out[r] = (int32_t)best;
  }
  free(used);
  return ORC_OK;
}

/* gguf_loader.cpp:3712-3731 */
int orc_normalize_weights(const float* w, int64_t k, float min_weight_sum,
                          float* out) {
  if (k <= 0) return ORC_EINVAL;
  if (!(min_weight_sum > 0.0f)) return ORC_EINVAL;
  float sum = 0.0f;
  for (int64_t i = 0; i < k; ++i) sum += w[i];
  const float den = sum > min_weight_sum ? sum : min_weight_sum;
  for (int64_t i = 0; i < k; ++i) out[i] = w[i] / den;
  return ORC_OK;
}

/* gguf_loader.cpp:3733-3743 (select_router_topk), with kMinWeightSum
 * 6.103515625e-5 at the MoE layer call site (gguf_loader.cpp:5664-5665). */
int orc_select_router_topk(const float* logits, int64_t n, int64_t k,
                           float min_weight_sum, int32_t* ids, float* weights,
                           float* normalized) {
  if (n <= 0 || k <= 0 || k > n) return ORC_EINVAL;
  float* p = (float*)malloc(sizeof(float) * (size_t)n);
  int rc = orc_softmax(logits, n, p);
  if (rc == ORC_OK) rc = orc_top_k(p, n, k, ids);
  if (rc == ORC_OK) {
    for (int64_t i = 0; i < k; ++i) weights[i] = p[ids[i]];
    rc = orc_normalize_weights(weights, k, min_weight_sum, normalized);
  }
  free(p);
  return rc;
}

/* Router for many tokens: logits [T][n] -> ids [T][k], normalized [T][k]. */
int orc_router_topk_tokens(const float* logits, int64_t tokens, int64_t n,
                           int64_t k, float min_weight_sum, int32_t* ids,
                           float* normalized) {
  float* w = (float*)malloc(sizeof(float) * (size_t)k);
  int rc = ORC_OK;
  for (int64_t t = 0; t < tokens && rc == ORC_OK; ++t) {
    rc = orc_select_router_topk(logits + t * n, n, k, min_weight_sum,
                                ids + t * k, w, normalized + t * k);
  }
  free(w);
  return rc;
}

/* gguf_loader.cpp:3745-3761: f32 product with the f64 sigmoid. */
int orc_swiglu_pair(const float* gate, const float* up, int64_t n, float* out) {
  if (n <= 0) return ORC_EINVAL;
  for (int64_t i = 0; i < n; ++i) {
    const float g = gate[i];
    out[i] = g * orc_sigmoid_scalar(g) * up[i];
  }
  return ORC_OK;
}

/* gguf_loader.cpp:4640-4668: per expert, the first `inter` rows are gate,
 * the next `inter` rows are up; f64 arithmetic, cast once. */
int orc_swiglu_from_gate_up(const float* gate_up, int64_t inter,
                            int64_t experts, float* out) {
  if (inter <= 0 || experts <= 0) return ORC_EINVAL;
  for (int64_t e = 0; e < experts; ++e) {
    const float* base = gate_up + e * 2 * inter;
    for (int64_t r = 0; r < inter; ++r) {
      const double g = base[r];
      const double u = base[inter + r];
      const double s = g >= 0.0 ? 1.0 / (1.0 + exp(-g)) : exp(g) / (1.0 + exp(g));
      out[e * inter + r] = (float)(g * s * u);
    }
  }
  return ORC_OK;
}

/* gguf_loader.cpp:3773-3797 */
int orc_apply_expert_weights(const float* down, const float* w, int64_t experts,
                             int64_t hidden, float* out) {
  if (hidden <= 0 || experts <= 0) return ORC_EINVAL;
  for (int64_t e = 0; e < experts; ++e) {
    for (int64_t i = 0; i < hidden; ++i) {
      out[e * hidden + i] = down[e * hidden + i] * w[e];
    }
  }
  return ORC_OK;
}

/* gguf_loader.cpp:3799-3819: per element, sequential over experts. */
int orc_aggregate_experts(const float* weighted, int64_t experts,
                          int64_t hidden, float* out) {
  if (hidden <= 0 || experts <= 0) return ORC_EINVAL;
  for (int64_t i = 0; i < hidden; ++i) {
    float acc = 0.0f;
    for (int64_t e = 0; e < experts; ++e) acc += weighted[e * hidden + i];
    out[i] = acc;
  }
  return ORC_OK;
}

/* gguf_loader.cpp:3368-3391 */
int orc_rms_norm(const float* x, const float* weight, int64_t n, float eps,
                 float* out) {
  if (n <= 0) return ORC_EINVAL;
  float ss = 0.0f;
  for (int64_t i = 0; i < n; ++i) ss += x[i] * x[i];
  const float ms = ss / (float)n;
  const float scale = 1.0f / sqrtf(ms + eps);
  for (int64_t i = 0; i < n; ++i) out[i] = x[i] * scale * weight[i];
  return ORC_OK;
}

/* ------------------------------------------------------------------------ */
/* MoE FFN for one token (gguf_loader.cpp:5654-5782, the non-fused route     */
/* 5723-5737 + 5752-5780), with the router result as an input.               */
/* ------------------------------------------------------------------------ */

typedef struct {
  const uint8_t* qweight; /* [experts][rows][k/2] */
  const uint16_t* scale;  /* [experts][rows][k/group] */
  const uint8_t* zp;      /* [experts][rows*k/group/2] */
  int64_t rows;           /* rows per expert */
  int64_t k;
  int64_t group;
  int64_t experts;
} orc_u4_tensor;

typedef struct {
  orc_u4_tensor gate_up;        /* routed: rows = 2*inter, k = hidden */
  orc_u4_tensor down;           /* routed: rows = hidden,  k = inter  */
  orc_u4_tensor shared_gate_up; /* experts = 1 */
  orc_u4_tensor shared_down;    /* experts = 1 */
  const float* shared_gate_vec; /* [hidden], f32 values of the f16 vector */
  int64_t hidden;
  int64_t inter;
  int64_t shared_inter;
} orc_moe_weights;

static int tensor_ok(const orc_u4_tensor* t) {
  return t->qweight && t->scale && t->zp && t->rows > 0 && t->k > 0 &&
         t->group > 0 && t->k % t->group == 0 && t->k % 2 == 0 &&
         t->experts > 0 && (t->rows * (t->k / t->group)) % 2 == 0;
}

static void expert_matvec(const orc_u4_tensor* t, int64_t expert,
                          const float* x, float* y) {
  const int64_t groups = t->k / t->group;
  const uint8_t* qw = t->qweight + expert * t->rows * (t->k / 2);
  const uint16_t* sc = t->scale + expert * t->rows * groups;
  const uint8_t* zp = t->zp + expert * (t->rows * groups / 2);
  for (int64_t r = 0; r < t->rows; ++r) {
    y[r] = u4_row_dot(qw, sc, zp, r, t->k, t->group, x);
  }
}

typedef struct {
  float* gate_up;     /* [k][2*inter] */
  float* swiglu;      /* [k][inter] */
  float* down;        /* [k][hidden] */
  float* weighted;    /* [k][hidden] */
  float* moe_out;     /* [hidden] */
  float* shared_gate_up; /* [2*shared_inter] */
  float* shared_swiglu;  /* [shared_inter] */
  float* shared_down;    /* [hidden] */
  float shared_gate;
  float shared_gate_sigmoid;
  float* ffn_out;     /* [hidden] */
} orc_moe_scratch;

/* The routed half of the layer: s->moe_out = aggregate_experts(
 * apply_expert_weights(down_r(swiglu(gate_up_r x)), w)) -- the expert part of
 * run_qwen36_moe_ffn_layer (gguf_loader.cpp:5711-5738) and the output of the
 * reference's grouped prefill RunLayer (grouped_s8_u4_prefill_runtime.hpp:
 * 100-121, routed sum only). */
static int moe_routed_token(const orc_moe_weights* mw, const float* x,
                            const int32_t* ids, const float* w, int64_t k,
                            orc_moe_scratch* s) {
  const int64_t H = mw->hidden, I = mw->inter;
  for (int64_t r = 0; r < k; ++r) {
    if (ids[r] < 0 || ids[r] >= mw->gate_up.experts) return ORC_ERANGE;
  }
  for (int64_t r = 0; r < k; ++r) {
    expert_matvec(&mw->gate_up, ids[r], x, s->gate_up + r * 2 * I);
  }
  orc_swiglu_from_gate_up(s->gate_up, I, k, s->swiglu);
  for (int64_t r = 0; r < k; ++r) {
    expert_matvec(&mw->down, ids[r], s->swiglu + r * I, s->down + r * H);
  }
  orc_apply_expert_weights(s->down, w, k, H, s->weighted);
  orc_aggregate_experts(s->weighted, k, H, s->moe_out);
  return ORC_OK;
}

/* x: expert input (ffn_norm), f32 [hidden]; residual: f32 [hidden] or NULL
 * (then out = ffn_out).  ids/w: k selected experts and normalized weights. */
static int moe_ffn_token(const orc_moe_weights* mw, const float* x,
                         const float* residual, const int32_t* ids,
                         const float* w, int64_t k, float* out,
                         orc_moe_scratch* s) {
  const int64_t H = mw->hidden, IS = mw->shared_inter;
  const int rc = moe_routed_token(mw, x, ids, w, k, s);
  if (rc != ORC_OK) return rc;

  expert_matvec(&mw->shared_gate_up, 0, x, s->shared_gate_up);
  orc_swiglu_pair(s->shared_gate_up, s->shared_gate_up + IS, IS, s->shared_swiglu);
  expert_matvec(&mw->shared_down, 0, s->shared_swiglu, s->shared_down);
  float g = 0.0f;
  for (int64_t i = 0; i < H; ++i) g += mw->shared_gate_vec[i] * x[i];
  s->shared_gate = g;
  s->shared_gate_sigmoid = orc_sigmoid_scalar(g);
  for (int64_t i = 0; i < H; ++i) {
    const float shared_gated = s->shared_down[i] * s->shared_gate_sigmoid;
    s->ffn_out[i] = s->moe_out[i] + shared_gated;
    out[i] = residual ? residual[i] + s->ffn_out[i] : s->ffn_out[i];
  }
  return ORC_OK;
}

static int moe_weights_ok(const orc_moe_weights* mw) {
  if (!mw || !mw->shared_gate_vec) return 0;
  if (!tensor_ok(&mw->gate_up) || !tensor_ok(&mw->down) ||
      !tensor_ok(&mw->shared_gate_up) || !tensor_ok(&mw->shared_down)) {
    return 0;
  }
  const int64_t H = mw->hidden, I = mw->inter, IS = mw->shared_inter;
  return mw->gate_up.rows == 2 * I && mw->gate_up.k == H &&
         mw->down.rows == H && mw->down.k == I &&
         mw->down.experts == mw->gate_up.experts &&
         mw->shared_gate_up.rows == 2 * IS && mw->shared_gate_up.k == H &&
         mw->shared_down.rows == H && mw->shared_down.k == IS;
}

static int scratch_alloc(const orc_moe_weights* mw, int64_t k,
                         orc_moe_scratch* s) {
  const int64_t H = mw->hidden, I = mw->inter, IS = mw->shared_inter;
  memset(s, 0, sizeof(*s));
  s->gate_up = (float*)malloc(sizeof(float) * (size_t)(k * 2 * I));
  s->swiglu = (float*)malloc(sizeof(float) * (size_t)(k * I));
  s->down = (float*)malloc(sizeof(float) * (size_t)(k * H));
  s->weighted = (float*)malloc(sizeof(float) * (size_t)(k * H));
  s->moe_out = (float*)malloc(sizeof(float) * (size_t)H);
  s->shared_gate_up = (float*)malloc(sizeof(float) * (size_t)(2 * IS));
  s->shared_swiglu = (float*)malloc(sizeof(float) * (size_t)IS);
  s->shared_down = (float*)malloc(sizeof(float) * (size_t)H);
  s->ffn_out = (float*)malloc(sizeof(float) * (size_t)H);
  return s->gate_up && s->swiglu && s->down && s->weighted && s->moe_out &&
         s->shared_gate_up && s->shared_swiglu && s->shared_down && s->ffn_out;
}

static void scratch_free(orc_moe_scratch* s) {
  free(s->gate_up);
  free(s->swiglu);
  free(s->down);
  free(s->weighted);
  free(s->moe_out);
  free(s->shared_gate_up);
  free(s->shared_swiglu);
  free(s->shared_down);
  free(s->ffn_out);
}

/* One token with every intermediate exposed (used by the tests that compare
 * intermediates against the reference's Qwen36MoeFfnLayerResult fields,
 * gguf_loader.hpp:144-161). */
int orc_moe_ffn_token_detail(const orc_moe_weights* mw, const float* x,
                             const float* residual, const int32_t* ids,
                             const float* w, int64_t k, float* out,
                             float* gate_up, float* swiglu, float* down,
                             float* moe_out, float* shared_gate_up,
                             float* shared_swiglu, float* shared_down,
                             float* shared_gate_and_sigmoid, float* ffn_out) {
  if (!moe_weights_ok(mw) || k <= 0) return ORC_EINVAL;
  orc_moe_scratch s;
  if (!scratch_alloc(mw, k, &s)) {
    scratch_free(&s);
    return ORC_ERUNTIME;
  }
  int rc = moe_ffn_token(mw, x, residual, ids, w, k, out, &s);
  if (rc == ORC_OK) {
    const int64_t H = mw->hidden, I = mw->inter, IS = mw->shared_inter;
    if (gate_up) memcpy(gate_up, s.gate_up, sizeof(float) * (size_t)(k * 2 * I));
    if (swiglu) memcpy(swiglu, s.swiglu, sizeof(float) * (size_t)(k * I));
    if (down) memcpy(down, s.down, sizeof(float) * (size_t)(k * H));
    if (moe_out) memcpy(moe_out, s.moe_out, sizeof(float) * (size_t)H);
    if (shared_gate_up) {
      memcpy(shared_gate_up, s.shared_gate_up, sizeof(float) * (size_t)(2 * IS));
    }
    if (shared_swiglu) memcpy(shared_swiglu, s.shared_swiglu, sizeof(float) * (size_t)IS);
    if (shared_down) memcpy(shared_down, s.shared_down, sizeof(float) * (size_t)H);
    if (shared_gate_and_sigmoid) {
      shared_gate_and_sigmoid[0] = s.shared_gate;
      shared_gate_and_sigmoid[1] = s.shared_gate_sigmoid;
    }
    if (ffn_out) memcpy(ffn_out, s.ffn_out, sizeof(float) * (size_t)H);
  }
  scratch_free(&s);
  return rc;
}

typedef struct {
  const orc_moe_weights* mw;
  const float* x;        /* [T][H] */
  const float* residual; /* [T][H] or NULL */
  const int32_t* ids;    /* [T][k] */
  const float* w;        /* [T][k] */
  int64_t k;
  float* out;            /* [T][H] */
  int routed_only;       /* out = the routed sum only */
  int rc;
  pthread_mutex_t lock;
} tokens_ctx;

static void tokens_range(void* p, int64_t begin, int64_t end) {
  tokens_ctx* c = (tokens_ctx*)p;
  const int64_t H = c->mw->hidden;
  orc_moe_scratch s;
  int rc = ORC_OK;
  if (!scratch_alloc(c->mw, c->k, &s)) rc = ORC_ERUNTIME;
  for (int64_t t = begin; t < end && rc == ORC_OK; ++t) {
    if (c->routed_only) {
      rc = moe_routed_token(c->mw, c->x + t * H, c->ids + t * c->k, c->w + t * c->k, c->k, &s);
      if (rc == ORC_OK) memcpy(c->out + t * H, s.moe_out, sizeof(float) * (size_t)H);
    } else {
      rc = moe_ffn_token(c->mw, c->x + t * H,
                         c->residual ? c->residual + t * H : NULL,
                         c->ids + t * c->k, c->w + t * c->k, c->k,
                         c->out + t * H, &s);
    }
  }
  scratch_free(&s);
  if (rc != ORC_OK) {
    pthread_mutex_lock(&c->lock);
    if (c->rc == ORC_OK) c->rc = rc;
    pthread_mutex_unlock(&c->lock);
  }
}

/* T tokens, token-parallel.  Semantics of one grouped-prefill layer: every
 * token's output is the rank-ordered weighted aggregate of its experts plus
 * the gated shared expert (openvino_moe_micro_support.cl:154-172 for the
 * complete-FFN scatter; grouped_s8_u4_f16_contribution_moe.cl:847-861 for
 * the rank-ordered routed sum) with the CPU arithmetic above. */
int orc_moe_ffn_tokens(const orc_moe_weights* mw, int64_t tokens,
                       const float* x, const float* residual,
                       const int32_t* ids, const float* w, int64_t k,
                       float* out, int64_t threads) {
  if (!moe_weights_ok(mw) || k <= 0 || tokens < 0) return ORC_EINVAL;
  tokens_ctx c;
  c.mw = mw;
  c.x = x;
  c.residual = residual;
  c.ids = ids;
  c.w = w;
  c.k = k;
  c.out = out;
  c.routed_only = 0;
  c.rc = ORC_OK;
  pthread_mutex_init(&c.lock, NULL);
  orc_parallel_for_rows(tokens, threads, tokens_range, &c);
  pthread_mutex_destroy(&c.lock);
  return c.rc;
}

/* T tokens, routed sum only (RunLayer's f32 output), token-parallel. */
int orc_moe_routed_tokens(const orc_moe_weights* mw, int64_t tokens,
                          const float* x, const int32_t* ids, const float* w,
                          int64_t k, float* out, int64_t threads) {
  if (!moe_weights_ok(mw) || k <= 0 || tokens < 0) return ORC_EINVAL;
  tokens_ctx c;
  c.mw = mw;
  c.x = x;
  c.residual = NULL;
  c.ids = ids;
  c.w = w;
  c.k = k;
  c.out = out;
  c.routed_only = 1;
  c.rc = ORC_OK;
  pthread_mutex_init(&c.lock, NULL);
  orc_parallel_for_rows(tokens, threads, tokens_range, &c);
  pthread_mutex_destroy(&c.lock);
  return c.rc;
}

/* Single-token decode with row-parallel matvecs, the way the reference CPU
 * path parallelizes one token (parallel_for_rows per matvec call,
 * gguf_loader.cpp:513-544, 4361-4429).  Used as the CPU baseline. */
typedef struct {
  const orc_u4_tensor* t;
  int64_t expert;
  const float* x;
  float* y;
} expert_rows_ctx;

static void expert_rows_range(void* p, int64_t begin, int64_t end) {
  expert_rows_ctx* c = (expert_rows_ctx*)p;
  const orc_u4_tensor* t = c->t;
  const int64_t groups = t->k / t->group;
  const uint8_t* qw = t->qweight + c->expert * t->rows * (t->k / 2);
  const uint16_t* sc = t->scale + c->expert * t->rows * groups;
  const uint8_t* zp = t->zp + c->expert * (t->rows * groups / 2);
  for (int64_t r = begin; r < end; ++r) {
    c->y[r] = u4_row_dot(qw, sc, zp, r, t->k, t->group, c->x);
  }
}

static void expert_matvec_threaded(const orc_u4_tensor* t, int64_t expert,
                                   const float* x, float* y, int64_t threads) {
  expert_rows_ctx c = {t, expert, x, y};
  orc_parallel_for_rows(t->rows, threads, expert_rows_range, &c);
}

int orc_moe_ffn_decode_threaded(const orc_moe_weights* mw, const float* x,
                                const float* residual, const int32_t* ids,
                                const float* w, int64_t k, float* out,
                                int64_t threads) {
  if (!moe_weights_ok(mw) || k <= 0) return ORC_EINVAL;
  const int64_t H = mw->hidden, I = mw->inter, IS = mw->shared_inter;
  for (int64_t r = 0; r < k; ++r) {
    if (ids[r] < 0 || ids[r] >= mw->gate_up.experts) return ORC_ERANGE;
  }
  orc_moe_scratch s;
  if (!scratch_alloc(mw, k, &s)) {
    scratch_free(&s);
    return ORC_ERUNTIME;
  }
  for (int64_t r = 0; r < k; ++r) {
    expert_matvec_threaded(&mw->gate_up, ids[r], x, s.gate_up + r * 2 * I, threads);
  }
  orc_swiglu_from_gate_up(s.gate_up, I, k, s.swiglu);
  for (int64_t r = 0; r < k; ++r) {
    expert_matvec_threaded(&mw->down, ids[r], s.swiglu + r * I, s.down + r * H,
                           threads);
  }
  orc_apply_expert_weights(s.down, w, k, H, s.weighted);
  orc_aggregate_experts(s.weighted, k, H, s.moe_out);
  expert_matvec_threaded(&mw->shared_gate_up, 0, x, s.shared_gate_up, threads);
  orc_swiglu_pair(s.shared_gate_up, s.shared_gate_up + IS, IS, s.shared_swiglu);
  expert_matvec_threaded(&mw->shared_down, 0, s.shared_swiglu, s.shared_down,
                         threads);
  float g = 0.0f;
  for (int64_t i = 0; i < H; ++i) g += mw->shared_gate_vec[i] * x[i];
  const float sg = orc_sigmoid_scalar(g);
  for (int64_t i = 0; i < H; ++i) {
    const float ffn = s.moe_out[i] + s.shared_down[i] * sg;
    out[i] = residual ? residual[i] + ffn : ffn;
  }
  scratch_free(&s);
  return ORC_OK;
}

/* ------------------------------------------------------------------------ */
/* Grouped schedule: grouped_s8_u4_prefill_runtime.cpp:231-346               */
/* (BuildGroupedSchedule), generalised from the fixed 1024x8 shape to        */
/* T tokens x k ranks x E experts.  Rows within an expert are ordered by     */
/* (token, rank); offsets[e] is the exclusive END of expert e's rows, as in  */
/* the reference (:292-293).                                                 */
/* ------------------------------------------------------------------------ */

int orc_build_grouped_schedule(const int32_t* ids, int64_t tokens, int64_t k,
                               int64_t experts, const float* router_weights,
                               int32_t* offsets, int32_t* token_map,
                               int32_t* inverse_map, float* compact_weights,
                               int64_t* active_experts, int64_t* max_group) {
  if (tokens < 0 || k <= 0 || experts <= 0) return ORC_EINVAL;
  const int64_t A = tokens * k;
  int32_t* counts = (int32_t*)calloc((size_t)experts, sizeof(int32_t));
  int32_t* cursors = (int32_t*)calloc((size_t)experts, sizeof(int32_t));
  int rc = ORC_OK;
  for (int64_t t = 0; t < tokens && rc == ORC_OK; ++t) {
    for (int64_t r = 0; r < k; ++r) {
      const int32_t e = ids[t * k + r];
      if (e < 0 || e >= experts) {
        rc = ORC_ERANGE; /* "top-k expert is out of range" (:253-255) */
        break;
      }
      for (int64_t p = 0; p < r; ++p) {
        if (ids[t * k + p] == e) rc = ORC_ERANGE; /* duplicated (:256-260) */
      }
      if (rc != ORC_OK) break;
      ++counts[e];
    }
  }
  if (rc == ORC_OK) {
    int64_t cumulative = 0, active = 0, mx = 0;
    for (int64_t e = 0; e < experts; ++e) {
      cursors[e] = (int32_t)cumulative;
      active += counts[e] != 0;
      if (counts[e] > mx) mx = counts[e];
      cumulative += counts[e];
      offsets[e] = (int32_t)cumulative;
    }
    if (active_experts) *active_experts = active;
    if (max_group) *max_group = mx;
    for (int64_t i = 0; i < A; ++i) inverse_map[i] = -1;
    for (int64_t t = 0; t < tokens; ++t) {
      for (int64_t r = 0; r < k; ++r) {
        const int32_t e = ids[t * k + r];
        const int32_t row = cursors[e]++;
        token_map[row] = (int32_t)t;
        inverse_map[t * k + r] = row;
        if (compact_weights) compact_weights[row] = router_weights[t * k + r];
      }
    }
    for (int64_t i = 0; i < A; ++i) {
      if (inverse_map[i] < 0) rc = ORC_ERUNTIME; /* incomplete (:341-344) */
    }
  }
  free(counts);
  free(cursors);
  return rc;
}

/* ------------------------------------------------------------------------ */
/* Precision models of the stack (TEST INFRASTRUCTURE, not a parity          */
/* reference).  They recompute one layer with the rounding points and        */
/* summation orders of other correct implementations, so that a test can    */
/* measure how far two implementations of the 40-layer stack drift apart     */
/* through the f16 residual alone (the floor any end-to-end comparison with  */
/* the reference's order sits on).  Flags:                                   */
/*   ORC_MODEL_ACT_F16     SwiGLU outputs (routed and shared) rounded to f16 */
/*                         before the down matvec (the device operand)       */
/*   ORC_MODEL_SLICED      the persistent decode's order: P_x = w_x * d_x +  */
/*                         sigma * shared_down[:, slice x](act), x = 0..7,   */
/*                         out = residual + (P_0 + ... + P_7)                */
/*   ORC_MODEL_CHUNKED     every dot product as 32-element f32 chunk sums    */
/*                         combined by a pairwise tree (a different f32      */
/*                         order, like the device's lane partial sums)       */
/*   ORC_MODEL_WEIGHT_F16  dequantized weights rounded to f16 (the grouped   */
/*                         prefill's MFMA operand)                           */
/*   ORC_MODEL_CONTRIB_F16 the grouped prefill's combine: routed rows        */
/*                         f16(w_r * d_r), shared row f16(d_sh), f32 rank-   */
/*                         order sum, fma(shared, sigma, sum) + residual     */
/*   ORC_MODEL_F64         dot products, SwiGLU, weighting and sums in f64   */
/*                         (exact arithmetic up to the stack's own f16 h and */
/*                         r roundings)                                      */
/* With flags = 0 the result equals orc_moe_ffn_tokens bit for bit.          */
/* ------------------------------------------------------------------------ */

#define ORC_MODEL_ACT_F16 1
#define ORC_MODEL_SLICED 2
#define ORC_MODEL_CHUNKED 4
#define ORC_MODEL_WEIGHT_F16 8
#define ORC_MODEL_CONTRIB_F16 16
#define ORC_MODEL_F64 32

static double model_dot(const float* w, const double* x, int64_t n, int flags) {
  if (flags & ORC_MODEL_F64) {
    double s = 0.0;
    for (int64_t i = 0; i < n; ++i) s += (double)w[i] * x[i];
    return s;
  }
  if (flags & ORC_MODEL_CHUNKED) {
    float part[512];
    int64_t m = 0;
    for (int64_t c = 0; c < n; c += 32, ++m) {
      float s = 0.0f;
      for (int64_t i = c; i < c + 32 && i < n; ++i) s += w[i] * (float)x[i];
      part[m] = s;
    }
    while (m > 1) {
      int64_t h = (m + 1) / 2;
      for (int64_t i = 0; i < m / 2; ++i) part[i] = part[2 * i] + part[2 * i + 1];
      if (m & 1) part[m / 2] = part[m - 1];
      m = h;
    }
    return part[0];
  }
  float s = 0.0f;
  for (int64_t i = 0; i < n; ++i) s += w[i] * (float)x[i];
  return s;
}

static void model_row(const orc_u4_tensor* t, int64_t expert, int64_t row,
                      int flags, float* out) {
  const int64_t groups = t->k / t->group;
  const uint8_t* qw = t->qweight + expert * t->rows * (t->k / 2);
  const uint16_t* sc = t->scale + expert * t->rows * groups;
  const uint8_t* zp = t->zp + expert * (t->rows * groups / 2);
  for (int64_t k = 0; k < t->k; ++k) {
    float w = u4_weight(qw, sc, zp, row, k, t->k, groups, t->group);
    if (flags & ORC_MODEL_WEIGHT_F16) w = orc_half_to_float(orc_float_to_half(w));
    out[k] = w;
  }
}

static double model_swiglu(double g, double u, int flags) {
  const double s = g >= 0.0 ? 1.0 / (1.0 + exp(-g)) : exp(g) / (1.0 + exp(g));
  if (flags & ORC_MODEL_F64) return g * s * u;
  float a = (float)(g * s * u);
  if (flags & ORC_MODEL_ACT_F16) a = orc_half_to_float(orc_float_to_half(a));
  return a;
}

/* gate/up, SwiGLU and down of one expert: act [inter], d [hidden].  Values
 * are kept as double but hold f32 numbers unless ORC_MODEL_F64. */
static void model_expert(const orc_u4_tensor* gu, const orc_u4_tensor* dn,
                         int64_t e, const double* x, int flags, float* row,
                         double* act, double* d) {
  const int64_t I = gu->rows / 2, H = dn->rows;
  for (int64_t i = 0; i < I; ++i) {
    model_row(gu, e, i, flags, row);
    const double g = model_dot(row, x, gu->k, flags);
    model_row(gu, e, I + i, flags, row);
    const double u = model_dot(row, x, gu->k, flags);
    act[i] = model_swiglu(g, u, flags);
  }
  for (int64_t h = 0; h < H; ++h) {
    model_row(dn, e, h, flags, row);
    d[h] = model_dot(row, act, dn->k, flags);
  }
}

static int model_token(const orc_moe_weights* mw, const float* xf,
                       const float* residual, const int32_t* ids,
                       const float* w, int64_t k, int flags, float* out) {
  const int64_t H = mw->hidden, I = mw->inter, IS = mw->shared_inter;
  const int f64 = flags & ORC_MODEL_F64;
  for (int64_t r = 0; r < k; ++r) {
    if (ids[r] < 0 || ids[r] >= mw->gate_up.experts) return ORC_ERANGE;
  }
  int64_t kmax = H > I ? H : I;
  if (IS > kmax) kmax = IS;
  double* x = (double*)malloc(sizeof(double) * (size_t)H);
  float* row = (float*)malloc(sizeof(float) * (size_t)kmax);
  double* act = (double*)malloc(sizeof(double) * (size_t)(I > IS ? I : IS));
  double* d = (double*)malloc(sizeof(double) * (size_t)(k * H));
  double* dsh = (double*)malloc(sizeof(double) * (size_t)H);
  double* shs = (double*)malloc(sizeof(double) * (size_t)(8 * H));
  if (!x || !row || !act || !d || !dsh || !shs) {
    free(x); free(row); free(act); free(d); free(dsh); free(shs);
    return ORC_ERUNTIME;
  }
  for (int64_t i = 0; i < H; ++i) x[i] = xf[i];
  for (int64_t r = 0; r < k; ++r) {
    model_expert(&mw->gate_up, &mw->down, ids[r], x, flags, row, act, d + r * H);
  }
  /* shared expert: gate/up + SwiGLU, then its down matvec whole or per slice */
  for (int64_t i = 0; i < IS; ++i) {
    model_row(&mw->shared_gate_up, 0, i, flags, row);
    const double g = model_dot(row, x, H, flags);
    model_row(&mw->shared_gate_up, 0, IS + i, flags, row);
    const double u = model_dot(row, x, H, flags);
    if (f64) {
      act[i] = model_swiglu(g, u, flags);
    } else {
      /* the shared expert's f32 form (orc_swiglu_pair) */
      float a = (float)g * orc_sigmoid_scalar((float)g) * (float)u;
      if (flags & ORC_MODEL_ACT_F16) a = orc_half_to_float(orc_float_to_half(a));
      act[i] = a;
    }
  }
  const int64_t sl = IS / 8;
  for (int64_t h = 0; h < H; ++h) {
    model_row(&mw->shared_down, 0, h, flags, row);
    dsh[h] = model_dot(row, act, IS, flags);
    if ((flags & ORC_MODEL_SLICED) && sl > 0) {
      for (int64_t s = 0; s < 8; ++s) shs[s * H + h] = model_dot(row + s * sl, act + s * sl, sl, flags);
    }
  }
  double gsum = 0.0;
  float gf = 0.0f;
  for (int64_t i = 0; i < H; ++i) {
    gsum += (double)mw->shared_gate_vec[i] * x[i];
    gf += mw->shared_gate_vec[i] * xf[i];
  }
  const double sig = f64 ? (gsum >= 0.0 ? 1.0 / (1.0 + exp(-gsum)) : exp(gsum) / (1.0 + exp(gsum)))
                         : (double)orc_sigmoid_scalar(gf);
  for (int64_t h = 0; h < H; ++h) {
    const float res = residual ? residual[h] : 0.0f;
    if (f64) {
      double moe = 0.0;
      for (int64_t r = 0; r < k; ++r) moe += d[r * H + h] * (double)w[r];
      out[h] = (float)((double)res + (moe + dsh[h] * sig));
    } else if ((flags & ORC_MODEL_SLICED) && sl > 0) {
      float s = 0.0f;
      for (int64_t q = 0; q < 8; ++q) {
        float p = (float)sig * (float)shs[q * H + h];
        if (q < k) p = fmaf(w[q], (float)d[q * H + h], p);
        s += p;
      }
      out[h] = res + s;
    } else if (flags & ORC_MODEL_CONTRIB_F16) {
      float s = 0.0f;
      for (int64_t r = 0; r < k; ++r) {
        s += orc_half_to_float(orc_float_to_half((float)d[r * H + h] * w[r]));
      }
      const float o = fmaf(orc_half_to_float(orc_float_to_half((float)dsh[h])), (float)sig, s);
      out[h] = res + o;
    } else {
      float moe = 0.0f;
      for (int64_t r = 0; r < k; ++r) moe += (float)d[r * H + h] * w[r];
      const float ffn = moe + (float)dsh[h] * (float)sig;
      out[h] = residual ? res + ffn : ffn;
    }
  }
  free(x); free(row); free(act); free(d); free(dsh); free(shs);
  return ORC_OK;
}

typedef struct {
  const orc_moe_weights* mw;
  const float* x;
  const float* residual;
  const int32_t* ids;
  const float* w;
  int64_t k;
  int flags;
  float* out;
  int rc;
  pthread_mutex_t lock;
} model_ctx;

static void model_range(void* p, int64_t begin, int64_t end) {
  model_ctx* c = (model_ctx*)p;
  const int64_t H = c->mw->hidden;
  for (int64_t t = begin; t < end; ++t) {
    const int rc = model_token(c->mw, c->x + t * H, c->residual ? c->residual + t * H : NULL,
                               c->ids + t * c->k, c->w + t * c->k, c->k, c->flags,
                               c->out + t * H);
    if (rc != ORC_OK) {
      pthread_mutex_lock(&c->lock);
      if (c->rc == ORC_OK) c->rc = rc;
      pthread_mutex_unlock(&c->lock);
      return;
    }
  }
}

int orc_moe_ffn_tokens_model(const orc_moe_weights* mw, int64_t tokens,
                             const float* x, const float* residual,
                             const int32_t* ids, const float* w, int64_t k,
                             int flags, float* out, int64_t threads) {
  if (!moe_weights_ok(mw) || k <= 0 || k > 64 || tokens < 0) return ORC_EINVAL;
  if (mw->hidden > 16384 || mw->inter > 16384 || mw->shared_inter > 16384) return ORC_EINVAL;
  if ((flags & ORC_MODEL_SLICED) && (k > 8 || mw->shared_inter % 8 != 0)) return ORC_EINVAL;
  model_ctx c = {mw, x, residual, ids, w, k, flags, out, ORC_OK, PTHREAD_MUTEX_INITIALIZER};
  orc_parallel_for_rows(tokens, threads, model_range, &c);
  return c.rc;
}
