/* CPU baseline of the U4 MoE hot path -- TEST / MEASUREMENT INFRASTRUCTURE.
 *
 * Only bench.py's cpu_baseline leg loads this library: it times the
 * reference's CPU path on the GPU box's host cores beside the GPU numbers.
 * It is never part of the product path.  It is built on the machine that
 * runs it with -O3 -march=native (oracle/Makefile, target `baseline`).
 *
 * What it restates (the reference CPU ops, engine/src/gguf_loader.cpp):
 *   - the row-parallel matvec of matvec_tensor / matvec_expert_tensor
 *     (gguf_loader.cpp:513-544 thread pool, 4316-4465 expert matvec), here
 *     with OpenMP over rows and the U4 dequantization w = (q - z) * s folded
 *     per 128-wide group: y = sum_g s_g * (sum_k q_k x_k - z_g * sum_k x_k),
 *     which is the same sum reassociated so that the inner loop over the
 *     packed bytes vectorizes (scale and zero point hoisted per group);
 *   - the MoE FFN layer of run_qwen36_moe_ffn_layer (gguf_loader.cpp:
 *     5654-5782): RMSNorm, the k routed experts' gate/up matvecs, SwiGLU,
 *     down matvecs, rank-order weighted aggregate, the sigmoid-gated shared
 *     expert and the residual (softmax / sigmoid in f64 as the reference).
 * The bit-exact restatement used for parity is u4moe_oracle.c; this file
 * trades its summation order for speed and is checked against it to the
 * parity tolerance (tests/test_cpu_baseline.py).
 */
#include <math.h>
#include <omp.h>
#include <stdint.h>
#include <stdlib.h>
#include <string.h>

#define CPB_OK 0
#define CPB_EINVAL (-1)
#define CPB_ENOMEM (-2)

static int g_threads = 1;

int cpb_set_threads(int threads) {
  if (threads < 1) return CPB_EINVAL;
  g_threads = threads;
  omp_set_num_threads(threads);
  return CPB_OK;
}

int cpb_max_threads(void) { return omp_get_max_threads(); }

static inline float half_to_float(uint16_t h) {
  const uint32_t sign = (uint32_t)(h & 0x8000u) << 16;
  uint32_t exp = (h >> 10) & 0x1fu, man = h & 0x3ffu;
  uint32_t bits;
  if (exp == 0) {
    if (man == 0) {
      bits = sign;
    } else {  /* subnormal: normalize */
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
  memcpy(&f, &bits, 4);
  return f;
}

/* An input vector prepared once per matvec: for every 128-wide group the
 * even and odd elements (low and high nibbles of the packed bytes) and the
 * group sum. */
typedef struct {
  float* xe;    /* [k/2] even elements */
  float* xo;    /* [k/2] odd elements */
  float* gsum;  /* [k/group] */
} cpb_xprep;

static int xprep(const float* x, int64_t k, int64_t group, cpb_xprep* p) {
  p->xe = (float*)aligned_alloc(64, sizeof(float) * (size_t)((k / 2 + 15) / 16 * 16));
  p->xo = (float*)aligned_alloc(64, sizeof(float) * (size_t)((k / 2 + 15) / 16 * 16));
  p->gsum = (float*)malloc(sizeof(float) * (size_t)(k / group));
  if (!p->xe || !p->xo || !p->gsum) return CPB_ENOMEM;
  for (int64_t i = 0; i < k / 2; ++i) {
    p->xe[i] = x[2 * i];
    p->xo[i] = x[2 * i + 1];
  }
  for (int64_t g = 0; g < k / group; ++g) {
    float s = 0.f;
    for (int64_t i = 0; i < group; ++i) s += x[g * group + i];
    p->gsum[g] = s;
  }
  return CPB_OK;
}

static void xfree(cpb_xprep* p) {
  free(p->xe);
  free(p->xo);
  free(p->gsum);
}

/* One row: sum_g s_g * (sum q x - z_g * sum x) over the row's groups. */
static inline float row_dot(const uint8_t* restrict q, const uint16_t* restrict s,
                            const uint8_t* restrict zp, int64_t zbase, int64_t k,
                            int64_t group, const cpb_xprep* p) {
  const int64_t G = k / group, hb = group / 2;
  float acc = 0.f;
  for (int64_t g = 0; g < G; ++g) {
    const uint8_t* qb = q + g * hb;
    const float* xe = p->xe + g * hb;
    const float* xo = p->xo + g * hb;
    float a = 0.f;
#pragma omp simd reduction(+ : a)
    for (int64_t b = 0; b < hb; ++b) {
      a += (float)(qb[b] & 15) * xe[b] + (float)(qb[b] >> 4) * xo[b];
    }
    const int64_t zi = zbase + g;
    const float z = (float)((zp[zi >> 1] >> ((zi & 1) * 4)) & 15);
    acc += half_to_float(s[g]) * (a - z * p->gsum[g]);
  }
  return acc;
}

/* y[n] = W x for a U4 matrix [n][k] (f32 x and y). */
int cpb_u4_matvec(const uint8_t* qweight, const uint16_t* scale, const uint8_t* zp,
                  int64_t n, int64_t k, int64_t group, const float* x, float* y) {
  if (!qweight || !scale || !zp || !x || !y || n <= 0 || k <= 0 || group <= 0 ||
      k % group || group % 2) {
    return CPB_EINVAL;
  }
  cpb_xprep p;
  if (xprep(x, k, group, &p) != CPB_OK) {
    xfree(&p);
    return CPB_ENOMEM;
  }
  const int64_t G = k / group;
#pragma omp parallel for schedule(static) num_threads(g_threads)
  for (int64_t r = 0; r < n; ++r) {
    y[r] = row_dot(qweight + r * (k / 2), scale + r * G, zp, r * G, k, group, &p);
  }
  xfree(&p);
  return CPB_OK;
}

/* One MoE FFN layer's tensors for k selected experts (host copies):
 * gate_up[r] = expert r's [2I][H] (gate rows then up rows), down[r] =
 * [H][I]; slot k is the shared expert. */
typedef struct {
  const uint8_t* const* gu_q;
  const uint16_t* const* gu_s;
  const uint8_t* const* gu_z;
  const uint8_t* const* dn_q;
  const uint16_t* const* dn_s;
  const uint8_t* const* dn_z;
  const float* shared_gate_vec;  /* [H] */
  const float* norm_weight;      /* [H] */
  int64_t hidden, inter, group;
} cpb_layer;

static float sigmoid_d(double v) {
  return (float)(v >= 0.0 ? 1.0 / (1.0 + exp(-v)) : exp(v) / (1.0 + exp(v)));
}

/* r_out = r + moe(rmsnorm(r)) for one token, k routed experts + shared. */
int cpb_moe_layer_token(const cpb_layer* L, int64_t k, const float* w, float eps,
                        const float* r, float* r_out) {
  if (!L || !w || !r || !r_out || k <= 0) return CPB_EINVAL;
  const int64_t H = L->hidden, I = L->inter, group = L->group;
  const int64_t slots = k + 1;
  float* x = (float*)malloc(sizeof(float) * (size_t)H);
  float* gu = (float*)malloc(sizeof(float) * (size_t)(slots * 2 * I));
  float* act = (float*)malloc(sizeof(float) * (size_t)(slots * I));
  cpb_xprep px, pa[17];
  memset(pa, 0, sizeof(pa));
  int rc = (x && gu && act && slots <= 17) ? CPB_OK : CPB_ENOMEM;
  if (rc == CPB_OK) {
    double ss = 0.0;
    for (int64_t i = 0; i < H; ++i) ss += (double)r[i] * r[i];
    const float inv = 1.0f / sqrtf((float)(ss / (double)H) + eps);
    for (int64_t i = 0; i < H; ++i) x[i] = r[i] * inv * L->norm_weight[i];
    rc = xprep(x, H, group, &px);
  }
  if (rc == CPB_OK) {
    const int64_t G = H / group;
    /* gate/up of every slot, one parallel loop over all rows */
#pragma omp parallel for schedule(static) num_threads(g_threads)
    for (int64_t t = 0; t < slots * 2 * I; ++t) {
      const int64_t sl = t / (2 * I), row = t % (2 * I);
      gu[t] = row_dot(L->gu_q[sl] + row * (H / 2), L->gu_s[sl] + row * G, L->gu_z[sl], row * G,
                      H, group, &px);
    }
    for (int64_t sl = 0; sl < slots; ++sl) {
      for (int64_t j = 0; j < I; ++j) {
        const float g = gu[sl * 2 * I + j], u = gu[sl * 2 * I + I + j];
        act[sl * I + j] = (float)((double)g * (double)sigmoid_d(g) * (double)u);
      }
      if (xprep(act + sl * I, I, group, &pa[sl]) != CPB_OK) rc = CPB_ENOMEM;
    }
    double gd = 0.0;
    for (int64_t i = 0; i < H; ++i) gd += (double)L->shared_gate_vec[i] * x[i];
    const float sigma = sigmoid_d(gd);
    const int64_t GI = I / group;
    if (rc == CPB_OK) {
      /* down + rank-order aggregate + gated shared + residual, per row */
#pragma omp parallel for schedule(static) num_threads(g_threads)
      for (int64_t h = 0; h < H; ++h) {
        float moe = 0.f;
        for (int64_t sl = 0; sl < k; ++sl) {
          moe += w[sl] * row_dot(L->dn_q[sl] + h * (I / 2), L->dn_s[sl] + h * GI, L->dn_z[sl],
                                 h * GI, I, group, &pa[sl]);
        }
        const float sh = row_dot(L->dn_q[k] + h * (I / 2), L->dn_s[k] + h * GI, L->dn_z[k],
                                 h * GI, I, group, &pa[k]);
        r_out[h] = r[h] + (moe + sh * sigma);
      }
    }
    xfree(&px);
  }
  for (int64_t sl = 0; sl < 17; ++sl) xfree(&pa[sl]);
  free(x);
  free(gu);
  free(act);
  return rc;
}
