// U4 dequant, batch-1 U4 matvec, RMSNorm and router top-k for gfx950.  The
// matvec's block body (matvec_block) is in matvec_block.h.
#include "common.h"
#include "matvec_block.h"

#include <math.h>

namespace aima {

// ---------------------------------------------------------------------------
// dequant: out[n][k] = f32(q - z) * f32(s), one thread per 8 codes
// ---------------------------------------------------------------------------
__global__ __launch_bounds__(256) void u4_dequant_kernel(
    const uint32_t* __restrict__ qw, const uint16_t* __restrict__ scale,
    const uint8_t* __restrict__ zp, int64_t words, int64_t k, int group,
    float4* __restrict__ out) {
  const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (i >= words) return;
  const int64_t words_per_row = k / 8;
  const int64_t row = i / words_per_row;
  const int64_t k0 = (i % words_per_row) * 8;
  const int64_t groups = k / group;
  const int64_t gi = row * groups + k0 / group;
  const float s = h2f(scale[gi]);
  const int z = (int)u4_code(zp, gi);
  const uint32_t v = qw[i];
  float f[8];
#pragma unroll
  for (int j = 0; j < 8; ++j) f[j] = (float)((int)((v >> (4 * j)) & 0xfu) - z) * s;
  out[2 * i] = make_float4(f[0], f[1], f[2], f[3]);
  out[2 * i + 1] = make_float4(f[4], f[5], f[6], f[7]);
}

// ---------------------------------------------------------------------------
// f16 dequant: out[n][k] = f16(f32(q - z) * f32(s)), one thread per 8 codes,
// through dequant8 -- the operand the grouped GEMM feeds its MFMAs
// ---------------------------------------------------------------------------
__global__ __launch_bounds__(256) void u4_dequant_f16_kernel(
    const uint32_t* __restrict__ qw, const uint16_t* __restrict__ scale,
    const uint8_t* __restrict__ zp, int64_t words, int64_t k, int group,
    f16x8* __restrict__ out) {
  const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (i >= words) return;
  const int64_t words_per_row = k / 8;
  const int64_t row = i / words_per_row;
  const int64_t k0 = (i % words_per_row) * 8;
  const int64_t gi = row * (k / group) + k0 / group;
  out[i] = dequant8(qw[i], u4_zz2(u4_code(zp, gi)), u4_ss2(scale[gi]), u4_magic());
}

// Scale-and-min U4 rows (the Q4_K-derived form, groups of 32: one per
// 16-byte chunk): w = q * s - m with f16 s and f32 m per group, row-major
// [n][k/32] each.  y[n] = sum_g (s_g * sum q x - m_g * sum x) over the row's
// groups, the min applied to each group's activation sum as the reference's
// micro runtime applies it after its GEMM (openvino_moe_micro_runtime.cpp:
// 735-745, input_sums and mins).  Same block geometry and load order as
// matvec_block.
template <int KCH, int RG>
__device__ __forceinline__ void q4s_matvec_block(
    const uint16_t* __restrict__ x, const uint8_t* __restrict__ qw,
    const uint16_t* __restrict__ scale, const float* __restrict__ mins, int64_t n,
    void* __restrict__ y, int out_f32, int64_t blk) {
  using G = RowGeom<KCH>;
  constexpr int BR = 4 * RG * G::RPI;
  constexpr int kGroups = G::K / 32;  // groups (chunks) per row
  constexpr int kSW = (BR * kGroups / 2 + 255) / 256;
  constexpr int kMW = (BR * kGroups + 255) / 256;
  __shared__ __attribute__((aligned(16))) uint16_t s_lds[BR * kGroups];
  __shared__ __attribute__((aligned(16))) float m_lds[BR * kGroups];
  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = tid >> 6;
  const int seg = lane / G::SEG;
  const int cl = lane % G::SEG;
  const uint32_t magic = u4_magic();
  const int64_t brow0 = blk * BR;
  const int64_t row0 = brow0 + (int64_t)wave * (RG * G::RPI);
  const int64_t rows_here = n - brow0 < BR ? n - brow0 : BR;
  const int nsc = (int)rows_here * kGroups;
  const uint16_t* sblk = scale + brow0 * kGroups;
  const float* mblk = mins + brow0 * kGroups;
  const bool s_words = (reinterpret_cast<uintptr_t>(sblk) & 3u) == 0;
  const int s_full = s_words ? nsc / 2 : 0;
  uint32_t sw[kSW];
  float mw[kMW];
#pragma unroll
  for (int j = 0; j < kSW; ++j) {
    const int i = tid + 256 * j;
    sw[j] = i < s_full ? reinterpret_cast<const uint32_t*>(sblk)[i] : 0u;
  }
#pragma unroll
  for (int j = 0; j < kMW; ++j) {
    const int i = tid + 256 * j;
    mw[j] = i < nsc ? mblk[i] : 0.f;
  }
  u32x4 xr[G::NC][4];
  load_x_raw<KCH>(x, cl, xr);
  u32x4 w[RG][G::NC];
#pragma unroll
  for (int r = 0; r < RG; ++r) {
    const int64_t row = row0 + r * G::RPI + seg;
    const int64_t rowc = row < n ? row : n - 1;
#pragma unroll
    for (int i = 0; i < G::NC; ++i) {
      const int c = cl + i * G::SEG;
      w[r][i] = load16_nt(qw + rowc * (G::K / 2) + (int64_t)c * 16);
    }
  }
#pragma unroll
  for (int j = 0; j < kSW; ++j) {
    const int i = tid + 256 * j;
    if (i < s_full) reinterpret_cast<uint32_t*>(s_lds)[i] = sw[j];
  }
#pragma unroll
  for (int j = 0; j < kMW; ++j) {
    const int i = tid + 256 * j;
    if (i < nsc) m_lds[i] = mw[j];
  }
  for (int t = 2 * s_full + tid; t < nsc; t += 256) s_lds[t] = sblk[t];
  XChunk xc[G::NC];
  build_x_chunks<KCH>(xr, xc);
  __syncthreads();
#pragma unroll
  for (int r = 0; r < RG; ++r) {
    const int rl = wave * (RG * G::RPI) + r * G::RPI + seg;
    const int64_t row = brow0 + rl;
    float acc = 0.f;
#pragma unroll
    for (int i = 0; i < G::NC; ++i) {
      const int gi = rl * kGroups + cl + i * G::SEG;  // chunk c = group c
      const float sv = row < n ? h2f(s_lds[gi]) : 0.f;
      const float mv = row < n ? m_lds[gi] : 0.f;
      acc += u4_chunk_dot(w[r][i], xc[i], 0u, sv, magic) - mv * xc[i].xsum;
    }
    acc = segment_sum<G::SEG>(acc);
    if (cl == 0 && row < n) {
      if (out_f32) {
        reinterpret_cast<float*>(y)[row] = acc;
      } else {
        reinterpret_cast<uint16_t*>(y)[row] = f2h(acc);
      }
    }
  }
}

template <int KCH, int RG>
__global__ __launch_bounds__(256) void q4s_matvec_kernel(
    const uint16_t* __restrict__ x, const uint8_t* __restrict__ qw,
    const uint16_t* __restrict__ scale, const float* __restrict__ mins, int64_t n,
    void* __restrict__ y, int out_f32) {
  q4s_matvec_block<KCH, RG>(x, qw, scale, mins, n, y, out_f32, blockIdx.x);
}

template <int KCH, int RG>
__global__ __launch_bounds__(256) void u4_matvec_kernel(
    const uint16_t* __restrict__ x, const uint8_t* __restrict__ qw,
    const uint16_t* __restrict__ scale, const uint8_t* __restrict__ zp,
    int64_t n, int group_log2, void* __restrict__ y, int out_f32) {
  matvec_block<KCH, RG>(x, qw, scale, zp, n, group_log2, y, out_f32, blockIdx.x);
}

constexpr int kMaxMultiOut = AIMA_MAX_MULTI_OUT;

// Several matrices over one input x (the reference's multi-output fixed FC):
// block b belongs to the matrix whose block range holds it, so the pointer
// selection is uniform per block.
struct MultiMatvec {
  const uint8_t* qw[kMaxMultiOut];
  const uint16_t* scale[kMaxMultiOut];
  const uint8_t* zp[kMaxMultiOut];
  void* y[kMaxMultiOut];
  int64_t n[kMaxMultiOut];
  int32_t out_f32[kMaxMultiOut];
  int32_t first_block[kMaxMultiOut + 1];
  int32_t count;
};

template <int KCH, int RG>
__global__ __launch_bounds__(256) void u4_matvec_multi_kernel(const uint16_t* __restrict__ x,
                                                              MultiMatvec m, int group_log2) {
  const int b = blockIdx.x;
  int j = 0;
#pragma unroll
  for (int t = 1; t < kMaxMultiOut; ++t)
    if (t < m.count && b >= m.first_block[t]) j = t;
  matvec_block<KCH, RG>(x, m.qw[j], m.scale[j], m.zp[j], m.n[j], group_log2, m.y[j],
                        m.out_f32[j], b - m.first_block[j]);
}

template <int KCH>
static void launch_matvec(const uint16_t* x, const uint8_t* qw, const uint16_t* scale,
                          const uint8_t* zp, int64_t n, int glog2, void* y, int out_f32,
                          hipStream_t st) {
  // 8 row passes per wave (8 KB in flight per wave at K = 2048) once that
  // still leaves two blocks per CU; 4 below (measured at N = 248320: 13 %
  // faster than 4 passes, slower at 12 or 16)
  const int64_t rows8 = 4 * 8 * RowGeom<KCH>::RPI;
  if ((n + rows8 - 1) / rows8 >= 512) {
    hipLaunchKernelGGL((u4_matvec_kernel<KCH, 8>), dim3((unsigned)((n + rows8 - 1) / rows8)),
                       dim3(256), 0, st, x, qw, scale, zp, n, glog2, y, out_f32);
  } else {
    const int64_t rows4 = 4 * 4 * RowGeom<KCH>::RPI;
    hipLaunchKernelGGL((u4_matvec_kernel<KCH, 4>), dim3((unsigned)((n + rows4 - 1) / rows4)),
                       dim3(256), 0, st, x, qw, scale, zp, n, glog2, y, out_f32);
  }
}

template <int KCH>
static void launch_q4s_matvec(const uint16_t* x, const uint8_t* qw, const uint16_t* scale,
                              const float* mins, int64_t n, void* y, int out_f32,
                              hipStream_t st) {
  // the row-group rule of launch_matvec
  const int64_t rows8 = 4 * 8 * RowGeom<KCH>::RPI;
  if ((n + rows8 - 1) / rows8 >= 512) {
    hipLaunchKernelGGL((q4s_matvec_kernel<KCH, 8>), dim3((unsigned)((n + rows8 - 1) / rows8)),
                       dim3(256), 0, st, x, qw, scale, mins, n, y, out_f32);
  } else {
    const int64_t rows4 = 4 * 4 * RowGeom<KCH>::RPI;
    hipLaunchKernelGGL((q4s_matvec_kernel<KCH, 4>), dim3((unsigned)((n + rows4 - 1) / rows4)),
                       dim3(256), 0, st, x, qw, scale, mins, n, y, out_f32);
  }
}

// ---------------------------------------------------------------------------
// RMSNorm: one 256-thread block per row
// ---------------------------------------------------------------------------
__global__ __launch_bounds__(256) void rmsnorm_kernel(const uint16_t* __restrict__ x,
                                                      const float* __restrict__ weight,
                                                      int64_t hidden, float eps,
                                                      uint16_t* __restrict__ out) {
  __shared__ float red[4];
  const int64_t row = blockIdx.x;
  rmsnorm_row(x + row * hidden, weight, hidden, eps, out + row * hidden, red);
}

int rmsnorm_launch(const uint16_t* x, const float* weight, int64_t rows, int64_t hidden,
                   float eps, uint16_t* out, hipStream_t st) {
  AIMA_REQUIRE(hidden % 8 == 0 && aligned(x, 16) && aligned(out, 16),
               "rmsnorm: hidden must be a multiple of 8 and x, out 16-byte aligned");
  hipLaunchKernelGGL(rmsnorm_kernel, dim3((unsigned)rows), dim3(256), 0, st, x, weight, hidden,
                     eps, out);
  return launch_check("rmsnorm");
}

// ---------------------------------------------------------------------------
// Router top-k: one wave per token.  f64 softmax (gguf_loader.cpp:3646-3670),
// selection by (probability desc, id asc) (gguf_loader.cpp:3672-3697),
// renormalization by max(sum, min) in f32 (gguf_loader.cpp:3712-3731).
// ---------------------------------------------------------------------------
constexpr int kRouterMaxPerLane = 16;  // experts <= 1024

// PER = logits per lane (experts <= 64 PER); lane r keeps the rank-r pick in
// registers, and lane 0 sums the picks in rank order through shuffles.
template <int PER>
__global__ __launch_bounds__(256) void router_topk_kernel(
    const float* __restrict__ logits, int64_t tokens, int experts, int k,
    float min_weight_sum, int32_t* __restrict__ ids, float* __restrict__ weights,
    float* __restrict__ probs) {
  const int lane = threadIdx.x & 63;
  const int64_t token = (int64_t)blockIdx.x * 4 + (threadIdx.x >> 6);
  if (token >= tokens) return;
  int pick;
  float w, p;
  router_select_wave<PER>(logits + token * experts, experts, k, min_weight_sum, pick, w, p);
  if (lane < k) {
    ids[token * k + lane] = pick;
    weights[token * k + lane] = w;
    if (probs) probs[token * k + lane] = p;  // the picks' softmax probabilities
  }
}

static void launch_router_topk(const float* logits, int64_t tokens, int experts, int k,
                               float min_weight_sum, int32_t* ids, float* weights,
                               hipStream_t st, float* probs = nullptr) {
  const unsigned blocks = (unsigned)((tokens + 3) / 4);
  const int per = (experts + 63) / 64;
  if (per <= 1) {
    hipLaunchKernelGGL(router_topk_kernel<1>, dim3(blocks), dim3(256), 0, st, logits, tokens,
                       experts, k, min_weight_sum, ids, weights, probs);
  } else if (per <= 2) {
    hipLaunchKernelGGL(router_topk_kernel<2>, dim3(blocks), dim3(256), 0, st, logits, tokens,
                       experts, k, min_weight_sum, ids, weights, probs);
  } else if (per <= 4) {
    hipLaunchKernelGGL(router_topk_kernel<4>, dim3(blocks), dim3(256), 0, st, logits, tokens,
                       experts, k, min_weight_sum, ids, weights, probs);
  } else if (per <= 8) {
    hipLaunchKernelGGL(router_topk_kernel<8>, dim3(blocks), dim3(256), 0, st, logits, tokens,
                       experts, k, min_weight_sum, ids, weights, probs);
  } else {
    hipLaunchKernelGGL(router_topk_kernel<kRouterMaxPerLane>, dim3(blocks), dim3(256), 0, st,
                       logits, tokens, experts, k, min_weight_sum, ids, weights, probs);
  }
}

// probs (nullable): the picks' softmax probabilities before renormalization.
int router_topk_launch(const float* logits, int64_t tokens, int experts, int k,
                       float min_weight_sum, int32_t* ids, float* weights, hipStream_t st,
                       float* probs) {
  launch_router_topk(logits, tokens, experts, k, min_weight_sum, ids, weights, st, probs);
  return launch_check("router_topk");
}

int u4_matvec_dispatch(const uint16_t* x, const uint8_t* qw, const uint16_t* scale,
                       const uint8_t* zp, int64_t n, int64_t k, int glog2, void* y,
                       int out_f32, hipStream_t st) {
  switch (k) {
    case 128: launch_matvec<4>(x, qw, scale, zp, n, glog2, y, out_f32, st); break;
    case 256: launch_matvec<8>(x, qw, scale, zp, n, glog2, y, out_f32, st); break;
    case 512: launch_matvec<16>(x, qw, scale, zp, n, glog2, y, out_f32, st); break;
    case 1024: launch_matvec<32>(x, qw, scale, zp, n, glog2, y, out_f32, st); break;
    case 2048: launch_matvec<64>(x, qw, scale, zp, n, glog2, y, out_f32, st); break;
    case 4096: launch_matvec<128>(x, qw, scale, zp, n, glog2, y, out_f32, st); break;
    case 8192: launch_matvec<256>(x, qw, scale, zp, n, glog2, y, out_f32, st); break;
    default:
      return fail(AIMA_E_UNSUPPORTED, "u4_matvec: K must be a power of two in [128, 8192]");
  }
  return launch_check("u4_matvec");
}

template <int KCH>
static void launch_matvec_multi(const uint16_t* x, MultiMatvec m, int glog2, hipStream_t st) {
  // the single-matrix rule (8 row passes per wave once that still leaves
  // two blocks per CU) applied to the summed block count
  const int64_t rows8 = 4 * 8 * RowGeom<KCH>::RPI;
  int64_t blocks8 = 0;
  for (int j = 0; j < m.count; ++j) blocks8 += (m.n[j] + rows8 - 1) / rows8;
  const int rg = blocks8 >= 512 ? 8 : 4;
  const int64_t br = 4 * rg * RowGeom<KCH>::RPI;
  int64_t b = 0;
  for (int j = 0; j < m.count; ++j) {
    m.first_block[j] = (int32_t)b;
    b += (m.n[j] + br - 1) / br;
  }
  m.first_block[m.count] = (int32_t)b;
  if (rg == 8) {
    hipLaunchKernelGGL((u4_matvec_multi_kernel<KCH, 8>), dim3((unsigned)b), dim3(256), 0, st, x, m,
                       glog2);
  } else {
    hipLaunchKernelGGL((u4_matvec_multi_kernel<KCH, 4>), dim3((unsigned)b), dim3(256), 0, st, x, m,
                       glog2);
  }
}

static int u4_matvec_multi_dispatch(const uint16_t* x, const MultiMatvec& m, int64_t k, int glog2,
                                    hipStream_t st) {
  switch (k) {
    case 128: launch_matvec_multi<4>(x, m, glog2, st); break;
    case 256: launch_matvec_multi<8>(x, m, glog2, st); break;
    case 512: launch_matvec_multi<16>(x, m, glog2, st); break;
    case 1024: launch_matvec_multi<32>(x, m, glog2, st); break;
    case 2048: launch_matvec_multi<64>(x, m, glog2, st); break;
    case 4096: launch_matvec_multi<128>(x, m, glog2, st); break;
    case 8192: launch_matvec_multi<256>(x, m, glog2, st); break;
    default:
      return fail(AIMA_E_UNSUPPORTED, "u4_matvec_multi: K must be a power of two in [128, 8192]");
  }
  return launch_check("u4_matvec_multi");
}

int group_log2_of(int group) {
  switch (group) {
    case 32: return 5;
    case 64: return 6;
    case 128: return 7;
    case 256: return 8;
    default: return -1;
  }
}

}  // namespace aima

using namespace aima;

extern "C" int aima_u4_dequant(const uint8_t* qweight, const uint16_t* scale,
                               const uint8_t* zp, int64_t n, int64_t k, int32_t group,
                               float* out, void* stream) {
  AIMA_REQUIRE(qweight && scale && zp && out, "u4_dequant: null pointer");
  AIMA_REQUIRE(n > 0 && k > 0, "u4_dequant: n and k must be positive");
  AIMA_REQUIRE(group > 0 && group % 32 == 0 && k % group == 0,
               "u4_dequant: group must be a multiple of 32 dividing k");
  AIMA_REQUIRE(aligned(qweight, 4) && aligned(out, 16), "u4_dequant: misaligned pointer");
  const int64_t words = n * k / 8;
  const int64_t blocks = (words + 255) / 256;
  hipLaunchKernelGGL(u4_dequant_kernel, dim3((unsigned)blocks), dim3(256), 0,
                     (hipStream_t)stream, reinterpret_cast<const uint32_t*>(qweight),
                     scale, zp, words, k, (int)group, reinterpret_cast<float4*>(out));
  return launch_check("u4_dequant");
}

extern "C" int aima_u4_dequant_f16(const uint8_t* qweight, const uint16_t* scale,
                                   const uint8_t* zp, int64_t n, int64_t k, int32_t group,
                                   uint16_t* out, void* stream) {
  AIMA_REQUIRE(qweight && scale && zp && out, "u4_dequant_f16: null pointer");
  AIMA_REQUIRE(n > 0 && k > 0, "u4_dequant_f16: n and k must be positive");
  AIMA_REQUIRE(group > 0 && group % 32 == 0 && k % group == 0,
               "u4_dequant_f16: group must be a multiple of 32 dividing k");
  AIMA_REQUIRE(aligned(qweight, 4) && aligned(out, 16), "u4_dequant_f16: misaligned pointer");
  const int64_t words = n * k / 8;
  const int64_t blocks = (words + 255) / 256;
  hipLaunchKernelGGL(u4_dequant_f16_kernel, dim3((unsigned)blocks), dim3(256), 0,
                     (hipStream_t)stream, reinterpret_cast<const uint32_t*>(qweight),
                     scale, zp, words, k, (int)group, reinterpret_cast<f16x8*>(out));
  return launch_check("u4_dequant_f16");
}

extern "C" int aima_u4_matvec(const uint16_t* x, const uint8_t* qweight,
                              const uint16_t* scale, const uint8_t* zp, int64_t n,
                              int64_t k, int32_t group, void* y, int32_t out_dtype,
                              void* stream) {
  AIMA_REQUIRE(x && qweight && scale && zp && y, "u4_matvec: null pointer");
  AIMA_REQUIRE(n > 0, "u4_matvec: n must be positive");
  AIMA_REQUIRE(out_dtype == AIMA_OUT_F16 || out_dtype == AIMA_OUT_F32,
               "u4_matvec: out_dtype must be AIMA_OUT_F16 or AIMA_OUT_F32");
  const int glog2 = group_log2_of(group);
  AIMA_REQUIRE(glog2 > 0, "u4_matvec: group must be 32, 64, 128 or 256");
  AIMA_REQUIRE(k % group == 0, "u4_matvec: k must be a multiple of group");
  AIMA_REQUIRE(aligned(qweight, 16) && aligned(x, 16),
               "u4_matvec: qweight and x must be 16-byte aligned");
  return u4_matvec_dispatch(x, qweight, scale, zp, n, k, glog2, y, out_dtype,
                            (hipStream_t)stream);
}

extern "C" int aima_q4s_matvec(const uint16_t* x, const uint8_t* codes, const uint16_t* scale,
                               const float* mins, int64_t n, int64_t k, void* y,
                               int32_t out_dtype, void* stream) {
  AIMA_REQUIRE(x && codes && scale && mins && y, "q4s_matvec: null pointer");
  AIMA_REQUIRE(n > 0, "q4s_matvec: n must be positive");
  AIMA_REQUIRE(out_dtype == AIMA_OUT_F16 || out_dtype == AIMA_OUT_F32,
               "q4s_matvec: out_dtype must be AIMA_OUT_F16 or AIMA_OUT_F32");
  AIMA_REQUIRE(aligned(codes, 16) && aligned(x, 16) && aligned(mins, 4),
               "q4s_matvec: codes and x must be 16-byte aligned, mins 4-byte aligned");
  const hipStream_t st = (hipStream_t)stream;
  switch (k) {
    case 128: launch_q4s_matvec<4>(x, codes, scale, mins, n, y, out_dtype, st); break;
    case 256: launch_q4s_matvec<8>(x, codes, scale, mins, n, y, out_dtype, st); break;
    case 512: launch_q4s_matvec<16>(x, codes, scale, mins, n, y, out_dtype, st); break;
    case 1024: launch_q4s_matvec<32>(x, codes, scale, mins, n, y, out_dtype, st); break;
    case 2048: launch_q4s_matvec<64>(x, codes, scale, mins, n, y, out_dtype, st); break;
    case 4096: launch_q4s_matvec<128>(x, codes, scale, mins, n, y, out_dtype, st); break;
    case 8192: launch_q4s_matvec<256>(x, codes, scale, mins, n, y, out_dtype, st); break;
    default:
      return fail(AIMA_E_UNSUPPORTED, "q4s_matvec: K must be a power of two in [128, 8192]");
  }
  return launch_check("q4s_matvec");
}

extern "C" int aima_u4_matvec_multi(const uint16_t* x, int32_t count,
                                    const aima_u4_tensor* weights, const int64_t* n, int64_t k,
                                    int32_t group, void* const* y, const int32_t* out_dtype,
                                    void* stream) {
  AIMA_REQUIRE(x && weights && n && y && out_dtype, "u4_matvec_multi: null pointer");
  AIMA_REQUIRE(count >= 1 && count <= kMaxMultiOut,
               "u4_matvec_multi: count must be in [1, AIMA_MAX_MULTI_OUT]");
  const int glog2 = group_log2_of(group);
  AIMA_REQUIRE(glog2 > 0, "u4_matvec_multi: group must be 32, 64, 128 or 256");
  AIMA_REQUIRE(k % group == 0, "u4_matvec_multi: k must be a multiple of group");
  AIMA_REQUIRE(aligned(x, 16), "u4_matvec_multi: x must be 16-byte aligned");
  MultiMatvec m{};
  m.count = count;
  int64_t rows = 0;
  for (int j = 0; j < count; ++j) {
    const aima_u4_tensor& w = weights[j];
    AIMA_REQUIRE(w.qweight && w.scale && w.zp && y[j], "u4_matvec_multi: null output or tensor");
    AIMA_REQUIRE(aligned(w.qweight, 16), "u4_matvec_multi: qweight must be 16-byte aligned");
    AIMA_REQUIRE(n[j] > 0, "u4_matvec_multi: every n must be positive");
    AIMA_REQUIRE(out_dtype[j] == AIMA_OUT_F16 || out_dtype[j] == AIMA_OUT_F32,
                 "u4_matvec_multi: out_dtype must be AIMA_OUT_F16 or AIMA_OUT_F32");
    m.qw[j] = w.qweight;
    m.scale[j] = w.scale;
    m.zp[j] = w.zp;
    m.y[j] = y[j];
    m.n[j] = n[j];
    m.out_f32[j] = out_dtype[j] == AIMA_OUT_F32;
    rows += n[j];
  }
  AIMA_REQUIRE(rows < ((int64_t)1 << 31), "u4_matvec_multi: too many rows");
  return u4_matvec_multi_dispatch(x, m, k, glog2, (hipStream_t)stream);
}

extern "C" int aima_rmsnorm(const uint16_t* x, const float* weight, int64_t rows,
                            int64_t hidden, float eps, uint16_t* out, void* stream) {
  AIMA_REQUIRE(x && weight && out, "rmsnorm: null pointer");
  AIMA_REQUIRE(rows > 0 && hidden > 0, "rmsnorm: rows and hidden must be positive");
  AIMA_REQUIRE(rows <= 0x7fffffff, "rmsnorm: too many rows");
  return rmsnorm_launch(x, weight, rows, hidden, eps, out, (hipStream_t)stream);
}

extern "C" int aima_router_topk(const float* logits, int64_t tokens, int32_t experts,
                                int32_t k, float min_weight_sum, int32_t* ids,
                                float* weights, void* stream) {
  AIMA_REQUIRE(logits && ids && weights, "router_topk: null pointer");
  AIMA_REQUIRE(tokens > 0, "router_topk: tokens must be positive");
  AIMA_REQUIRE(experts > 0 && experts <= 64 * kRouterMaxPerLane,
               "router_topk: experts must be in [1, 1024]");
  AIMA_REQUIRE(k > 0 && k <= 16 && k <= experts, "router_topk: k must be in [1, min(16, experts)]");
  AIMA_REQUIRE(min_weight_sum > 0.f, "router_topk: minimum weight sum must be positive");
  launch_router_topk(logits, tokens, experts, k, min_weight_sum, ids, weights,
                     (hipStream_t)stream);
  return launch_check("router_topk");
}

extern "C" int aima_router_fc_topk(const uint16_t* h, const aima_u4_tensor* router,
                                   int32_t experts, int64_t hidden, int32_t group, int32_t k,
                                   float min_weight_sum, float* logits, int32_t* ids,
                                   float* weights, void* stream) {
  AIMA_REQUIRE(h && router && router->qweight && router->scale && router->zp && logits && ids &&
                   weights,
               "router_fc_topk: null pointer");
  AIMA_REQUIRE(experts > 0 && experts <= 64 * kRouterMaxPerLane,
               "router_fc_topk: experts must be in [1, 1024]");
  AIMA_REQUIRE(k > 0 && k <= 16 && k <= experts,
               "router_fc_topk: k must be in [1, min(16, experts)]");
  AIMA_REQUIRE(min_weight_sum > 0.f, "router_fc_topk: minimum weight sum must be positive");
  const int glog2 = group_log2_of(group);
  AIMA_REQUIRE(glog2 > 0, "router_fc_topk: group must be 32, 64, 128 or 256");
  AIMA_REQUIRE(hidden % group == 0, "router_fc_topk: hidden must be a multiple of group");
  AIMA_REQUIRE(aligned(router->qweight, 16) && aligned(h, 16),
               "router_fc_topk: qweight and h must be 16-byte aligned");
  const hipStream_t st = (hipStream_t)stream;
  const int rc = u4_matvec_dispatch(h, router->qweight, router->scale, router->zp, experts,
                                    hidden, glog2, logits, 1, st);
  if (rc != AIMA_OK) return rc;
  launch_router_topk(logits, 1, experts, k, min_weight_sum, ids, weights, st);
  return launch_check("router_fc_topk");
}
