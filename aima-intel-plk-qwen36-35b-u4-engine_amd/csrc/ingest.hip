// Weight ingestion on the device: layout conversions into (and out of) the
// boundary U4 layout, and the GGUF Q4_K unpack.
//
// Boundary layout of W[N][K] at group g (G = K / g): qweight u8[N][K/2] (low
// nibble = even k), scale f16[N][G], zp u4 over the flat [N*G] index (low
// nibble = even).  An OpenVINO IR U4 FC carries exactly this: u4 weight
// [N][G][g], f16 scale [N][G][1], u4 zero point [N][G][1]
// (tools/intel_qwen36_openvino_fixed_fc.py:107-144).  The reference's
// fixed-FC package stores scale and zero points group-major instead, [G][N]
// (tools/intel_qwen36_openvino_fixed_fc.py:218-265); the two conversions
// below move between the orders.  One thread per output element.
//
// Q4_K (GGUF): per row, super-blocks of 256 values in 144 bytes -- f16 d,
// f16 dmin, 12 bytes of packed 6-bit sub-block scales and mins, 128 bytes of
// codes; 64-value segment s holds its first 32 values in the low nibbles of
// bytes 32 s .. 32 s + 31 and the next 32 in the high nibbles; the value is
// d * sc_j * q - dmin * m_j for its 32-value sub-block j.  The unpack
// writes the codes in the boundary packing, f16(d * sc_j) as a group-32
// scale and dmin * m_j (f32) as a per-group min, the package the reference
// builds from a Q4_K tensor (tools/intel-qwen36-openvino-moe-micro-prepack.py:
// 76-124), here row-major like the boundary scale.
#include "common.h"

namespace aima {
namespace {

__global__ __launch_bounds__(256) void gm_to_rows_scale_kernel(const uint16_t* __restrict__ gm,
                                                               int64_t n, int64_t groups,
                                                               uint16_t* __restrict__ out) {
  const int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x;  // row-major index n * G + g
  if (i >= n * groups) return;
  const int64_t r = i / groups, g = i % groups;
  out[i] = gm[g * n + r];
}

__global__ __launch_bounds__(256) void rows_to_gm_scale_kernel(const uint16_t* __restrict__ rows,
                                                               int64_t n, int64_t groups,
                                                               uint16_t* __restrict__ out) {
  const int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x;  // group-major index g * N + r
  if (i >= n * groups) return;
  const int64_t g = i / n, r = i % n;
  out[i] = rows[r * groups + g];
}

__device__ __forceinline__ uint32_t nibble(const uint8_t* p, int64_t i) {
  return (p[i >> 1] >> ((i & 1) * 4)) & 0xfu;
}

// one thread per output byte (two nibbles)
template <bool TO_ROWS>
__global__ __launch_bounds__(256) void zp_order_kernel(const uint8_t* __restrict__ in, int64_t n,
                                                       int64_t groups, uint8_t* __restrict__ out) {
  const int64_t b = (int64_t)blockIdx.x * 256 + threadIdx.x;
  const int64_t total = n * groups;
  if (2 * b >= total) return;
  uint32_t v = 0;
#pragma unroll
  for (int h = 0; h < 2; ++h) {
    const int64_t i = 2 * b + h;
    if (i >= total) break;
    int64_t src;
    if (TO_ROWS) {
      const int64_t r = i / groups, g = i % groups;
      src = g * n + r;
    } else {
      const int64_t g = i / n, r = i % n;
      src = r * groups + g;
    }
    v |= nibble(in, src) << (4 * h);
  }
  out[b] = (uint8_t)v;
}

constexpr int kQ4KValues = 256;
constexpr int kQ4KBytes = 144;

// one thread per 32-value sub-block: 16 code bytes, one scale, one min
__global__ __launch_bounds__(256) void q4k_unpack_kernel(const uint8_t* __restrict__ blocks,
                                                         int64_t rows, int64_t cols,
                                                         uint8_t* __restrict__ qweight,
                                                         uint16_t* __restrict__ scale,
                                                         float* __restrict__ mins) {
  const int64_t t = (int64_t)blockIdx.x * 256 + threadIdx.x;
  const int64_t sub_per_row = cols / 32;
  if (t >= rows * sub_per_row) return;
  const int64_t r = t / sub_per_row;
  const int64_t js = t % sub_per_row;  // sub-block along the row
  const int64_t blk = js / 8;
  const int j = (int)(js % 8);
  const uint8_t* b = blocks + (r * (cols / kQ4KValues) + blk) * kQ4KBytes;
  const float d = h2f((uint16_t)(b[0] | (b[1] << 8)));
  const float dmin = h2f((uint16_t)(b[2] | (b[3] << 8)));
  const uint8_t* sc = b + 4;
  uint32_t s, m;
  if (j < 4) {
    s = sc[j] & 63u;
    m = sc[j + 4] & 63u;
  } else {
    s = (sc[j + 4] & 15u) | ((uint32_t)(sc[j - 4] >> 6) << 4);
    m = (uint32_t)(sc[j + 4] >> 4) | ((uint32_t)(sc[j] >> 6) << 4);
  }
  const uint8_t* qs = b + 16 + (j / 2) * 32;
  const int shift = (j & 1) * 4;
  uint8_t* dst = qweight + r * (cols / 2) + js * 16;
#pragma unroll
  for (int i = 0; i < 16; ++i) {
    const uint32_t lo = (qs[2 * i] >> shift) & 15u;
    const uint32_t hi = (qs[2 * i + 1] >> shift) & 15u;
    dst[i] = (uint8_t)(lo | (hi << 4));
  }
  // The f32 product is pinned in a register before the f16 rounding: left
  // alone, the compiler fuses convert-multiply-round into one mixed-precision
  // FMA with a +0 addend, which turns a -0 product (negative d, zero scale
  // code) into +0.
  float ds = d * (float)s;
  asm volatile("" : "+v"(ds));
  scale[t] = f2h(ds);
  mins[t] = dmin * (float)m;
}

unsigned grid_of(int64_t threads) { return (unsigned)((threads + 255) / 256); }

}  // namespace
}  // namespace aima

using namespace aima;

extern "C" int aima_u4_group_major_to_rows(const uint16_t* scale_gm, const uint8_t* zp_gm,
                                           int64_t n, int64_t groups, uint16_t* scale,
                                           uint8_t* zp, void* stream) {
  AIMA_REQUIRE(scale_gm && zp_gm && scale && zp, "u4_group_major_to_rows: null pointer");
  AIMA_REQUIRE(n > 0 && groups > 0, "u4_group_major_to_rows: n and groups must be positive");
  AIMA_REQUIRE((n * groups) % 2 == 0,
               "u4_group_major_to_rows: the group-major zero-point stream needs an even count");
  AIMA_REQUIRE(n * groups < ((int64_t)1 << 38), "u4_group_major_to_rows: too large");
  const hipStream_t st = (hipStream_t)stream;
  hipLaunchKernelGGL(gm_to_rows_scale_kernel, dim3(grid_of(n * groups)), dim3(256), 0, st,
                     scale_gm, n, groups, scale);
  hipLaunchKernelGGL(zp_order_kernel<true>, dim3(grid_of((n * groups + 1) / 2)), dim3(256), 0, st,
                     zp_gm, n, groups, zp);
  return launch_check("u4_group_major_to_rows");
}

extern "C" int aima_u4_rows_to_group_major(const uint16_t* scale, const uint8_t* zp, int64_t n,
                                           int64_t groups, uint16_t* scale_gm, uint8_t* zp_gm,
                                           void* stream) {
  AIMA_REQUIRE(scale && zp && scale_gm && zp_gm, "u4_rows_to_group_major: null pointer");
  AIMA_REQUIRE(n > 0 && groups > 0, "u4_rows_to_group_major: n and groups must be positive");
  AIMA_REQUIRE((n * groups) % 2 == 0,
               "u4_rows_to_group_major: the group-major zero-point stream needs an even count");
  AIMA_REQUIRE(n * groups < ((int64_t)1 << 38), "u4_rows_to_group_major: too large");
  const hipStream_t st = (hipStream_t)stream;
  hipLaunchKernelGGL(rows_to_gm_scale_kernel, dim3(grid_of(n * groups)), dim3(256), 0, st, scale,
                     n, groups, scale_gm);
  hipLaunchKernelGGL(zp_order_kernel<false>, dim3(grid_of((n * groups + 1) / 2)), dim3(256), 0,
                     st, zp, n, groups, zp_gm);
  return launch_check("u4_rows_to_group_major");
}

extern "C" int aima_q4k_unpack(const uint8_t* blocks, int64_t rows, int64_t cols,
                               uint8_t* qweight, uint16_t* scale, float* mins, void* stream) {
  AIMA_REQUIRE(blocks && qweight && scale && mins, "q4k_unpack: null pointer");
  AIMA_REQUIRE(rows > 0 && cols > 0 && cols % kQ4KValues == 0,
               "q4k_unpack: cols must be a positive multiple of 256");
  AIMA_REQUIRE(rows * (cols / 32) < ((int64_t)1 << 38), "q4k_unpack: too large");
  hipLaunchKernelGGL(q4k_unpack_kernel, dim3(grid_of(rows * (cols / 32))), dim3(256), 0,
                     (hipStream_t)stream, blocks, rows, cols, qweight, scale, mins);
  return launch_check("q4k_unpack");
}
