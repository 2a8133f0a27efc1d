// Shared device helpers for the gfx950 U4 MoE kernels.
#pragma once

#include <hip/hip_runtime.h>
#include <stddef.h>
#include <stdint.h>

#include <string>

#include "aima_u4moe.h"

typedef _Float16 f16x2 __attribute__((ext_vector_type(2)));
typedef _Float16 f16x8 __attribute__((ext_vector_type(8)));
typedef float f32x16 __attribute__((ext_vector_type(16)));
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
typedef uint32_t u32x2 __attribute__((ext_vector_type(2)));

namespace aima {

// ---------------------------------------------------------------------------
// host-side error state (thread-local message behind aima_last_error)
// ---------------------------------------------------------------------------
void set_error(const std::string& msg);
int fail(int code, const std::string& msg);
int hip_check(hipError_t e, const char* what);

#define AIMA_REQUIRE(cond, msg)                                   \
  do {                                                            \
    if (!(cond)) return ::aima::fail(AIMA_E_INVALID, (msg));      \
  } while (0)

#define AIMA_HIP(call)                                                  \
  do {                                                                  \
    int rc_ = ::aima::hip_check((call), #call);                         \
    if (rc_ != AIMA_OK) return rc_;                                     \
  } while (0)

inline bool aligned(const void* p, size_t a) {
  return (reinterpret_cast<uintptr_t>(p) % a) == 0;
}

inline bool is_pow2(int64_t v) { return v > 0 && (v & (v - 1)) == 0; }

// Every workspace starts with this header; the error word is the first u32.
constexpr size_t kWsHeader = 256;

inline size_t round_up(size_t v, size_t a) { return (v + a - 1) / a * a; }

// Launch status check after a kernel launch.
int launch_check(const char* what);

// log2 of a supported group size (32, 64, 128, 256), else -1.
int group_log2_of(int group);

// Gate and up projections of an expert stack in either boundary form:
//   concatenated: gate_up = E x [2I][H], up rows after the gate rows (the CPU
//                 reference's convention, engine/src/gguf_loader.cpp:4654-4660);
//   split:        gate = E x [I][H] and up = E x [I][H] (the OpenVINO
//                 MOE3GemmFusedCompressed operands,
//                 engine/openvino/iq36-fixed-fc-moe-router-compat.patch:49-56),
//                 selected by a non-null up.qweight.
// Projection h (0 gate, 1 up) of unit j of expert e is row row(e, h, j) of
// tensor h; its scales and zero points are at the same flat row index.
struct GateUpView {
  const uint8_t* q[2];
  const uint16_t* s[2];
  const uint8_t* z[2];
  int64_t expert_rows;  // rows per expert in each tensor (2I or I)
  int64_t up_row0;      // first up row of an expert in tensor 1 (I or 0)
  __host__ __device__ int64_t row(int64_t e, int h, int64_t j) const {
    return e * expert_rows + (h ? up_row0 : 0) + j;
  }
};

__host__ __device__ inline GateUpView gate_up_view(const aima_u4_tensor& gate_up, const aima_u4_tensor& up,
                               int64_t inter) {
  GateUpView v;
  const bool split = up.qweight != nullptr;
  v.q[0] = gate_up.qweight;
  v.s[0] = gate_up.scale;
  v.z[0] = gate_up.zp;
  v.q[1] = split ? up.qweight : gate_up.qweight;
  v.s[1] = split ? up.scale : gate_up.scale;
  v.z[1] = split ? up.zp : gate_up.zp;
  v.expert_rows = split ? inter : 2 * inter;
  v.up_row0 = split ? 0 : inter;
  return v;
}
__host__ __device__ inline GateUpView routed_gate_up(const aima_moe_layer& L) {
  return gate_up_view(L.gate_up, L.up, L.inter);
}
__host__ __device__ inline GateUpView shared_gate_up(const aima_moe_layer& L) {
  return gate_up_view(L.shared_gate_up, L.shared_up, L.shared_inter);
}
// Null checks and qweight alignment of the optional split up tensors.
inline bool split_tensors_ok(const aima_moe_layer& L) {
  auto ok = [](const aima_u4_tensor& t) {
    return t.qweight == nullptr ? (t.scale == nullptr && t.zp == nullptr)
                                : (t.scale != nullptr && t.zp != nullptr && aligned(t.qweight, 16));
  };
  return ok(L.up) && ok(L.shared_up);
}

// ---------------------------------------------------------------------------
// device helpers
// ---------------------------------------------------------------------------
// Bit casts take their operand by value: __builtin_bit_cast applied directly
// to an element of an ext_vector_type (v[i]) reads element 0 with this
// compiler, so vector elements always pass through one of these helpers.
__device__ __forceinline__ f16x2 as_h2(uint32_t v) {
  return __builtin_bit_cast(f16x2, v);
}
__device__ __forceinline__ float as_f32(uint32_t v) {
  return __builtin_bit_cast(float, v);
}
__device__ __forceinline__ uint32_t h2_bits(f16x2 v) {
  return __builtin_bit_cast(uint32_t, v);
}
__device__ __forceinline__ float h2f(uint16_t b) {
  return (float)__builtin_bit_cast(_Float16, b);
}
// f32 -> f16 round to nearest even (v_cvt_f16_f32 in the default mode).
__device__ __forceinline__ uint16_t f2h(float f) {
  return __builtin_bit_cast(uint16_t, (_Float16)f);
}
// Two floats -> f16x2 bits (lo in bits 0..15), round to nearest even: one
// v_cvt_pk_f16_f32 on gfx950.
__device__ __forceinline__ uint32_t pack_h2(float lo, float hi) {
  typedef float f32x2_t __attribute__((ext_vector_type(2)));
  return __builtin_bit_cast(uint32_t, __builtin_convertvector((f32x2_t{lo, hi}), f16x2));
}

__device__ __forceinline__ uint32_t u4_code(const uint8_t* packed, int64_t i) {
  const uint32_t b = packed[i >> 1];
  return (i & 1) ? (b >> 4) : (b & 0x0fu);
}

// Sums over aligned lane segments with DPP (register-to-register lane moves,
// a few cycles each, no LDS round trip).  Inside a 16-lane row:
// quad_perm [1,0,3,2] and [2,3,0,1] give every lane its quad total,
// row_half_mirror adds the mirrored quad of the 8-lane half, row_mirror the
// mirrored half of the row, so every lane holds its row total.  Across rows
// the four row totals are read with readlane (wave-uniform result).
// Every lane of the wave must be active.
template <int CTRL>
__device__ __forceinline__ float dpp_mov(float v) {
  return __builtin_bit_cast(
      float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, v), CTRL, 0xF, 0xF, false));
}

__device__ __forceinline__ float lane_read(float v, int lane) {
  return __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, v), lane));
}

// Every lane of each aligned WIDTH-lane segment ends with the segment total.
template <int WIDTH>
__device__ __forceinline__ float segment_sum(float v) {
  static_assert(WIDTH == 1 || WIDTH == 2 || WIDTH == 4 || WIDTH == 8 || WIDTH == 16 ||
                    WIDTH == 32 || WIDTH == 64,
                "segment width must be a power of two <= 64");
  if (WIDTH >= 2) v += dpp_mov<0xB1>(v);   // quad_perm [1,0,3,2]
  if (WIDTH >= 4) v += dpp_mov<0x4E>(v);   // quad_perm [2,3,0,1]
  if (WIDTH >= 8) v += dpp_mov<0x141>(v);  // row_half_mirror
  if (WIDTH >= 16) v += dpp_mov<0x140>(v); // row_mirror
  if (WIDTH == 32) v += __shfl_xor(v, 16, 64);
  if (WIDTH == 64) {
    v = (lane_read(v, 0) + lane_read(v, 16)) + (lane_read(v, 32) + lane_read(v, 48));
  }
  return v;
}

// Wave-wide best (value, index) pair: larger value, then smaller index.
// DPP steps inside each 16-lane row, then the four row winners read out and
// combined in a fixed order; the result is wave-uniform.  Every lane of the
// wave must be active.
// (bitwise on the comparisons: no short-circuit branches)
__device__ __forceinline__ bool pair_better(float v, int i, float bv, int bi) {
  return (v > bv) | ((v == bv) & (i < bi));
}
template <int CTRL>
__device__ __forceinline__ void pair_step(float& bv, int& bi) {
  const float ov = dpp_mov<CTRL>(bv);
  const int oi = __builtin_amdgcn_update_dpp(0, bi, CTRL, 0xF, 0xF, false);
  if (pair_better(ov, oi, bv, bi)) {
    bv = ov;
    bi = oi;
  }
}
__device__ __forceinline__ void wave_best_pair(float& bv, int& bi) {
  pair_step<0xB1>(bv, bi);   // quad_perm [1,0,3,2]
  pair_step<0x4E>(bv, bi);   // quad_perm [2,3,0,1]
  pair_step<0x141>(bv, bi);  // row_half_mirror
  pair_step<0x140>(bv, bi);  // row_mirror
  float cv = lane_read(bv, 0);
  int ci = __builtin_amdgcn_readlane(bi, 0);
#pragma unroll
  for (int row = 1; row < 4; ++row) {
    const float ov = lane_read(bv, 16 * row);
    const int oi = __builtin_amdgcn_readlane(bi, 16 * row);
    if (pair_better(ov, oi, cv, ci)) {
      cv = ov;
      ci = oi;
    }
  }
  bv = cv;
  bi = ci;
}

// ---------------------------------------------------------------------------
// U4 x f16 chunk dot product (32 nibbles of one row against 32 activations).
//
// A 32-bit word holds nibbles k0..k7 at bits 0,4,...,28.  Masking with
// 0x000F000F and OR-ing 0x6400 into each half gives the f16 pair
// (1024+q0, 1024+q4); masking with 0x00F000F0 gives (1024+16 q1, 1024+16 q5);
// the same on (word >> 8) gives (q2, q6) and (16 q3, 16 q7).  Two dot2 chains
// (v_dot2_f32_f16, exact f16 products, f32 accumulate) then hold
//   a1  = sum_even (1024 + q) x          a16 = sum_odd (1024 + 16 q) x
// so a1 + a16/16 = sum q x + 1024 X_even + 64 X_odd.  The per-lane constants
// `bias` = 1024 X_even + 64 X_odd and `xsum` = X_even + X_odd turn that into
// sum (q - z) x = a1 + a16/16 - bias - z * xsum, exact up to f32 rounding of
// the running sums (relative error ~1e-5 of the chunk value).
// ---------------------------------------------------------------------------
struct XChunk {
  f16x2 p[16];  // per word d: (x0,x4), (x1,x5), (x2,x6), (x3,x7)
  float bias;
  float xsum;
};

// Build the pairs for 32 consecutive f16 activations given as 16 words.
__device__ __forceinline__ void make_xchunk(const uint32_t (&xw)[16], XChunk& c) {
  float xe = 0.f, xo = 0.f;
#pragma unroll
  for (int d = 0; d < 4; ++d) {
    const uint32_t w0 = xw[4 * d + 0], w1 = xw[4 * d + 1];
    const uint32_t w2 = xw[4 * d + 2], w3 = xw[4 * d + 3];
    // words: w0=(x0,x1) w1=(x2,x3) w2=(x4,x5) w3=(x6,x7)
    c.p[4 * d + 0] = as_h2(__builtin_amdgcn_perm(w2, w0, 0x05040100u));  // (x0,x4)
    c.p[4 * d + 1] = as_h2(__builtin_amdgcn_perm(w2, w0, 0x07060302u));  // (x1,x5)
    c.p[4 * d + 2] = as_h2(__builtin_amdgcn_perm(w3, w1, 0x05040100u));  // (x2,x6)
    c.p[4 * d + 3] = as_h2(__builtin_amdgcn_perm(w3, w1, 0x07060302u));  // (x3,x7)
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const f16x2 v = as_h2(xw[4 * d + j]);
      xe += (float)v.x;
      xo += (float)v.y;
    }
  }
  c.bias = 1024.f * xe + 64.f * xo;
  c.xsum = xe + xo;
}

// 0x64006400 (two f16 1024.0) held in a VGPR.  With the nibble mask in an
// SGPR, each "extract + bias" below is then a single v_and_or_b32 (a VOP3
// instruction takes at most one scalar operand and no literal on gfx9).
// Create it once outside a loop and pass it to the chunk routines.
__device__ __forceinline__ uint32_t u4_magic() {
  uint32_t m = 0x64006400u;
  asm volatile("" : "+v"(m));
  return m;
}

__device__ __forceinline__ float u4_chunk_raw(const u32x4 w, const XChunk& c, uint32_t magic) {
  float a1 = 0.f, a16 = 0.f;
#pragma unroll
  for (int d = 0; d < 4; ++d) {
    const uint32_t v = w[d];
    const uint32_t v8 = v >> 8;
    a1 = __builtin_amdgcn_fdot2(as_h2((v & 0x000F000Fu) | magic), c.p[4 * d + 0], a1, false);
    a16 = __builtin_amdgcn_fdot2(as_h2((v & 0x00F000F0u) | magic), c.p[4 * d + 1], a16, false);
    a1 = __builtin_amdgcn_fdot2(as_h2((v8 & 0x000F000Fu) | magic), c.p[4 * d + 2], a1, false);
    a16 = __builtin_amdgcn_fdot2(as_h2((v8 & 0x00F000F0u) | magic), c.p[4 * d + 3], a16, false);
  }
  return a1 + a16 * 0.0625f;
}

// sum_k (q_k - z) * s * x_k over the chunk.
__device__ __forceinline__ float u4_chunk_dot(const u32x4 w, const XChunk& c, uint32_t z,
                                              float s, uint32_t magic) {
  return (u4_chunk_raw(w, c, magic) - c.bias - (float)z * c.xsum) * s;
}

// ---------------------------------------------------------------------------
// f16 dequantization of 8 nibbles (the MFMA operand of the grouped GEMM).
//
// One 32-bit word holds k0..k7; the result is f16((q - z) * s) for k0..k7 in
// natural order (k0,k1),(k2,k3),(k4,k5),(k6,k7).  A byte permute puts byte i
// of the word in bits 0..7 and byte i of (word >> 4) in bits 16..23, so the
// mask 0x000F000F leaves (q_2i, q_2i+1) in the two halves; OR-ing 0x6400
// makes each half the f16 value 1024 + q exactly.  Subtracting zz2 =
// {1024 + z, 1024 + z} is exact ((q - z) is an integer in [-15, 15]) and the
// product with ss2 = {s, s} is the one rounding: the result equals
// f16(f32(q - z) * f32(s)) for every f16 scale, subnormals included (both
// halves use the scale itself, never a rescaled copy of it).  `magic` is
// 0x64006400 in a VGPR (see u4_magic).
// ---------------------------------------------------------------------------
__device__ __forceinline__ f16x2 u4_zz2(uint32_t z) {
  return as_h2((0x6400u | z) * 0x00010001u);
}
__device__ __forceinline__ f16x2 u4_ss2(uint32_t scale_bits) {
  return as_h2((scale_bits & 0xffffu) * 0x00010001u);
}
__device__ __forceinline__ f16x8 dequant8(uint32_t d, f16x2 zz2, f16x2 ss2, uint32_t magic) {
  const uint32_t d4 = d >> 4;
  const f16x2 p0 = (as_h2((__builtin_amdgcn_perm(d4, d, 0x0C040C00u) & 0x000F000Fu) | magic) - zz2) * ss2;
  const f16x2 p1 = (as_h2((__builtin_amdgcn_perm(d4, d, 0x0C050C01u) & 0x000F000Fu) | magic) - zz2) * ss2;
  const f16x2 p2 = (as_h2((__builtin_amdgcn_perm(d4, d, 0x0C060C02u) & 0x000F000Fu) | magic) - zz2) * ss2;
  const f16x2 p3 = (as_h2((__builtin_amdgcn_perm(d4, d, 0x0C070C03u) & 0x000F000Fu) | magic) - zz2) * ss2;
  const u32x4 v{h2_bits(p0), h2_bits(p1), h2_bits(p2), h2_bits(p3)};
  return __builtin_bit_cast(f16x8, v);
}

// Loads through pointers the compiler cannot prove global (e.g. read from a
// device-side table) would otherwise become flat loads, which also count
// against the LDS counter and so stall at the next LDS wait.  These force the
// global address space.
#define AIMA_GLOBAL __attribute__((address_space(1)))

__device__ __forceinline__ u32x4 gload16(const void* p) {
  return *((const AIMA_GLOBAL u32x4*)(p));
}

__device__ __forceinline__ u32x4 load16_nt(const void* p) {
  return __builtin_nontemporal_load(reinterpret_cast<const u32x4*>(p));
}

// Sum over a 256-thread block; every thread gets the total.  `red` is a
// 4-float shared array.
__device__ __forceinline__ float block_sum_256(float v, float* red) {
  v = segment_sum<64>(v);
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  if (lane == 0) red[wave] = v;
  __syncthreads();
  const float t = (red[0] + red[1]) + (red[2] + red[3]);
  __syncthreads();
  return t;
}

// Row helpers for 256-thread blocks over an f16 row of H elements (H a
// multiple of 8, row 16-byte aligned): thread i handles the 8-element chunks
// i, i + 256, ... with 16-byte accesses.  Every caller of a helper sums in
// the same order with explicit fused multiply-adds (fmaf: the compiler's own
// contraction depends on the surrounding code), so fused and standalone uses
// agree bit for bit.
__device__ __forceinline__ float row_dot_f16(const uint16_t* __restrict__ a,
                                             const uint16_t* __restrict__ b, int64_t H,
                                             float* red) {
  float s = 0.f;
  for (int64_t i = threadIdx.x * 8; i < H; i += 2048) {
    const u32x4 va = *reinterpret_cast<const u32x4*>(a + i);
    const u32x4 vb = *reinterpret_cast<const u32x4*>(b + i);
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      s = fmaf(h2f((uint16_t)(va[j] & 0xffffu)), h2f((uint16_t)(vb[j] & 0xffffu)), s);
      s = fmaf(h2f((uint16_t)(va[j] >> 16)), h2f((uint16_t)(vb[j] >> 16)), s);
    }
  }
  return block_sum_256(s, red);
}

// out = f16(x * (1 / sqrt(mean(x^2) + eps)) * w)
__device__ __forceinline__ void rmsnorm_row(const uint16_t* __restrict__ x,
                                            const float* __restrict__ w, int64_t H, float eps,
                                            uint16_t* __restrict__ out, float* red) {
  float ss = 0.f;
  for (int64_t i = threadIdx.x * 8; i < H; i += 2048) {
    const u32x4 v = *reinterpret_cast<const u32x4*>(x + i);
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const float lo = h2f((uint16_t)(v[j] & 0xffffu)), hi = h2f((uint16_t)(v[j] >> 16));
      ss = fmaf(lo, lo, ss);
      ss = fmaf(hi, hi, ss);
    }
  }
  ss = block_sum_256(ss, red);
  const float scale = 1.0f / sqrtf(ss / (float)H + eps);
  for (int64_t i = threadIdx.x * 8; i < H; i += 2048) {
    const u32x4 v = *reinterpret_cast<const u32x4*>(x + i);
    u32x4 o;
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const float lo = h2f((uint16_t)(v[j] & 0xffffu)) * scale * w[i + 2 * j];
      const float hi = h2f((uint16_t)(v[j] >> 16)) * scale * w[i + 2 * j + 1];
      o[j] = pack_h2(lo, hi);
    }
    *reinterpret_cast<u32x4*>(out + i) = o;
  }
}

// Router selection for one token by one wave (all 64 lanes active):
// softmax over `experts` logits in f64 (max and sum by xor shuffles), top-k
// by (probability desc, id asc) on the f32 probabilities, then the picks
// renormalized by max(sum, min_weight_sum) summed in rank order.  Lane r < k
// returns pick r: its id, normalized weight and probability.  PER = logits
// per lane (experts <= 64 PER).  The select_router_topk semantics
// (gguf_loader.hpp:371-373).
template <int PER>
__device__ __forceinline__ void router_select_wave(const float* __restrict__ l, int experts, int k,
                                                   float min_weight_sum, int& out_id,
                                                   float& out_w, float& out_p) {
  const int lane = threadIdx.x & 63;
  float v[PER];
  float mx = -INFINITY;
#pragma unroll
  for (int j = 0; j < PER; ++j) {
    const int i = lane + 64 * j;
    v[j] = i < experts ? l[i] : -INFINITY;
    mx = fmaxf(mx, v[j]);
  }
#pragma unroll
  for (int off = 32; off > 0; off >>= 1) mx = fmaxf(mx, __shfl_xor(mx, off, 64));
  double e[PER];
  double sum = 0.0;
#pragma unroll
  for (int j = 0; j < PER; ++j) {
    const int i = lane + 64 * j;
    e[j] = i < experts ? exp((double)v[j] - (double)mx) : 0.0;
    sum += e[j];
  }
#pragma unroll
  for (int off = 32; off > 0; off >>= 1) sum += __shfl_xor(sum, off, 64);
  float p[PER];
#pragma unroll
  for (int j = 0; j < PER; ++j) {
    const int i = lane + 64 * j;
    p[j] = i < experts ? (float)(e[j] / sum) : -INFINITY;
  }
  float my_p = 0.f;
  int my_i = 0;
  for (int r = 0; r < k; ++r) {
    float bp = -INFINITY;
    int bi = 0x7fffffff;
#pragma unroll
    for (int j = 0; j < PER; ++j) {
      const int i = lane + 64 * j;
      if ((i < experts) & pair_better(p[j], i, bp, bi)) {
        bp = p[j];
        bi = i;
      }
    }
    wave_best_pair(bp, bi);
    if (lane == r) {
      my_p = bp;
      my_i = bi;
    }
#pragma unroll
    for (int j = 0; j < PER; ++j) {
      if (lane + 64 * j == bi) p[j] = -INFINITY;
    }
  }
  float s = 0.f;
  for (int r = 0; r < k; ++r) s += __shfl(my_p, r, 64);
  const float den = s > min_weight_sum ? s : min_weight_sum;
  out_id = my_i;
  out_w = my_p / den;
  out_p = my_p;
}

// Orders one wave's LDS writes before its following LDS reads by other lanes
// of the same wave (a wave executes its LDS operations in order; the fences
// keep the compiler from moving the accesses across).
__device__ __forceinline__ void wave_lds_sync() {
  __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
  __builtin_amdgcn_wave_barrier();
  __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
}

__device__ __forceinline__ float silu_mul(float g, float u) {
  const float s = g >= 0.f ? 1.f / (1.f + expf(-g)) : expf(g) / (1.f + expf(g));
  return g * s * u;
}

}  // namespace aima
