// Persistent batch-1 decode of an MoE FFN stack (all layers in one launch).
//
// Launch: 256 blocks of 512 threads, one per CU (all resident at once).
// MI355X has 8 XCDs of 32 CUs, each XCD with its own L2; blocks are placed
// on the XCDs round-robin.  A block reads its XCD id (x) from the hardware
// and takes rank j = blockIdx / 8 inside it.  The work of a layer is split
// by XCD so that only one exchange per layer crosses XCDs:
//   XCD x owns routed slot x (the rank-x expert of the top-k) and slice x of
//   the shared expert (its intermediate units 64x .. 64x+63).
//   A_L  block (x, j) computes 18 of the XCD's 576 gate/up pairs (SwiGLU)
//        and publishes them to its XCD (act_L, XCD-local).
//   B_L  block (x, j) computes output rows 64j .. 64j+63 of
//        P_x = c_x * down_x(act_x) + sigma * shared_down[:, slice x](act_sh,x)
//        and publishes them to every XCD (cross-XCD).
//   relay  block (x, j) sums P_0..P_7 for its 64 rows, adds the residual
//        and publishes r_{L+1} rows to its XCD (XCD-local); every block of
//        the XCD then reads all 2048 rows of r_{L+1}.
// XCD-local words are written with plain stores, which stay in the XCD's
// L2, and read with device-scope loads, which hit there (about 0.3 us one
// way against 0.45 us for a device-scope store/load pair across XCDs,
// measured on MI355X); cross-XCD words use device-scope stores and loads.
// Each XCD-local buffer is indexed by the hardware XCD id, so only the CUs
// of that XCD ever write or read it.
//
// Every value another block consumes is a self-validating word: {f16 value,
// u16 epoch} for the residual, {3 x f16, u16 epoch} 64-bit records for the
// activations, {f32, u32 epoch} for the partial outputs P, {id, epoch} /
// {f32, epoch} for the routes.  A consumer polls until every epoch matches
// the one expected for this launch and phase, so the wait and the transfer
// are one round trip.  Buffers alternate by layer parity, and a buffer is
// rewritten two layers later only after every reader finished with it:
// act_{L+2} is published after reading r_{L+2}, which needs P_{L+1} of every
// block, each published after its XCD's act_{L+1} was complete, i.e. after
// every block had finished B_L (its reads of act_L).  P_{L+2} needs act_{L+2}
// of the XCD, hence r_{L+2}, hence the XCD's relays of layer L+1, which read
// P_{L+1} of every block; each block published P_{L+1} after reading r_{L+1},
// i.e. after all relays of its XCD had consumed P_L.  r_{L+3} is published by
// a relay after reading P_{L+2} of its own block, i.e. after every block of
// the XCD had read r_{L+2} (and so finished with r_{L+1}).  Epochs are unique
// per launch: every block reads the launch counter when it starts, and block
// 0 advances it on exit, which happens only after every block has published
// (block 0's last residual read depends on P of every block; with one layer
// block 0 waits for all P words explicitly).
// Every poll has a spin limit: on expiry the block records
// AIMA_DEVERR_TIMEOUT and all its waves return.
#include "common.h"

#include <math.h>

#include <cstdlib>
#include <string>
#include <vector>

namespace aima {

namespace {

typedef uint32_t u32x2 __attribute__((ext_vector_type(2)));

constexpr int kThreads = 512;
constexpr int kWaves = kThreads / 64;
constexpr int kStreamWaves = 1;                          // the streaming wave (ring instance)
constexpr int kRingThreads = kThreads + 64 * kStreamWaves;
constexpr int kH = 2048;                                 // hidden (specialization)
constexpr int kI = 512;                                  // expert intermediate (specialization)
constexpr int kXcds = 8;
constexpr int kPerXcd = 32;                              // blocks per XCD
constexpr int kBlocks = kXcds * kPerXcd;                 // 256
constexpr int kSlice = kI / kXcds;                       // shared-expert units per XCD
constexpr int kXcdPairs = kI + kSlice;                   // 576 gate/up pairs per XCD
constexpr int kPairs = kXcdPairs / kPerXcd;              // 18 pairs per block
constexpr int kRowsA = 2 * kPairs;                       // 36 gate/up rows per block
constexpr int kMaxRowsA = (kRowsA + kWaves - 1) / kWaves;  // 5 rows per wave at most
constexpr int kRowsB = kH / kPerXcd;                     // 64 output rows per block
constexpr int kWaveRowsB = kRowsB / kWaves;              // 8 output rows per wave
constexpr int kActRecords = kXcdPairs / 3;               // 192 act records per XCD
constexpr int kActStride = 256;                          // records per (XCD, parity) buffer
constexpr int kChunksA = kH / 32;                        // A-phase operand chunks
constexpr int kChunksB = kXcdPairs / 32;                 // 18 B-phase operand chunks
constexpr int kMaxK = 8;
constexpr uint32_t kSpinLimit = 1u << 22;
constexpr int kMaxLayers = 79;
constexpr int kRouterRows = kPerXcd * kWaves;            // 256: router rows per XCD (routed plan)
static_assert(kPairs % 3 == 0, "blocks own whole act records");
static_assert(kActRecords <= 192, "the activation poll covers records 0..191");
static_assert(kRowsB % kWaves == 0 && kWaveRowsB == 8, "8 output rows per wave");

// One layer's tensors, resolved on the host for the kernel: the routed gate
// (h = 0) and up (h = 1) projections as their expert-0, unit-0 rows plus a
// byte stride per expert (either boundary form of aima_moe_layer: the
// concatenated gate_up has the up rows I rows after the gate rows, the split
// form two tensors), the shared expert's gate/up at unit 0, both down
// projections, the shared gate vector and the RMSNorm weight.
struct PlanLayer {
  const uint8_t *gq0, *gq1;  // (named fields, no arrays: a register copy of
  const uint16_t *gs0, *gs1;  // an entry is then never indexed at run time)
  const uint8_t *gz0, *gz1;
  const uint8_t *sq0, *sq1;
  const uint16_t *ss0, *ss1;
  const uint8_t *sz0, *sz1;
  const uint8_t* dq;
  const uint16_t* ds;
  const uint8_t* dz;
  const uint8_t* sdq;             // shared down, slice-major copy [xcd][kH][32 B]
  const uint16_t* sds;
  const uint8_t* sdz;
  const uint16_t* gate_vec;
  const float* norm;
  const uint8_t* rq;              // router [experts][kH] (routed plan; else null)
  const uint16_t* rs;
  const uint8_t* rz;
  uint32_t estride_q, estride_s, estride_z;  // routed gate/up bytes per expert
  uint32_t pad;
};
static_assert(sizeof(PlanLayer) % 4 == 0, "the table is copied as 32-bit words");

struct PersistArgs {
  const PlanLayer* layers;        // device table [n_layers]
  int n_layers;
  int k;
  int experts;
  int group_log2;
  const float* logits;            // [L][E] or null
  const int32_t* ids_in;          // [L][k] (when logits is null)
  const float* w_in;              // [L][k]
  float min_weight_sum;
  float eps;
  const uint16_t* r0;             // f16 [H]
  uint16_t* out;                  // f16 [H]
  uint32_t* rx;                   // [xcd][2][H]            {f16, epoch}, XCD-local
  uint64_t* actx;                 // [xcd][2][kActStride]   {3 x f16, epoch}, XCD-local
  uint64_t* pbuf;                 // [2][xcd][H]            {f32, epoch}
  uint32_t* route_ids;            // [L][k]                 {id, epoch}
  uint64_t* route_w;              // [L][k]                 {f32, epoch}
  uint64_t* lgx;                  // [xcd][2][kRouterRows]  {f32, epoch}, XCD-local
  float* logits_out;              // routed plan: [L][E] or null
  int32_t* ids_out;               // routed plan: [L][k] or null
  float* w_out;                   // routed plan: [L][k] or null
  uint32_t* epoch_counter;
  uint32_t* err;
};

__device__ __forceinline__ uint32_t ld_coherent32(const uint32_t* p) {
  return __hip_atomic_load(p, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ uint64_t ld_coherent64(const uint64_t* p) {
  return __hip_atomic_load(p, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ void st_coherent32(uint32_t* p, uint32_t v) {
  __hip_atomic_store(p, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ void st_coherent64(uint64_t* p, uint64_t v) {
  __hip_atomic_store(p, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
// XCD-local stores: plain global stores, which complete in the XCD's L2.
__device__ __forceinline__ void st_local32(uint32_t* p, uint32_t v) {
  asm volatile("global_store_dword %0, %1, off" : : "v"(p), "v"(v) : "memory");
}
__device__ __forceinline__ void st_local64(uint64_t* p, uint64_t v) {
  asm volatile("global_store_dwordx2 %0, %1, off" : : "v"(p), "v"(v) : "memory");
}
// Poll loads: device-scope (sc1) 16-byte loads issued together, then one
// wait.  Written as asm so that repeated polls are never merged or hoisted
// (a volatile buffer load would also set sc0, which measured slower).
__device__ __forceinline__ u32x4 poll1(const void* p) {
  u32x4 v;
  asm volatile("global_load_dwordx4 %0, %1, off sc1\n\ts_waitcnt vmcnt(0)"
               : "=v"(v) : "v"(p) : "memory");
  return v;
}
__device__ __forceinline__ void poll2(const void* p, const void* q, u32x4& v, u32x4& w) {
  asm volatile(
      "global_load_dwordx4 %0, %2, off sc1\n\t"
      "global_load_dwordx4 %1, %3, off sc1\n\t"
      "s_waitcnt vmcnt(0)"
      : "=&v"(v), "=&v"(w) : "v"(p), "v"(q) : "memory");
}
// eight 8-byte loads `stride` bytes apart
__device__ __forceinline__ void poll8(const void* p, int stride, uint64_t (&v)[8]) {
  const char* c = reinterpret_cast<const char*>(p);
  asm volatile(
      "global_load_dwordx2 %0, %8, off sc1\n\t"
      "global_load_dwordx2 %1, %9, off sc1\n\t"
      "global_load_dwordx2 %2, %10, off sc1\n\t"
      "global_load_dwordx2 %3, %11, off sc1\n\t"
      "global_load_dwordx2 %4, %12, off sc1\n\t"
      "global_load_dwordx2 %5, %13, off sc1\n\t"
      "global_load_dwordx2 %6, %14, off sc1\n\t"
      "global_load_dwordx2 %7, %15, off sc1\n\t"
      "s_waitcnt vmcnt(0)"
      : "=&v"(v[0]), "=&v"(v[1]), "=&v"(v[2]), "=&v"(v[3]), "=&v"(v[4]), "=&v"(v[5]),
        "=&v"(v[6]), "=&v"(v[7])
      : "v"(c), "v"(c + stride), "v"(c + 2 * stride), "v"(c + 3 * stride), "v"(c + 4 * stride),
        "v"(c + 5 * stride), "v"(c + 6 * stride), "v"(c + 7 * stride)
      : "memory");
}

// four 8-byte loads `stride` bytes apart
__device__ __forceinline__ void poll4(const void* p, int stride, uint64_t (&v)[4]) {
  const char* c = reinterpret_cast<const char*>(p);
  asm volatile(
      "global_load_dwordx2 %0, %4, off sc1\n\t"
      "global_load_dwordx2 %1, %5, off sc1\n\t"
      "global_load_dwordx2 %2, %6, off sc1\n\t"
      "global_load_dwordx2 %3, %7, off sc1\n\t"
      "s_waitcnt vmcnt(0)"
      : "=&v"(v[0]), "=&v"(v[1]), "=&v"(v[2]), "=&v"(v[3])
      : "v"(c), "v"(c + stride), "v"(c + 2 * stride), "v"(c + 3 * stride)
      : "memory");
}

__device__ __forceinline__ uint32_t pack_word(uint16_t v, uint32_t epoch) {
  return (uint32_t)v | (epoch << 16);
}
// A lane's part of one row's dot product (u4_chunk_dot), rounded as written:
// the empty asm keeps the compiler from fusing the final product into the
// first step of the row sum that follows, which it does or not depending on
// the surrounding code.  Every instance of the kernel (weight ring, register
// prefetch, routed) must produce the same sums bit for bit.
__device__ __forceinline__ float lane_dot(const u32x4 w, const XChunk& c, uint32_t z, float s,
                                          uint32_t magic) {
  float t = __builtin_fmaf(-(float)z, c.xsum, u4_chunk_raw(w, c, magic) - c.bias);
  t = t * s;
  asm volatile("" : "+v"(t));
  return t;
}

// f32 -> f16 of a value rounded to f32 first, as the arithmetic reads (and
// as the CPU reference converts): without the empty asm the compiler may
// fold the final multiply or add into a mixed-precision FMA that rounds once
// to f16, or not, depending on the surrounding code -- rare one-ulp
// differences between the kernel's instances.
__device__ __forceinline__ uint16_t f2h_rounded(float f) {
  asm volatile("" : "+v"(f));
  return f2h(f);
}

__device__ __forceinline__ uint64_t pack_f32(float v, uint32_t epoch) {
  return (uint64_t)__builtin_bit_cast(uint32_t, v) | ((uint64_t)epoch << 32);
}

struct SharedState {
  u32x4 xa_p[4][kChunksA];             // A operands: chunk pairs, word-group major
  float xa_bias[kChunksA];
  float xa_xsum[kChunksA];
  u32x4 xb_p[4][kChunksB];             // B operands (16 routed + 2 shared chunks)
  float xb_bias[kChunksB];
  float xb_xsum[kChunksB];
  alignas(16) uint32_t act[kXcdPairs / 2];  // act_L of this XCD, f16 pairs
  alignas(16) uint32_t rl[kH / 2];      // r_L, f16 pairs (read by the relay)
  float ss[kWaves];                    // per-wave sums of squares of r_L
  float gp[kWaves];                    // per-wave shared-gate partial dots
  // gate/up row sums as four 16-lane partials (lanes 0-15, 16-31, 32-47,
  // 48-63), summed (p0 + p1) + (p2 + p3) where used: segment_sum<64>'s order
  alignas(16) float rowpart[kRowsA][4];
  PlanLayer table[kMaxLayers];         // the layer table, copied once
  int32_t route_id[kMaxLayers][kMaxK];
  float route_w[kMaxLayers][kMaxK];
  float sigma;
  int abort;
  int reroute;                         // routed plan: the layer's route changed
  int32_t rank[kMaxK + 1];             // routed plan: ranks 0..k by logit
};

// One slot of the weight ring (ring instance): everything the 8 compute
// waves of a block read for one layer, in the per-lane order they read it.
// Written by the streaming wave one layer ahead (two slots: layer L reads
// slot L & 1 while layer L + 1's rows fill the other).
struct RingSlot {
  u32x4 a[kRowsA][64];                 // gate/up rows: block row ri, lane l's 32 nibbles
  u32x4 b[kWaves][2][64];              // routed down rows of wave w, units 0 and 1
  u32x4 bs[kWaves][16];                // shared down slice of wave w (16 lanes' chunks)
  // Scale and zero-point words, each kind in the order it lies in memory, so
  // that the streaming wave loads and stores them lane by lane:
  // as[h * 144 + 8 pp + w]: word w (16 f16 scales) of the block's pair pp,
  // gate (h = 0) or up (h = 1); az[h * 36 + 2 pp + w]: its zero-point words;
  // bgs[128 s + 16 wv + q]: scale word q of wave wv's 8 down rows, routed
  // (s = 0) or the shared slice (s = 1); bgz[32 s + 4 wv + q]: zero points.
  uint32_t as[2 * kPairs * 8];
  uint32_t az[2 * kPairs * 2];
  uint32_t bgs[2 * kWaves * 16];
  uint32_t bgz[2 * kWaves * 4];
};
static_assert(sizeof(RingSlot) % 16 == 0, "ring slots stay 16-byte aligned");

// Router top-k for one layer (one wave): f64 softmax over the logits,
// (probability desc, id asc) selection, renormalization by max(sum, min).
// Lane `r` < k returns the rank-r id and weight.  Reductions use DPP inside
// 16-lane rows and readlane across rows (no LDS round trips).
template <int CTRL>
__device__ __forceinline__ int dpp_int(int v) {
  return __builtin_amdgcn_update_dpp(0, v, CTRL, 0xF, 0xF, false);
}
__device__ __forceinline__ bool route_better(float p, int i, float bp, int bi) {
  return (p > bp) | ((p == bp) & (i < bi));
}
template <int CTRL>
__device__ __forceinline__ void argmax_step(float& bp, int& bi) {
  const float op = dpp_mov<CTRL>(bp);
  const int oi = dpp_int<CTRL>(bi);
  if (route_better(op, oi, bp, bi)) {
    bp = op;
    bi = oi;
  }
}
__device__ void route_layer(const float* __restrict__ l, int E, int k, float min_sum,
                            int32_t* ids, float* w) {
  const int lane = threadIdx.x & 63;
  const int per = (E + 63) / 64;
  float lv[16];
  float mx = -INFINITY;
#pragma unroll
  for (int j = 0; j < 16; ++j) {
    const int i = lane + 64 * j;
    lv[j] = (j < per && i < E) ? l[i] : -INFINITY;
    mx = fmaxf(mx, lv[j]);
  }
  mx = fmaxf(mx, dpp_mov<0xB1>(mx));
  mx = fmaxf(mx, dpp_mov<0x4E>(mx));
  mx = fmaxf(mx, dpp_mov<0x141>(mx));
  mx = fmaxf(mx, dpp_mov<0x140>(mx));
  mx = fmaxf(fmaxf(lane_read(mx, 0), lane_read(mx, 16)), fmaxf(lane_read(mx, 32), lane_read(mx, 48)));
  double ev[16];
  double sum = 0.0;
#pragma unroll
  for (int j = 0; j < 16; ++j) {
    const int i = lane + 64 * j;
    ev[j] = (j < per && i < E) ? exp((double)lv[j] - (double)mx) : 0.0;
    sum += ev[j];
  }
#pragma unroll
  for (int off = 32; off > 0; off >>= 1) sum += __shfl_xor(sum, off, 64);
  float p[16];
#pragma unroll
  for (int j = 0; j < 16; ++j) {
    const int i = lane + 64 * j;
    p[j] = (j < per && i < E) ? (float)(ev[j] / sum) : -INFINITY;
  }
  float psum = 0.f;
  for (int r = 0; r < k; ++r) {
    float bp = -INFINITY;
    int bi = 0x7fffffff;
#pragma unroll
    for (int j = 0; j < 16; ++j) {
      const int i = lane + 64 * j;
      if (i < E && route_better(p[j], i, bp, bi)) {
        bp = p[j];
        bi = i;
      }
    }
    argmax_step<0xB1>(bp, bi);
    argmax_step<0x4E>(bp, bi);
    argmax_step<0x141>(bp, bi);
    argmax_step<0x140>(bp, bi);
    // the four row winners, combined in a fixed order (wave-uniform result)
    float cp = lane_read(bp, 0);
    int ci = __builtin_amdgcn_readlane(bi, 0);
#pragma unroll
    for (int row = 1; row < 4; ++row) {
      const float op = lane_read(bp, 16 * row);
      const int oi = __builtin_amdgcn_readlane(bi, 16 * row);
      if (route_better(op, oi, cp, ci)) {
        cp = op;
        ci = oi;
      }
    }
#pragma unroll
    for (int j = 0; j < 16; ++j) {
      if (lane + 64 * j == ci) p[j] = -INFINITY;
    }
    if (lane == r) {
      ids[0] = ci;
      w[0] = cp;
    }
    psum = (r == 0) ? cp : psum + cp;  // sequential f32 sum in rank order
  }
  const float den = psum > min_sum ? psum : min_sum;
  if (lane < k) w[0] = w[0] / den;
}

// Router top-k of one layer for the routed plan (experts <= 256; lane l of
// a wave holds the logits of experts l + 64 t).  The rule is
// select_router_topk's (gguf_loader.hpp:371-373): softmax in f64, the top k
// by (probability desc, id asc) on the f32 probabilities, the picks
// renormalized by max(rank-order sum, min_sum).
//
// The probabilities are a non-decreasing function of the logits, so ranking
// the logits almost always gives the answer, and the ranking needs no
// exponentials: rank_logits (one wave) ranks 32-bit keys made of the top 24
// bits of the logit's order-preserving image and the complemented id, one
// wave maximum per rank, while another wave computes the probabilities
// (softmax_probs).  The layer's weight loads start from the ranking;
// route_confirm then checks it exactly: if the probabilities of ranks 0..k
// decrease strictly and exactly k + 1 probabilities are >= that of rank k,
// then every other probability is below rank k's, so ranks 0..k-1 are the k
// largest probabilities in order, and the route stands.  Otherwise (equal or
// nearly equal logits, rare) select_probs ranks the probabilities themselves
// and the loads are issued again.
__device__ __forceinline__ uint64_t u64_of(uint32_t lo, uint32_t hi) {
  return ((uint64_t)hi << 32) | lo;
}
template <int CTRL>
__device__ __forceinline__ uint32_t dpp_u32(uint32_t v) {
  return (uint32_t)__builtin_amdgcn_update_dpp(0, (int)v, CTRL, 0xF, 0xF, false);
}
template <int CTRL>
__device__ __forceinline__ uint64_t dpp_u64(uint64_t v) {
  return u64_of(dpp_u32<CTRL>((uint32_t)v), dpp_u32<CTRL>((uint32_t)(v >> 32)));
}
__device__ __forceinline__ uint32_t readlane_u32(uint32_t v, int l) {
  return (uint32_t)__builtin_amdgcn_readlane((int)v, l);
}
__device__ __forceinline__ uint64_t readlane_u64(uint64_t v, int l) {
  return u64_of(readlane_u32((uint32_t)v, l), readlane_u32((uint32_t)(v >> 32), l));
}
__device__ __forceinline__ uint64_t max_u64(uint64_t a, uint64_t b) { return a > b ? a : b; }
// Wave reductions: DPP inside 16-lane rows (quad_perm [1,0,3,2], [2,3,0,1],
// row_half_mirror, row_mirror), then across rows, so every lane gets the same
// value.  The u32 forms cross rows with row_bcast:15 (rows 1 and 3 take the
// last lane of the row below) and row_bcast:31 (rows 2 and 3 take lane 31),
// which leaves the total in lane 63; the others read the four rows in a
// fixed order.
template <int CTRL, int ROWS>
__device__ __forceinline__ uint32_t dpp_rows_u32(uint32_t v) {
  return (uint32_t)__builtin_amdgcn_update_dpp((int)v, (int)v, CTRL, ROWS, 0xF, false);
}
__device__ __forceinline__ uint32_t wave_max_u32(uint32_t v) {
  v = max(v, dpp_u32<0xB1>(v));
  v = max(v, dpp_u32<0x4E>(v));
  v = max(v, dpp_u32<0x141>(v));
  v = max(v, dpp_u32<0x140>(v));
  v = max(v, dpp_rows_u32<0x142, 0xA>(v));
  v = max(v, dpp_rows_u32<0x143, 0xC>(v));
  return readlane_u32(v, 63);
}
__device__ __forceinline__ uint64_t wave_max_u64(uint64_t v) {
  v = max_u64(v, dpp_u64<0xB1>(v));
  v = max_u64(v, dpp_u64<0x4E>(v));
  v = max_u64(v, dpp_u64<0x141>(v));
  v = max_u64(v, dpp_u64<0x140>(v));
  return max_u64(max_u64(readlane_u64(v, 0), readlane_u64(v, 16)),
                 max_u64(readlane_u64(v, 32), readlane_u64(v, 48)));
}

// Lane r <= k returns the expert id of rank r by the 32-bit key (-1 past
// the finite logits).  A lane keeps its four keys sorted; a round is one
// wave maximum of the lanes' heads (keys are unique: the low byte is the
// complemented id) and the winning lane dropping its head.
__device__ int rank_logits(const float (&v)[4], int experts, int k) {
  const int lane = threadIdx.x & 63;
  uint32_t q[4];
#pragma unroll
  for (int t = 0; t < 4; ++t) {
    const int i = lane + 64 * t;
    const uint32_t b = __builtin_bit_cast(uint32_t, v[t]);
    const uint32_t m = (b & 0x80000000u) ? ~b : (b | 0x80000000u);  // order-preserving
    // NaN and ids past the experts are never ranked; every finite logit
    // keeps a nonzero key (-inf maps to 0x007fffff)
    q[t] = (i < experts && v[t] == v[t]) ? ((m & 0xffffff00u) | (uint32_t)(255 - i)) : 0u;
  }
  auto cx = [&](int x, int y) {
    const uint32_t hi = max(q[x], q[y]), lo = min(q[x], q[y]);
    q[x] = hi;
    q[y] = lo;
  };
  cx(0, 1);
  cx(2, 3);
  cx(0, 2);
  cx(1, 3);
  cx(1, 2);
  int mine = -1;
  for (int r = 0; r <= k; ++r) {
    const uint32_t m = wave_max_u32(q[0]);
    if (lane == r) mine = m == 0 ? -1 : 255 - (int)(m & 0xffu);
    const bool pop = q[0] == m;
    q[0] = pop ? q[1] : q[0];
    q[1] = pop ? q[2] : q[1];
    q[2] = pop ? q[3] : q[2];
    q[3] = pop ? 0u : q[3];
  }
  return mine;
}

// f32 probabilities of the softmax (f64 exp and sum); -inf past `experts`.
// The f64 sum runs in select_router_topk's order (lane partials over t, then
// an xor butterfly), so the probabilities, and the weights made from them,
// are bit-identical to that kernel's.
__device__ void softmax_probs(const float (&v)[4], int experts, float (&p)[4]) {
  const int lane = threadIdx.x & 63;
  float mx = -INFINITY;
#pragma unroll
  for (int t = 0; t < 4; ++t) {
    if (lane + 64 * t < experts) mx = fmaxf(mx, v[t]);
  }
  mx = fmaxf(mx, dpp_mov<0xB1>(mx));
  mx = fmaxf(mx, dpp_mov<0x4E>(mx));
  mx = fmaxf(mx, dpp_mov<0x141>(mx));
  mx = fmaxf(mx, dpp_mov<0x140>(mx));
  mx = fmaxf(fmaxf(lane_read(mx, 0), lane_read(mx, 16)), fmaxf(lane_read(mx, 32), lane_read(mx, 48)));
  double e[4];
  double sum = 0.0;
#pragma unroll
  for (int t = 0; t < 4; ++t) {
    e[t] = lane + 64 * t < experts ? exp((double)v[t] - (double)mx) : 0.0;
    sum += e[t];
  }
#pragma unroll
  for (int off = 32; off > 0; off >>= 1) sum += __shfl_xor(sum, off, 64);
#pragma unroll
  for (int t = 0; t < 4; ++t) p[t] = lane + 64 * t < experts ? (float)(e[t] / sum) : -INFINITY;
}

// Lane r < k: weight of rank r given the rank-order probabilities pr.
__device__ __forceinline__ float rank_weight(float pr, int k, float min_sum) {
  float psum = 0.f;
  for (int r = 0; r < k; ++r) {
    const float x = lane_read(pr, r);
    psum = r == 0 ? x : psum + x;  // sequential f32 sum in rank order
  }
  return pr / (psum > min_sum ? psum : min_sum);
}

// The ranking of the probabilities themselves: 64-bit keys, probability
// bits (p >= 0, so they order like the values) above the complemented id.
// Lane r < k returns rank r's id (-1 when no finite probability is left)
// and weight.
__device__ void select_probs(const float (&p)[4], int experts, int k, float min_sum,
                             int& out_id, float& out_w) {
  const int lane = threadIdx.x & 63;
  uint64_t q[4];
#pragma unroll
  for (int t = 0; t < 4; ++t) {
    const int i = lane + 64 * t;
    q[t] = (i < experts && p[t] == p[t]) ? u64_of(~(uint32_t)i, __builtin_bit_cast(uint32_t, p[t]))
                                         : 0;
  }
  auto cx = [](uint64_t& a, uint64_t& b) {
    const uint64_t h = max_u64(a, b);
    b = a > b ? b : a;
    a = h;
  };
  cx(q[0], q[1]);
  cx(q[2], q[3]);
  cx(q[0], q[2]);
  cx(q[1], q[3]);
  cx(q[1], q[2]);
  uint64_t mine = 0;
  for (int r = 0; r < k; ++r) {
    const uint64_t m = wave_max_u64(q[0]);
    if (lane == r) mine = m;
    const bool pop = q[0] == m;
    q[0] = pop ? q[1] : q[0];
    q[1] = pop ? q[2] : q[1];
    q[2] = pop ? q[3] : q[2];
    q[3] = pop ? 0 : q[3];
  }
  out_id = mine == 0 ? -1 : (int)~(uint32_t)mine;
  out_w = rank_weight(__builtin_bit_cast(float, (uint32_t)(mine >> 32)), k, min_sum);
}

// Confirms the ranking `rank_id` (lane r <= k; -1 where no finite logit was
// left) against the probabilities p: true when they decrease strictly over
// ranks 0..k and no probability outside those ranks reaches rank k's, with
// lane r < k's weight in out_w.
__device__ bool route_confirm(const float (&p)[4], int experts, int rank_id, int k,
                              float min_sum, float& out_w) {
  const int lane = threadIdx.x & 63;
  const int src = rank_id & 63, t = rank_id >> 6;
  float pr = -INFINITY;
#pragma unroll
  for (int u = 0; u < 4; ++u) {
    const float x = __shfl(p[u], src, 64);
    if (rank_id >= 0 && t == u) pr = x;
  }
  const float next = __shfl(pr, lane + 1, 64);
  const uint64_t mask = (1ull << k) - 1ull;
  bool ok = (__ballot(lane < k && pr > next) & mask) == mask;
  const int last = __shfl(rank_id, k, 64);
  if (last >= 0) {
    // exactly ranks 0..k at or above rank k's probability
    const float pk = __shfl(pr, k, 64);
    int n = 0;
#pragma unroll
    for (int u = 0; u < 4; ++u) n += __popcll(__ballot(lane + 64 * u < experts && p[u] >= pk));
    ok = ok && n == k + 1;
  }
  out_w = rank_weight(pr, k, min_sum);
  return ok;
}

// One layer's route from its logits (experts <= 256, one wave): the ranking
// of the logits, confirmed against the probabilities (or replaced by their
// own ranking), as the routed plan does per layer.  Lane r < k gets rank r.
__device__ void route_layer_ranked(const float* __restrict__ l, int experts, int k, float min_sum,
                                   int32_t* id, float* w) {
  const int lane = threadIdx.x & 63;
  float lv[4];
#pragma unroll
  for (int t = 0; t < 4; ++t) {
    const int i = lane + 64 * t;
    lv[t] = i < experts ? l[i] : -INFINITY;
  }
  int rid = rank_logits(lv, experts, k);
  if (lane > k) rid = -1;
  float pv[4];
  softmax_probs(lv, experts, pv);
  float rw = 0.f;
  if (!route_confirm(pv, experts, rid, k, min_sum, rw)) select_probs(pv, experts, k, min_sum, rid, rw);
  if (lane < k) {
    *id = rid;
    *w = rw;
  }
}

__device__ __forceinline__ uint32_t h2bits(f16x2 v) { return __builtin_bit_cast(uint32_t, v); }

// XChunk <-> LDS (word-group major arrays indexed by chunk)
template <int N>
__device__ __forceinline__ void put_chunk(u32x4 (*p)[N], float* bias, float* xsum, int c,
                                          const XChunk& x) {
#pragma unroll
  for (int d = 0; d < 4; ++d) {
    p[d][c] = u32x4{h2bits(x.p[4 * d + 0]), h2bits(x.p[4 * d + 1]), h2bits(x.p[4 * d + 2]),
                    h2bits(x.p[4 * d + 3])};
  }
  bias[c] = x.bias;
  xsum[c] = x.xsum;
}
template <int N>
__device__ __forceinline__ void get_chunk(const u32x4 (*p)[N], const float* bias,
                                          const float* xsum, int c, XChunk& x) {
#pragma unroll
  for (int d = 0; d < 4; ++d) {
    const u32x4 v = p[d][c];
#pragma unroll
    for (int t = 0; t < 4; ++t) x.p[4 * d + t] = as_h2(v[t]);
  }
  x.bias = bias[c];
  x.xsum = xsum[c];
}

// 32 f16 values (16 words) at word offset w0 of an LDS array -> XChunk.
__device__ __forceinline__ void lds_xchunk(const uint32_t* src, int w0, XChunk& c) {
  uint32_t w[16];
  const u32x4* p = reinterpret_cast<const u32x4*>(src + w0);
#pragma unroll
  for (int q = 0; q < 4; ++q) {
    const u32x4 v = p[q];
    w[4 * q + 0] = v[0];
    w[4 * q + 1] = v[1];
    w[4 * q + 2] = v[2];
    w[4 * q + 3] = v[3];
  }
  make_xchunk(w, c);
}


#ifdef AIMA_DECODE_TRACE
// Diagnostics build only (never in the product library): phase timestamps of
// every block, 100 MHz real-time clock, g_trace[(L * 256 + block) * 32 + slot];
// row 40 (the prologue) keeps the block's hardware XCD id in slot 31.
// The stamps are global (not flat) stores: a flat store also counts against
// the LDS counter, so every later LDS wait would wait for the stamp to land.
__device__ uint64_t* g_trace = nullptr;
#define AIMA_TRACE(L, slot, T)                                                   \
  do {                                                                           \
    if (trace && threadIdx.x == (T) && b < 256)                                  \
      ((AIMA_GLOBAL uint64_t*)trace)[((L) * 256 + b) * 32 + (slot)] =            \
          __builtin_amdgcn_s_memrealtime();                                      \
  } while (0)
#else
#define AIMA_TRACE(L, slot, T) \
  do {                         \
  } while (0)
#endif

}  // namespace

// G128: specialized for 128-wide quantization groups (gathered scale and
// zero-point loads); the other instance serves every supported group size.
// ROUTED: each layer's route comes from its own normalized input (true
// decode, run_qwen36_moe_ffn_layer's router step, gguf_loader.cpp:5704-5711):
// after the RMSNorm every XCD computes all router logits itself (wave w of
// block j takes expert 8j + w, from router rows prefetched a layer ahead),
// exchanges them XCD-locally, and one wave of every block selects the top-k;
// only then are the layer's routed gate/up and down rows loaded.  Otherwise
// the routes of all layers come from the launch's logits or ids.
// RING (with G128, logits-fed only): a ninth wave streams every layer's
// rows into the LDS weight ring one layer ahead with ordinary global loads,
// at most one batch (18 row loads) in flight; the compute waves then issue
// no weight loads at all, so their dot products never stall on a full
// memory queue.  The streaming wave passes exactly the barriers the compute
// waves pass (see stream_rows below).
template <bool G128, bool ROUTED, bool RING = false>
__global__ __launch_bounds__(RING ? kRingThreads : kThreads, 1) void decode_persistent_kernel(
    PersistArgs a) {
  static_assert(!RING || (G128 && !ROUTED), "the ring serves the logits-fed 128-group plan");
  __shared__ SharedState S;
  __shared__ __attribute__((aligned(16))) uint8_t ring_mem[RING ? 2 * sizeof(RingSlot) : 16];
  RingSlot* const ring = reinterpret_cast<RingSlot*>(ring_mem);
  const int lane = threadIdx.x & 63;
  // wave-uniform values in scalar registers, so per-row branches and buffer
  // offsets below are scalar and never merge divergent loads
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int nb = gridDim.x;
  const int b = blockIdx.x;
  const int k = a.k;
  // hardware XCD id (HW_REG_XCC_ID bits 3:0) and the rank inside the XCD
  const int x = (int)(__builtin_amdgcn_s_getreg((3 << 11) | 20) & 0xfu);
  const int j = b >> 3;
  const uint32_t base = (*a.epoch_counter % 400u) * 160u + 1u;
  const uint32_t route_epoch = base + 2u * (uint32_t)a.n_layers;
  const int glog2 = a.group_log2;
  const int gA = kH >> glog2;  // groups per gate/up row
  const int gB = kI >> glog2;  // groups per down row
  const uint32_t magic = u4_magic();
#ifdef AIMA_DECODE_TRACE
  uint64_t* const trace = g_trace;
#endif
  AIMA_TRACE(40, 0, 0);  // kernel entry
#ifdef AIMA_DECODE_TRACE
  if (trace && threadIdx.x == 0 && b < 256)
    ((AIMA_GLOBAL uint64_t*)trace)[(40 * 256 + b) * 32 + 31] = (uint64_t)x;
  // each wave's SIMD (HW_REG_HW_ID bits 5:4) in slots 16 + wave
  if (trace && (threadIdx.x & 63) == 0 && b < 256)
    ((AIMA_GLOBAL uint64_t*)trace)[(40 * 256 + b) * 32 + 16 + wave] =
        (uint64_t)__builtin_amdgcn_s_getreg((1 << 11) | (4 << 6) | 4);
#endif

  if (threadIdx.x == 0) S.abort = 0;
  // block 0 advances the launch counter on every exit path
  auto finish = [&]() {
    if (b == 0 && threadIdx.x == 0) *a.epoch_counter = *a.epoch_counter + 1u;
  };
  auto fail_timeout = [&]() {
    if (lane == 0) {
      atomicOr(a.err, AIMA_DEVERR_TIMEOUT);
      S.abort = 1;
    }
  };
  if (x >= kXcds || nb != kBlocks) {
    // not on the 8 x 32 CU layout this kernel partitions for: every wait of
    // the other blocks then expires and reports a timeout
    if (threadIdx.x == 0) atomicOr(a.err, AIMA_DEVERR_TIMEOUT);
    finish();
    return;
  }

  auto local_route = [&](int L, int32_t* id, float* w) {
    if (a.logits && a.experts <= kRouterRows) {
      route_layer_ranked(a.logits + (int64_t)L * a.experts, a.experts, k, a.min_weight_sum, id, w);
    } else if (a.logits) {
      route_layer(a.logits + (int64_t)L * a.experts, a.experts, k, a.min_weight_sum, id, w);
    } else if (lane < k) {
      *id = a.ids_in[L * k + lane];
      *w = a.w_in[L * k + lane];
    }
  };
  // ---- prologue --------------------------------------------------------------
  // Block L computes and publishes layer L's route (wave 0) while the other
  // waves copy the layer table into LDS; then every block reads all routes
  // into LDS (one wave per layer, in parallel).
  if (!ROUTED && wave == 0) {
    for (int L = b; L < a.n_layers; L += nb) {
      int32_t id = 0;
      float w = 0.f;
      local_route(L, &id, &w);
      if (lane < k) {
        if (id < 0 || id >= a.experts) id = 0xffff;  // flagged when read
        st_coherent32(&a.route_ids[L * k + lane], pack_word((uint16_t)id, route_epoch));
        st_coherent64(&a.route_w[L * k + lane], pack_f32(w, route_epoch));
      }
    }
  }
  {
    const uint32_t* src = reinterpret_cast<const uint32_t*>(a.layers);
    uint32_t* dst = reinterpret_cast<uint32_t*>(S.table);
    const int words = a.n_layers * (int)(sizeof(PlanLayer) / 4);
    const int first = ROUTED ? 0 : 64;  // wave 0 routes in the logits-fed plan
    for (int i = (int)threadIdx.x - first; i >= 0 && i < words && wave < kWaves;
         i += kThreads - first) {
      dst[i] = src[i];
    }
  }
  __syncthreads();
  // lane l of wave w reads slot l & 7 of layer L0 + w + 8 (l >> 3)
  for (int L0 = 0; !ROUTED && wave < kWaves && L0 < a.n_layers; L0 += 8 * kWaves) {
    const int L = L0 + wave + kWaves * (lane >> 3);
    const int s = lane & 7;
    const bool mine = L < a.n_layers && s < k;
    uint32_t spins = 0;
    while (true) {
      bool ok = true;
      uint32_t idw = 0;
      uint64_t ww = 0;
      if (mine) {
        idw = ld_coherent32(&a.route_ids[L * k + s]);
        ww = ld_coherent64(&a.route_w[L * k + s]);
        ok = (idw >> 16) == route_epoch && (uint32_t)(ww >> 32) == route_epoch;
      }
      if (__all(ok)) {
        if (mine) {
          int id = (int)(idw & 0xffffu);
          if (id >= a.experts) {
            atomicOr(a.err, AIMA_DEVERR_EXPERT_RANGE);
            id = -1;
          }
          S.route_id[L][s] = id;
          S.route_w[L][s] = __builtin_bit_cast(float, (uint32_t)ww);
        }
        break;
      }
      if (++spins > kSpinLimit) {
        fail_timeout();
        break;
      }
      __builtin_amdgcn_s_sleep(2);
    }
  }
  __syncthreads();
  if (S.abort) {
    finish();
    return;
  }

  // ---- per-wave prefetch state ----------------------------------------------
  // raw prefetched words: weights, f16 scale bits, zero-point byte + nibble
  // shift; converted only when used so no wait sits between the loads.
  // Double-buffered: the *_n registers receive the next layer's rows while
  // the current ones are in use and are copied over at barrier #1.  The next
  // layer's down rows and vectors are issued at barrier #2 and its gate/up
  // rows one per dot product during A_L, so the stream overlaps the dot
  // products (measured: issuing them next to the exchanges delays every poll
  // behind them in the CU's memory pipeline).
  u32x4 wa[kMaxRowsA], wa_n[kMaxRowsA];
  uint32_t sa[kMaxRowsA], sa_n[kMaxRowsA];
  uint32_t za[kMaxRowsA], za_n[kMaxRowsA];
  u32x4 wb[3], wb_n[3];
  uint32_t sb[3], sb_n[3];
  uint32_t zb[3], zb_n[3];
  // norm weight (f32) and shared gate vector (f16) of this wave's 256 values
  u32x4 nw, nw_n;
  u32x2 gv, gv_n;
  // With 128-wide groups every scale and zero-point word a wave needs for a
  // phase comes from one gathering load (lane q fetches word q of the list
  // below) instead of two loads per row; the words are handed to the lanes
  // that use them by ds_bpermute when the buffers rotate.  The per-row loads
  // serve the other group sizes.
  constexpr bool g128 = G128;
  uint32_t gsa_n = 0, gsb_n = 0;
  auto nib = [](uint32_t word, int gi) { return (word >> ((gi & 7) * 4)) & 0xfu; };
  auto scl = [](uint32_t word, int gi) { return h2f((uint16_t)(word >> ((gi & 1) * 16))); };

  // Weight loads: scalar base (readfirstlane of the table pointer, so it is
  // provably wave-uniform) plus a 32-bit per-lane offset.  Each prefetch is
  // straight-line code: surplus row slots are clamped onto a row the block
  // loads anyway (a cache hit) and an out-of-range expert id onto expert 0
  // (its contribution is dropped and the error bit is set), so every load
  // is in bounds and issued back to back.
  auto uptr = [](const void* p) {
    const uint64_t v = reinterpret_cast<uint64_t>(p);
    const uint32_t lo = __builtin_amdgcn_readfirstlane((uint32_t)v);
    const uint32_t hi = __builtin_amdgcn_readfirstlane((uint32_t)(v >> 32));
    return reinterpret_cast<const AIMA_GLOBAL uint8_t*>(((uint64_t)hi << 32) | lo);
  };
  // Weight rows: the logits-fed plan streams them a layer ahead with the
  // nontemporal hint (plain loads measured 12 µs per token slower); the
  // routed plan's burst after each route measured 18 µs per token faster
  // with plain loads.
  auto ld_w = [](const AIMA_GLOBAL uint8_t* base_ptr, uint32_t off) {
    if constexpr (ROUTED) {
      return *reinterpret_cast<const AIMA_GLOBAL u32x4*>(base_ptr + off);
    } else {
      return __builtin_nontemporal_load(
          reinterpret_cast<const AIMA_GLOBAL u32x4*>(base_ptr + off));
    }
  };
  auto ld_u32 = [](const AIMA_GLOBAL uint8_t* base_ptr, uint32_t off) {
    return *reinterpret_cast<const AIMA_GLOBAL uint32_t*>(base_ptr + off);
  };
  // Per-lane offsets are recomputed at each prefetch from an opaque copy of
  // the lane index: hoisting them out of the layer loop would keep many
  // more registers live across every phase.
  auto opaque_v = [](int v) {
    asm volatile("" : "+v"(v));
    return v;
  };
  // the routed expert of this XCD in layer L (clamped to a valid id)
  auto slot_expert = [&](int L) -> uint32_t {
    const int e = x < k ? S.route_id[L][x] : 0;
    return (uint32_t)max(0, __builtin_amdgcn_readfirstlane(e));
  };
  // gate/up gather (groups of 128: 16 per row): lanes 0..39 = scale words
  // 0..7 of row slots 0..4, lanes 40..49 = zero-point words 0..1 of row slots
  // 0..4 (lanes above repeat lane 49)
  // The row loaders take the layer's table entry (in LDS) and routed expert.
  auto gather_a = [&](const PlanLayer& Ly, uint32_t e) {
    const int ln = opaque_v(threadIdx.x & 63);
    const int q = min(ln, 49);
    const bool is_s = q < 40;
    const int i = is_s ? (q >> 3) : ((q - 40) >> 1);
    const int w = is_s ? (q & 7) : ((q - 40) & 1);
    const int ri = min(((wave + 4) & 7) + kWaves * i, kRowsA - 1);
    const int p = j * kPairs + (ri >> 1);
    const bool routed = p < kI;
    const int unit = routed ? p : x * kSlice + (p - kI);
    const bool up = (ri & 1) != 0;
    const AIMA_GLOBAL uint8_t* rs0 = uptr(Ly.gs0) + (size_t)e * Ly.estride_s;
    const AIMA_GLOBAL uint8_t* rs1 = uptr(Ly.gs1) + (size_t)e * Ly.estride_s;
    const AIMA_GLOBAL uint8_t* rz0 = uptr(Ly.gz0) + (size_t)e * Ly.estride_z;
    const AIMA_GLOBAL uint8_t* rz1 = uptr(Ly.gz1) + (size_t)e * Ly.estride_z;
    const AIMA_GLOBAL uint8_t* hs = up ? uptr(Ly.ss1) : uptr(Ly.ss0);
    const AIMA_GLOBAL uint8_t* hz = up ? uptr(Ly.sz1) : uptr(Ly.sz0);
    const AIMA_GLOBAL uint8_t* rs = up ? rs1 : rs0;
    const AIMA_GLOBAL uint8_t* rz = up ? rz1 : rz0;
    const AIMA_GLOBAL uint8_t* base = is_s ? (routed ? rs : hs) : (routed ? rz : hz);
    const uint32_t off = is_s ? (uint32_t)unit * 32 + 4 * w : (uint32_t)unit * 8 + 4 * w;
    gsa_n = *reinterpret_cast<const AIMA_GLOBAL uint32_t*>(base + off);
  };
  // down gather (4 groups per row; the wave's 8 rows are consecutive):
  // lanes 0..15 = routed scale words, 16..19 = routed zero-point words,
  // 20..35 = shared scale words, 36..39 = shared zero-point words
  auto gather_b = [&](const PlanLayer& Ly, uint32_t e) {
    const int ln = opaque_v(threadIdx.x & 63);
    const uint32_t sbytes = (uint32_t)kH * 4 * 2;
    const uint32_t zbytes = (uint32_t)kH * 4 / 2;
    const uint32_t h0 = (uint32_t)(j * kRowsB + wave * kWaveRowsB);
    const int q = min(ln, 39);
    const AIMA_GLOBAL uint8_t* rs = uptr(Ly.ds) + (size_t)e * sbytes;
    const AIMA_GLOBAL uint8_t* rz = uptr(Ly.dz) + (size_t)e * zbytes;
    const AIMA_GLOBAL uint8_t* hs = uptr(Ly.sds);
    const AIMA_GLOBAL uint8_t* hz = uptr(Ly.sdz);
    const AIMA_GLOBAL uint8_t* base = q < 16 ? rs : q < 20 ? rz : q < 36 ? hs : hz;
    const uint32_t off = q < 16   ? h0 * 8 + 4 * q
                         : q < 20 ? h0 * 2 + 4 * (q - 16)
                         : q < 36 ? h0 * 8 + 4 * (q - 20)
                                  : h0 * 2 + 4 * (q - 36);
    gsb_n = *reinterpret_cast<const AIMA_GLOBAL uint32_t*>(base + off);
  };
  // gate/up rows: block row ri = 2 * (local pair) + (0 gate | 1 up); wave w
  // takes ri = ((w + 4) & 7) + 8 i, so waves 4..7 carry the fifth row and the
  // control duties of wave 0 fall on a wave with four.  prefetch_a1 loads the
  // wave's row slot i, prefetch_a all of them (a surplus slot is clamped onto
  // the block's last row).
  auto prefetch_a1 = [&](const PlanLayer& Ly, uint32_t e, int i) {
    const int ln = opaque_v(threadIdx.x & 63);
    const int ri = min(((wave + 4) & 7) + kWaves * i, kRowsA - 1);
    const int h = ri & 1;
    const int p = j * kPairs + (ri >> 1);
    const bool routed = p < kI;
    const AIMA_GLOBAL uint8_t* w =
        routed ? uptr(h ? Ly.gq1 : Ly.gq0) + (size_t)e * Ly.estride_q
               : uptr(h ? Ly.sq1 : Ly.sq0);
    const AIMA_GLOBAL uint8_t* sp =
        routed ? uptr(h ? Ly.gs1 : Ly.gs0) + (size_t)e * Ly.estride_s
               : uptr(h ? Ly.ss1 : Ly.ss0);
    const AIMA_GLOBAL uint8_t* zp =
        routed ? uptr(h ? Ly.gz1 : Ly.gz0) + (size_t)e * Ly.estride_z
               : uptr(h ? Ly.sz1 : Ly.sz0);
    const int unit = routed ? p : x * kSlice + (p - kI);
    const int gi = unit * gA + ((ln * 32) >> glog2);
    wa_n[i] = ld_w(w, (uint32_t)unit * (kH / 2) + ln * 16);
    if (g128) {
      if (i == 0) gather_a(Ly, e);
    } else {
      sa_n[i] = ld_u32(sp, (gi * 2) & ~3);
      za_n[i] = ld_u32(zp, (gi >> 1) & ~3);
    }
  };
  auto prefetch_a = [&](const PlanLayer& Ly, uint32_t e) {
#pragma unroll
    for (int i = 0; i < kMaxRowsA; ++i) prefetch_a1(Ly, e, i);
  };
  // down rows: wave w owns block rows 8w .. 8w+7; units 0, 1 = routed rows
  // 4u + (lane >> 4), chunk lane & 15; unit 2 = the shared slice, row
  // (lane & 15) >> 1, chunk 2x + (lane & 1) of the full shared row
  auto prefetch_b = [&](const PlanLayer& Ly, uint32_t e) {
    const int ln = opaque_v(threadIdx.x & 63);
    const uint32_t wbytes = (uint32_t)kH * (kI / 2);
    const uint32_t sbytes = (uint32_t)kH * gB * 2;
    const uint32_t zbytes = (uint32_t)kH * gB / 2;
    const AIMA_GLOBAL uint8_t* rw = uptr(Ly.dq) + (size_t)e * wbytes;
    const AIMA_GLOBAL uint8_t* rs = uptr(Ly.ds) + (size_t)e * sbytes;
    const AIMA_GLOBAL uint8_t* rz = uptr(Ly.dz) + (size_t)e * zbytes;
    const int h0 = j * kRowsB + wave * kWaveRowsB;
#pragma unroll
    for (int u = 0; u < 2; ++u) {
      const int row = h0 + 4 * u + (ln >> 4);
      const int cl = ln & 15;
      const int gi = row * gB + ((cl * 32) >> glog2);
      wb_n[u] = ld_w(rw, (uint32_t)row * (kI / 2) + cl * 16);
      if (!g128) {
        sb_n[u] = ld_u32(rs, (gi * 2) & ~3);
        zb_n[u] = ld_u32(rz, (gi >> 1) & ~3);
      }
    }
    {
      const int row = h0 + ((ln & 15) >> 1);
      const int ch = 2 * x + (ln & 1);
      const int gi = row * gB + ((ch * 32) >> glog2);
      wb_n[2] = ld_w(uptr(Ly.sdq), (uint32_t)x * (kH * 32) + row * 32 + (ln & 1) * 16);
      if (!g128) {
        sb_n[2] = ld_u32(uptr(Ly.sds), (gi * 2) & ~3);
        zb_n[2] = ld_u32(uptr(Ly.sdz), (gi >> 1) & ~3);
      }
    }
    if (g128) gather_b(Ly, e);
  };
  // All gate/up rows of layer L in one burst (routed plan): the table fields
  // are read first and each row's base chosen by selects, so the loads leave
  // back to back (the loaders above read the table per row, which the
  // prefetch interleaved with the dot products can afford; a burst that
  // starts when the route is known cannot).  Same rows, lanes and clamping
  // as prefetch_a and gather_a, but the rows go straight into the working
  // registers, the gathering load first: each dot product then waits for its
  // own row only (take_gather_a hands the scale and zero-point words out once
  // the gather has landed).  The layer's down rows follow with prefetch_b
  // once the wave's gate/up dot products are done (see the routed layer).
  auto issue_rows_a = [&](int L) {
    const int ln = opaque_v(threadIdx.x & 63);
    const PlanLayer& T = S.table[L];
    const uint32_t e = slot_expert(L);
    const uint64_t eq = (uint64_t)e * T.estride_q, es = (uint64_t)e * T.estride_s,
                   ez = (uint64_t)e * T.estride_z;
    const AIMA_GLOBAL uint8_t *rq0 = uptr(T.gq0) + eq, *rq1 = uptr(T.gq1) + eq;
    const AIMA_GLOBAL uint8_t *rs0 = uptr(T.gs0) + es, *rs1 = uptr(T.gs1) + es;
    const AIMA_GLOBAL uint8_t *rz0 = uptr(T.gz0) + ez, *rz1 = uptr(T.gz1) + ez;
    const AIMA_GLOBAL uint8_t *hq0 = uptr(T.sq0), *hq1 = uptr(T.sq1);
    const AIMA_GLOBAL uint8_t *hs0 = uptr(T.ss0), *hs1 = uptr(T.ss1);
    const AIMA_GLOBAL uint8_t *hz0 = uptr(T.sz0), *hz1 = uptr(T.sz1);
    if (g128) {
      const int q = min(ln, 49);
      const bool is_s = q < 40;
      const int i = is_s ? (q >> 3) : ((q - 40) >> 1);
      const int w = is_s ? (q & 7) : ((q - 40) & 1);
      const int ri = min(((wave + 4) & 7) + kWaves * i, kRowsA - 1);
      const int p = j * kPairs + (ri >> 1);
      const bool routed = p < kI;
      const int unit = routed ? p : x * kSlice + (p - kI);
      const bool up = (ri & 1) != 0;
      const AIMA_GLOBAL uint8_t* base =
          is_s ? (routed ? (up ? rs1 : rs0) : (up ? hs1 : hs0))
               : (routed ? (up ? rz1 : rz0) : (up ? hz1 : hz0));
      const uint32_t off = is_s ? (uint32_t)unit * 32 + 4 * w : (uint32_t)unit * 8 + 4 * w;
      gsa_n = *reinterpret_cast<const AIMA_GLOBAL uint32_t*>(base + off);
    }
    // gate/up rows
#pragma unroll
    for (int i = 0; i < kMaxRowsA; ++i) {
      const int ri = min(((wave + 4) & 7) + kWaves * i, kRowsA - 1);
      const bool h = (ri & 1) != 0;
      const int p = j * kPairs + (ri >> 1);
      const bool routed = p < kI;
      const int unit = routed ? p : x * kSlice + (p - kI);
      wa[i] = ld_w(routed ? (h ? rq1 : rq0) : (h ? hq1 : hq0),
                   (uint32_t)unit * (kH / 2) + ln * 16);
      if (!g128) {
        const int gi = unit * gA + ((ln * 32) >> glog2);
        sa[i] = ld_u32(routed ? (h ? rs1 : rs0) : (h ? hs1 : hs0), (gi * 2) & ~3);
        za[i] = ld_u32(routed ? (h ? rz1 : rz0) : (h ? hz1 : hz0), (gi >> 1) & ~3);
      }
    }
  };
  // this wave's 256 norm-weight floats and gate-vector halves: lane l holds
  // values 256 w + 4 l .. +3
  auto load_vec = [&](int L) {
    const int ln = opaque_v(threadIdx.x & 63);
    const PlanLayer& Ly = S.table[L];
    const int v0 = wave * 256 + ln * 4;
    nw_n = gload16(Ly.norm + v0);
    gv_n = *reinterpret_cast<const AIMA_GLOBAL u32x2*>(uptr(Ly.gate_vec) + v0 * 2);
  };
  // routed plan: this wave's router row, expert 8j + w (clamped onto the
  // last expert past the expert count), one 32-value chunk per lane
  u32x4 rw = {}, rw_n = {};
  uint32_t rsw = 0, rsw_n = 0, rzw = 0, rzw_n = 0;
  auto router_row = [&]() { return min(j * kWaves + wave, a.experts - 1); };
  auto prefetch_router = [&](int L) {
    const int ln = opaque_v(threadIdx.x & 63);
    const PlanLayer& Ly = S.table[L];
    const int e = router_row();
    const int gi = e * gA + ((ln * 32) >> glog2);
    rw_n = ld_w(uptr(Ly.rq), (uint32_t)e * (kH / 2) + ln * 16);
    rsw_n = ld_u32(uptr(Ly.rs), (gi * 2) & ~3);
    rzw_n = ld_u32(uptr(Ly.rz), (gi >> 1) & ~3);
  };
  // Moves the prefetched rows into the working registers (with 128-wide
  // groups, hands the gathered scale and zero-point words to their lanes).
  auto rotate_a = [&]() {
    const int ln = opaque_v(threadIdx.x & 63);
#pragma unroll
    for (int i = 0; i < kMaxRowsA; ++i) wa[i] = wa_n[i];
    if (g128) {
      // lane l: gate/up group l / 4 of row slot i
#pragma unroll
      for (int i = 0; i < kMaxRowsA; ++i) {
        sa[i] = (uint32_t)__builtin_amdgcn_ds_bpermute((8 * i + (ln >> 3)) * 4, (int)gsa_n);
        za[i] = (uint32_t)__builtin_amdgcn_ds_bpermute((40 + 2 * i + (ln >> 5)) * 4, (int)gsa_n);
      }
    } else {
#pragma unroll
      for (int i = 0; i < kMaxRowsA; ++i) {
        sa[i] = sa_n[i];
        za[i] = za_n[i];
      }
    }
  };
  // Routed plan: the gathered gate/up scale and zero-point words to their
  // lanes (the rows themselves were loaded in place).
  auto take_gather_a = [&]() {
    const int ln = opaque_v(threadIdx.x & 63);
    if (g128) {
#pragma unroll
      for (int i = 0; i < kMaxRowsA; ++i) {
        sa[i] = (uint32_t)__builtin_amdgcn_ds_bpermute((8 * i + (ln >> 3)) * 4, (int)gsa_n);
        za[i] = (uint32_t)__builtin_amdgcn_ds_bpermute((40 + 2 * i + (ln >> 5)) * 4, (int)gsa_n);
      }
    }
  };
  auto rotate_b = [&]() {
    const int ln = opaque_v(threadIdx.x & 63);
#pragma unroll
    for (int u = 0; u < 3; ++u) wb[u] = wb_n[u];
    if (g128) {
      // down routed row 4u + l / 16, group (l & 15) / 4; shared row
      // (l & 15) / 2, group x / 2
      auto pick = [](uint32_t v, int src) {
        return (uint32_t)__builtin_amdgcn_ds_bpermute(src * 4, (int)v);
      };
#pragma unroll
      for (int u = 0; u < 2; ++u) {
        const int r = 4 * u + (ln >> 4);
        sb[u] = pick(gsb_n, 2 * r + ((ln & 15) >> 3));
        zb[u] = pick(gsb_n, 16 + (r >> 1));
      }
      const int r8 = (ln & 15) >> 1;
      sb[2] = pick(gsb_n, 20 + 2 * r8 + (x >> 2));
      zb[2] = pick(gsb_n, 36 + (r8 >> 1));
    } else {
#pragma unroll
      for (int u = 0; u < 3; ++u) {
        sb[u] = sb_n[u];
        zb[u] = zb_n[u];
      }
    }
  };
  // Phase A's dot products: the block's 36 gate/up rows against the
  // operands in xc, row sums to LDS.  The logits-fed plan loads one row of
  // the next layer per dot product (held in place by a scheduling barrier);
  // the routed plan has no prefetch to pace, so every slot is computed (a
  // surplus one on the clamped row it loaded, result dropped) and the five
  // dot products can interleave.
  auto dots_a = [&](const XChunk& xc, int L) {
    const int ln = opaque_v(threadIdx.x & 63);
#pragma unroll
    for (int i = 0; i < kMaxRowsA; ++i) {
      const int ri = ((wave + 4) & 7) + kWaves * i;
      if (!ROUTED && !RING) {
        if (L + 1 < a.n_layers) prefetch_a1(S.table[L + 1], slot_expert(L + 1), i);
        __builtin_amdgcn_sched_barrier(0);
      }
      if (ROUTED || ri < kRowsA) {
        const int rc = min(ri, kRowsA - 1);
        const int p = j * kPairs + (rc >> 1);
        const int unit = p < kI ? p : x * kSlice + (p - kI);
        const int gi = unit * gA + ((ln * 32) >> glog2);
        const float dd =
            segment_sum<16>(lane_dot(wa[i], xc, nib(za[i], gi), scl(sa[i], gi), magic));
        if ((ln & 15) == 0 && ri < kRowsA) S.rowpart[ri][ln >> 4] = dd;
      }
    }
  };

  // ---- the streaming wave (ring instance) -------------------------------------
  // Layer M's rows go to ring slot M & 1 in four batches (t = 0, 1: gate/up
  // rows 18 t .. 18 t + 17; t = 2: the gate/up scale and zero-point words and
  // the routed down rows of unit 0 of the 8 compute waves; t = 3: the routed
  // down rows of unit 1, the shared down slices and the down scale and
  // zero-point words).  The addresses are prefetch_a1's, gather_a's,
  // prefetch_b's and gather_b's for every compute wave in turn.  Batch t of
  // layer L + 1 is issued after barrier #(t + 1) of layer L and written to
  // LDS after the next barrier, so at most one batch (18 KB) is in flight and
  // everything of layer L + 1 is in its slot by barrier #1 of layer L + 1
  // (the compute waves read gate/up rows after #2, down rows after #4;
  // layer 0: the compute waves fill slot 0 themselves).  Slot (L + 1) & 1 was
  // last read in phase B of layer L - 1, which ends before barrier #1 of
  // layer L; the first write into it follows barrier #2 of layer L.  The wave
  // passes the same barriers as the compute waves -- the two of the prologue
  // above, then #1 .. #4 of every layer -- and returns where they return
  // (S.abort is only written before a barrier that precedes its check).
  auto stream_rows = [&]() {
    u32x4 buf[kPairs];      // row loads in flight (one batch)
    uint32_t g2[8], g3[5];  // scale / zero-point words of batches 2 and 3
    // (lane-derived offsets from a fresh opaque lane index per call: hoisted
    // out of the layer loop they would stay live across it and spill)
    auto issue = [&](int M, int t, int at) {
      const int ln = opaque_v(threadIdx.x & 63);
      const PlanLayer& T = S.table[M];
      const uint32_t e = slot_expert(M);
      const uint64_t eq = (uint64_t)e * T.estride_q, es = (uint64_t)e * T.estride_s,
                     ez = (uint64_t)e * T.estride_z;
      if (t < 2) {
        const AIMA_GLOBAL uint8_t *rq0 = uptr(T.gq0) + eq, *rq1 = uptr(T.gq1) + eq;
        const AIMA_GLOBAL uint8_t *hq0 = uptr(T.sq0), *hq1 = uptr(T.sq1);
#pragma unroll
        for (int q = 0; q < kPairs; ++q) {
          const int ri = kPairs * t + q;
          const bool h = (ri & 1) != 0;
          const int p = j * kPairs + (ri >> 1);
          const bool routed = p < kI;
          const int unit = routed ? p : x * kSlice + (p - kI);
          buf[at + q] = ld_w(routed ? (h ? rq1 : rq0) : (h ? hq1 : hq0),
                             (uint32_t)unit * (kH / 2) + ln * 16);
        }
        return;
      }
      const AIMA_GLOBAL uint8_t* dw = uptr(T.dq) + (size_t)e * ((uint32_t)kH * (kI / 2));
      if (t == 2) {
        // The block's pairs are consecutive units -- routed up to pair
        // kI - 1, then shared-slice units -- so each kind of word is one
        // run in memory (gate scales, up scales, gate zero points, up zero
        // points): lane-linear loads, word u from the routed tensor while u
        // is below the routed pairs' words, else from the shared one.
        const int p0 = j * kPairs;            // the block's first pair
        const int su = x * kSlice - kI + p0;  // shared unit of pair p0 (< 0: routed pairs first)
        const int rp = kI - p0;               // routed pairs of the block (<= 0: none)
        auto word = [&](const AIMA_GLOBAL uint8_t* r, const AIMA_GLOBAL uint8_t* h, int per,
                        int u) {  // per: bytes per unit
          const bool routed = u < rp * (per / 4);
          const uint32_t off = (uint32_t)(4 * u + (routed ? p0 : su) * per);
          return *reinterpret_cast<const AIMA_GLOBAL uint32_t*>((routed ? r : h) + off);
        };
#pragma unroll
        for (int g = 0; g < 3; ++g) {
          const int u = min(64 * g + ln, kPairs * 8 - 1);
          g2[g] = word(uptr(T.gs0) + es, uptr(T.ss0), 32, u);
          g2[3 + g] = word(uptr(T.gs1) + es, uptr(T.ss1), 32, u);
        }
        const int uz = min(ln, kPairs * 2 - 1);
        g2[6] = word(uptr(T.gz0) + ez, uptr(T.sz0), 8, uz);
        g2[7] = word(uptr(T.gz1) + ez, uptr(T.sz1), 8, uz);
#pragma unroll
        for (int wv = 0; wv < kWaves; ++wv) {
          const int row = j * kRowsB + wv * kWaveRowsB + (ln >> 4);
          buf[at + wv] = ld_w(dw, (uint32_t)row * (kI / 2) + (ln & 15) * 16);
        }
        return;
      }
#pragma unroll
      for (int wv = 0; wv < kWaves; ++wv) {
        const int row = j * kRowsB + wv * kWaveRowsB + 4 + (ln >> 4);
        buf[at + wv] = ld_w(dw, (uint32_t)row * (kI / 2) + (ln & 15) * 16);
      }
#pragma unroll
      for (int g = 0; g < 2; ++g) {
        const int wv = 4 * g + (ln >> 4);
        const int row = j * kRowsB + wv * kWaveRowsB + ((ln & 15) >> 1);
        buf[at + kWaves + g] =
            ld_w(uptr(T.sdq), (uint32_t)x * (kH * 32) + row * 32 + (ln & 1) * 16);
      }
      // the block's 64 down rows hold 128 consecutive scale words and 32
      // zero-point words in each of the routed and the shared tensors
      const uint32_t sbytes = (uint32_t)kH * 4 * 2;
      const uint32_t zbytes = (uint32_t)kH * 4 / 2;
      const AIMA_GLOBAL uint8_t* rs = uptr(T.ds) + (size_t)e * sbytes + j * kRowsB * 8;
      const AIMA_GLOBAL uint8_t* hs = uptr(T.sds) + j * kRowsB * 8;
      const AIMA_GLOBAL uint8_t* rz = uptr(T.dz) + (size_t)e * zbytes + j * kRowsB * 2;
      const AIMA_GLOBAL uint8_t* hz = uptr(T.sdz) + j * kRowsB * 2;
      auto ld32 = [](const AIMA_GLOBAL uint8_t* q) {
        return *reinterpret_cast<const AIMA_GLOBAL uint32_t*>(q);
      };
      g3[0] = ld32(rs + 4 * ln);
      g3[1] = ld32(rs + 256 + 4 * ln);
      g3[2] = ld32(hs + 4 * ln);
      g3[3] = ld32(hs + 256 + 4 * ln);
      g3[4] = ld32((ln < 32 ? rz : hz) + 4 * (ln & 31));
    };
    auto write = [&](int M, int t, int at) {
      const int ln = opaque_v(threadIdx.x & 63);
      RingSlot& R = ring[M & 1];
      if (t < 2) {
#pragma unroll
        for (int q = 0; q < kPairs; ++q) R.a[kPairs * t + q][ln] = buf[at + q];
        return;
      }
      if (t == 2) {
#pragma unroll
        for (int g = 0; g < 3; ++g) {
          const int u = 64 * g + ln;
          if (u < kPairs * 8) {
            R.as[u] = g2[g];
            R.as[kPairs * 8 + u] = g2[3 + g];
          }
        }
        if (ln < kPairs * 2) {
          R.az[ln] = g2[6];
          R.az[kPairs * 2 + ln] = g2[7];
        }
#pragma unroll
        for (int wv = 0; wv < kWaves; ++wv) R.b[wv][0][ln] = buf[at + wv];
        return;
      }
#pragma unroll
      for (int wv = 0; wv < kWaves; ++wv) R.b[wv][1][ln] = buf[at + wv];
#pragma unroll
      for (int g = 0; g < 2; ++g) R.bs[4 * g + (ln >> 4)][ln & 15] = buf[at + kWaves + g];
#pragma unroll
      for (int g = 0; g < 4; ++g) R.bgs[64 * g + ln] = g3[g];
      R.bgz[ln] = g3[4];
    };
    for (int L = 0; L < a.n_layers; ++L) {
      const int M = L + 1;
      const bool more = M < a.n_layers;
      __syncthreads();  // #1
      if (S.abort) return;
      if (L > 0) write(L, 3, 0);
      AIMA_TRACE(L, 13, kWaves * 64);  // batch 3 written (stream)
      if (more) issue(M, 0, 0);
      AIMA_TRACE(L, 26, kWaves * 64);  // batch 3 written, batch 0 issued (stream)
      __syncthreads();  // #2
      if (more) {
        write(M, 0, 0);
        AIMA_TRACE(L, 17, kWaves * 64);  // batch 0 written (stream)
        issue(M, 1, 0);
      }
      AIMA_TRACE(L, 27, kWaves * 64);  // batch 0 written, batch 1 issued (stream)
      __syncthreads();  // #3
      AIMA_TRACE(L, 21, kWaves * 64);  // #3 passed (stream)
      if (more) {
        write(M, 1, 0);
        AIMA_TRACE(L, 22, kWaves * 64);  // batch 1 written (stream)
        issue(M, 2, 0);
      }
      AIMA_TRACE(L, 23, kWaves * 64);  // at #4 (stream)
      __syncthreads();  // #4
      if (S.abort) return;
      if (more) {
        write(M, 2, 0);
        issue(M, 3, 0);
      }
      AIMA_TRACE(L, 24, kWaves * 64);  // batch 2 written, batch 3 issued (stream)
    }
  };
  if constexpr (RING) {
    if (wave == kWaves) {
      stream_rows();
      return;
    }
  }
  load_vec(0);
  if (ROUTED) {
    prefetch_router(0);
  } else {
    prefetch_a(S.table[0], slot_expert(0));
    prefetch_b(S.table[0], slot_expert(0));
  }
  if (RING) {
    // layer 0's rows: every compute wave writes what it loaded into slot 0,
    // in the streaming wave's layout (row slots past the block's 36 rows and
    // the duplicate lanes of the shared slice and the gathers write nothing)
    RingSlot& R = ring[0];
    const int ln = opaque_v(threadIdx.x & 63);
#pragma unroll
    for (int i = 0; i < kMaxRowsA; ++i) {
      const int ri = ((wave + 4) & 7) + kWaves * i;
      if (ri < kRowsA) R.a[ri][ln] = wa_n[i];
    }
    if (ln < 40) {
      const int ri = ((wave + 4) & 7) + kWaves * (ln >> 3);
      if (ri < kRowsA) R.as[(ri & 1) * (kPairs * 8) + (ri >> 1) * 8 + (ln & 7)] = gsa_n;
    } else if (ln < 50) {
      const int ri = ((wave + 4) & 7) + kWaves * ((ln - 40) >> 1);
      if (ri < kRowsA) R.az[(ri & 1) * (kPairs * 2) + (ri >> 1) * 2 + ((ln - 40) & 1)] = gsa_n;
    }
    R.b[wave][0][ln] = wb_n[0];
    R.b[wave][1][ln] = wb_n[1];
    if (ln < 16) R.bs[wave][ln] = wb_n[2];
    if (ln < 16) {
      R.bgs[wave * 16 + ln] = gsb_n;
    } else if (ln < 20) {
      R.bgz[wave * 4 + ln - 16] = gsb_n;
    } else if (ln < 36) {
      R.bgs[kWaves * 16 + wave * 16 + ln - 20] = gsb_n;
    } else if (ln < 40) {
      R.bgz[kWaves * 4 + wave * 4 + ln - 36] = gsb_n;
    }
  }
  AIMA_TRACE(40, 1, 0);  // prologue done

  for (int L = 0; L < a.n_layers; ++L) {
    const int ln = opaque_v(threadIdx.x & 63);
    const uint32_t epA = base + 2u * (uint32_t)L;        // act_L
    const uint32_t epP = base + 2u * (uint32_t)L + 1u;   // P_L
    const uint32_t epR = base + 2u * (uint32_t)L - 1u;   // r_L (L > 0)
    const int par = L & 1;

    // ================= phase A_L =================
    // every wave reads its 256 values of r_L (one 16-byte load per lane)
    uint32_t rv[4];
    if (L == 0) {
      const u32x2 v = *(const AIMA_GLOBAL u32x2*)(a.r0 + wave * 256 + ln * 4);
      rv[0] = v[0] & 0xffffu;
      rv[1] = v[0] >> 16;
      rv[2] = v[1] & 0xffffu;
      rv[3] = v[1] >> 16;
    } else {
      const uint32_t* src = a.rx + ((size_t)x * 2 + par) * kH + wave * 256 + ln * 4;
      uint32_t spins = 0;
      while (true) {
        const u32x4 v = poll1(src);
        bool ok = true;
#pragma unroll
        for (int t = 0; t < 4; ++t) {
          rv[t] = v[t];
          ok = ok && (v[t] >> 16) == epR;
        }
        if (__all(ok)) break;
        if (++spins > kSpinLimit) {
          fail_timeout();
          break;
        }
      }
    }
    AIMA_TRACE(L, 0, 64);  // r_L read (wave 1)
    float rf[4];
    float ss = 0.f;
#pragma unroll
    for (int t = 0; t < 4; ++t) {
      rf[t] = h2f((uint16_t)rv[t]);
      ss += rf[t] * rf[t];
    }
    ss = segment_sum<64>(ss);
    if (lane == 0) S.ss[wave] = ss;
    *reinterpret_cast<u32x2*>(&S.rl[wave * 128 + ln * 2]) =
        u32x2{(rv[0] & 0xffffu) | (rv[1] << 16), (rv[2] & 0xffffu) | (rv[3] << 16)};
    if (!ROUTED) AIMA_TRACE(L, 14, 0);  // at #1 (wave 0)
    __syncthreads();  // #1: r_L sums of squares
    AIMA_TRACE(L, 1, 0);
    if (S.abort) {
      finish();
      return;
    }
    if (RING) {
      // the rows come from the ring after barrier #2 and #4
    } else if (!ROUTED) {
      rotate_a();
      rotate_b();
    } else {
      rw = rw_n;
      rsw = rsw_n;
      rzw = rzw_n;
    }
    nw = nw_n;
    gv = gv_n;
    // RMSNorm: x = f16(r * rsqrt(mean(r^2) + eps) * w), this wave's values;
    // lane l holds part l & 7 (values 4p .. 4p+3) of chunk 8w + (l >> 3)
    {
      float sst = 0.f;
#pragma unroll
      for (int w = 0; w < kWaves; ++w) sst += S.ss[w];
      const float scale = 1.0f / sqrtf(sst / (float)kH + a.eps);
      uint16_t xh[4];
#pragma unroll
      for (int t = 0; t < 4; ++t) xh[t] = f2h_rounded(rf[t] * scale * as_f32(nw[t]));
      const uint32_t X0 = (uint32_t)xh[0] | ((uint32_t)xh[1] << 16);
      const uint32_t X1 = (uint32_t)xh[2] | ((uint32_t)xh[3] << 16);
      // partner lane (l ^ 1) holds the other half of the 8-value word group
      const uint32_t Y0 = (uint32_t)__builtin_amdgcn_update_dpp(0, (int)X0, 0xB1, 0xF, 0xF, false);
      const uint32_t Y1 = (uint32_t)__builtin_amdgcn_update_dpp(0, (int)X1, 0xB1, 0xF, 0xF, false);
      const bool hi = (ln & 1) != 0;
      // low half (values 8d..8d+3): pairs (x0,x4), (x1,x5); high half: (x2,x6), (x3,x7)
      const uint32_t lo_src = hi ? Y1 : X0;
      const uint32_t hi_src = hi ? X1 : Y0;
      const uint32_t p0 = __builtin_amdgcn_perm(hi_src, lo_src, 0x05040100u);
      const uint32_t p1 = __builtin_amdgcn_perm(hi_src, lo_src, 0x07060302u);
      const int c = wave * 8 + (ln >> 3);
      const int d = (ln & 7) >> 1;
      *reinterpret_cast<u32x2*>(reinterpret_cast<char*>(&S.xa_p[d][c]) + (hi ? 8 : 0)) =
          u32x2{p0, p1};
      float xe = h2f(xh[0]) + h2f(xh[2]);
      float xo = h2f(xh[1]) + h2f(xh[3]);
      xe = segment_sum<8>(xe);
      xo = segment_sum<8>(xo);
      if ((ln & 7) == 0) {
        S.xa_bias[c] = 1024.f * xe + 64.f * xo;
        S.xa_xsum[c] = xe + xo;
      }
      // shared-expert gate: partial dot of this wave's values
      const f16x2 g0 = as_h2(gv[0]), g1 = as_h2(gv[1]);
      float g = (float)g0.x * h2f(xh[0]);
      g += (float)g0.y * h2f(xh[1]);
      g += (float)g1.x * h2f(xh[2]);
      g += (float)g1.y * h2f(xh[3]);
      g = segment_sum<64>(g);
      if (lane == 0) S.gp[wave] = g;
    }
    if (!ROUTED) {
      AIMA_TRACE(L, 11, 0);    // at #2 (wave 0)
      AIMA_TRACE(L, 12, 256);  // at #2 (wave 4)
    }
    __syncthreads();  // #2: A operands ready
    AIMA_TRACE(L, 2, 0);
    if (!ROUTED && L + 1 < a.n_layers) {
      load_vec(L + 1);
      if (!RING) prefetch_b(S.table[L + 1], slot_expert(L + 1));
    }
    if (RING) {
      // this layer's gate/up rows and their scale / zero-point words
      const RingSlot& R = ring[L & 1];
#pragma unroll
      for (int i = 0; i < kMaxRowsA; ++i) {
        const int ri = min(((wave + 4) & 7) + kWaves * i, kRowsA - 1);
        wa[i] = R.a[ri][ln];
        sa[i] = R.as[(ri & 1) * (kPairs * 8) + (ri >> 1) * 8 + (ln >> 3)];
        za[i] = R.az[(ri & 1) * (kPairs * 2) + (ri >> 1) * 2 + (ln >> 5)];
      }
    }
    {
      XChunk xc;
      get_chunk(S.xa_p, S.xa_bias, S.xa_xsum, ln, xc);
      if (ROUTED) {
        // router logit of expert 8j + w, published to the XCD
        const int e = j * kWaves + wave;
        const int gi = router_row() * gA + ((ln * 32) >> glog2);
        const float lg =
            segment_sum<64>(lane_dot(rw, xc, nib(rzw, gi), scl(rsw, gi), magic));
        if (lane == 0 && e < a.experts) {
          st_local64(&a.lgx[((size_t)x * 2 + par) * kRouterRows + e], pack_f32(lg, epA));
          if (x == 0 && a.logits_out) a.logits_out[(size_t)L * a.experts + e] = lg;
        }
        // waves 0 and 1: all logits of the layer (lane l: experts
        // l + 64 t); wave 0 ranks them, wave 1 computes the probabilities
        // (the same in every block)
        float pv[4];
        if (wave < 2) {
          const uint64_t* src = a.lgx + ((size_t)x * 2 + par) * kRouterRows + ln;
          uint64_t v[4];
          uint32_t spins = 0;
          while (true) {
            poll4(src, 64 * 8, v);
            bool ok = true;
#pragma unroll
            for (int t = 0; t < 4; ++t)
              ok = ok && (ln + 64 * t >= a.experts || (uint32_t)(v[t] >> 32) == epA);
            if (__all(ok)) break;
            if (++spins > kSpinLimit) {
              fail_timeout();
              break;
            }
          }
          AIMA_TRACE(L, 11, 0);  // logits read
          float lv[4];
#pragma unroll
          for (int t = 0; t < 4; ++t) lv[t] = as_f32((uint32_t)v[t]);
          if (wave == 0) {
            const int rank_id = rank_logits(lv, a.experts, k);
            if (ln <= k) S.rank[ln] = rank_id;
            if (ln < k) S.route_id[L][ln] = rank_id;
            AIMA_TRACE(L, 16, 0);  // ranked (wave 0)
          } else {
            softmax_probs(lv, a.experts, pv);
            AIMA_TRACE(L, 17, 64);  // probabilities (wave 1)
          }
        }
        __syncthreads();  // #2b: the layer's route by the ranking
        AIMA_TRACE(L, 12, 0);
        if (S.abort) {
          finish();
          return;
        }
        // every wave issues the layer's gate/up rows from that ranking; wave
        // 1 then checks it while the loads are in flight (a changed route is
        // loaded again after barrier #3)
        issue_rows_a(L);
        AIMA_TRACE(L, 14, 128);  // loads issued (wave 2)
        AIMA_TRACE(L, 18, 64);   // loads issued (wave 1)
        if (wave == 1) {
          int id = ln <= k ? S.rank[ln] : -1;
          float w = 0.f;
          const bool same = route_confirm(pv, a.experts, id, k, a.min_weight_sum, w);
          if (!same) select_probs(pv, a.experts, k, a.min_weight_sum, id, w);
          if (ln < k) {
            // non-finite logits select nothing: flagged, the slot is dropped
            if (id < 0 || id >= a.experts) {
              atomicOr(a.err, AIMA_DEVERR_EXPERT_RANGE);
              id = -1;
            }
            // (the ranking's ids stand unless the route changed; the other
            // waves may be reading them for their loads)
            if (!same) S.route_id[L][ln] = id;
            S.route_w[L][ln] = w;
            if (b == 0 && a.ids_out) a.ids_out[L * k + ln] = id;
            if (b == 0 && a.w_out) a.w_out[L * k + ln] = w;
          }
          if (ln == 0) S.reroute = same ? 0 : 1;
          AIMA_TRACE(L, 15, 64);  // route confirmed (wave 1)
        }
        take_gather_a();
        AIMA_TRACE(L, 19, 256);  // gate/up scales in registers (wave 4)
      }
      dots_a(xc, L);
      AIMA_TRACE(L, 28, 0);    // A dots done (wave 0)
      AIMA_TRACE(L, 29, 64);   // A dots done (wave 1)
      AIMA_TRACE(L, 30, 320);  // A dots done (wave 5)
      // routed plan: the layer's down rows once the wave's gate/up rows are
      // consumed.  Issued with the gate/up burst they shared each CU's
      // memory queue with it and delayed the last gate/up row; here they
      // land during the SwiGLU, the activation exchange and its staging.
      if (ROUTED) prefetch_b(S.table[L], slot_expert(L));
    }
    if (wave == 0) {
      // shared-expert gate sigma = sigmoid(gate_vec . x), per block
      float g = 0.f;
#pragma unroll
      for (int w = 0; w < kWaves; ++w) g += S.gp[w];
      if (lane == 0) {
        const double t = g;
        S.sigma = (float)(t >= 0.0 ? 1.0 / (1.0 + exp(-t)) : exp(t) / (1.0 + exp(t)));
      }
    }
    AIMA_TRACE(L, 3, 256);  // A dots done (wave 4)
    __syncthreads();  // #3: row sums ready
    if (ROUTED && S.reroute) {
      // the probabilities did not confirm the ranking (ties or near ties):
      // the confirmed route's rows, and the dot products again
      issue_rows_a(L);
      take_gather_a();
      XChunk xc;
      get_chunk(S.xa_p, S.xa_bias, S.xa_xsum, ln, xc);
      dots_a(xc, L);
      prefetch_b(S.table[L], slot_expert(L));
      __syncthreads();  // #3r: row sums of the confirmed route
    }
    AIMA_TRACE(L, 4, 0);
    if (wave == 0) {
      // SwiGLU for the block's 18 pairs, one pair per lane (three pairs per
      // lane in turn: 0.44 against 0.24-0.32 us from barrier #3 to the
      // published record; the wave runs alone here), then lane r < 6
      // publishes pairs 3r .. 3r + 2 as one record
      {
        const int lp = min(lane, kPairs - 1);
        auto row_total = [&](int ri) {
          const float4 q = *reinterpret_cast<const float4*>(&S.rowpart[ri][0]);
          return (q.x + q.y) + (q.z + q.w);
        };
        const int hv = (int)f2h_rounded(silu_mul(row_total(2 * lp), row_total(2 * lp + 1)));
        const uint32_t h0 = (uint32_t)__builtin_amdgcn_ds_bpermute(4 * (3 * lane), hv);
        const uint32_t h1 = (uint32_t)__builtin_amdgcn_ds_bpermute(4 * (3 * lane + 1), hv);
        const uint32_t h2 = (uint32_t)__builtin_amdgcn_ds_bpermute(4 * (3 * lane + 2), hv);
        if (lane < kPairs / 3) {
          const uint64_t rec = ((uint64_t)epA << 48) | ((uint64_t)(h2 & 0xffffu) << 32) |
                               ((h1 & 0xffffu) << 16) | (h0 & 0xffffu);
          st_local64(&a.actx[((size_t)x * 2 + par) * kActStride + j * (kPairs / 3) + lane], rec);
        }
      }
      AIMA_TRACE(L, 5, 0);  // act published
      // act_L of this XCD: 192 records, lanes read records 2l, 2l+1 and
      // 128 + 2(l & 31), +1
      const uint64_t* src = a.actx + ((size_t)x * 2 + par) * kActStride;
      const int r0 = 2 * ln, r1 = 128 + 2 * (ln & 31);
      uint32_t spins = 0;
      u32x4 v0, v1;
      while (true) {
        poll2(src + r0, src + r1, v0, v1);
        const bool ok = (v0[1] >> 16) == epA && (v0[3] >> 16) == epA &&
                        (v1[1] >> 16) == epA && (v1[3] >> 16) == epA;
        if (__all(ok)) break;
        if (++spins > kSpinLimit) {
          fail_timeout();
          break;
        }
      }
      AIMA_TRACE(L, 6, 0);  // act_L read
      // stage: record r holds act values 3r .. 3r+2 (f16 at byte 6r)
      auto stage = [&](int r, uint32_t lo, uint32_t hi) {
        uint8_t* d = reinterpret_cast<uint8_t*>(S.act);
        const bool even = (r & 1) == 0;
        const uint32_t word = even ? lo : ((lo >> 16) | (hi << 16));
        const uint16_t half = even ? (uint16_t)hi : (uint16_t)lo;
        *reinterpret_cast<uint32_t*>(d + 6 * r + (even ? 0 : 2)) = word;
        *reinterpret_cast<uint16_t*>(d + 6 * r + (even ? 4 : 0)) = half;
      };
      stage(r0, v0[0], v0[1]);
      stage(r0 + 1, v0[2], v0[3]);
      if (ln < 32) {
        stage(r1, v1[0], v1[1]);
        stage(r1 + 1, v1[2], v1[3]);
      }
      wave_lds_sync();
      // B operands: lane c < 18 builds chunk c (16 routed, 2 shared)
      if (ln < kChunksB) {
        XChunk c;
        lds_xchunk(S.act, ln * 16, c);
        put_chunk(S.xb_p, S.xb_bias, S.xb_xsum, ln, c);
      }
    }
    AIMA_TRACE(L, 25, 0);  // at #4 (wave 0)
    __syncthreads();  // #4: act_L operands staged
    AIMA_TRACE(L, 7, 0);
    if (S.abort) {
      finish();
      return;
    }
    if (ROUTED) {
      // the next layer's vectors and router rows (needed from its RMSNorm
      // on), then this layer's down rows into the working registers
      if (L + 1 < a.n_layers) {
        load_vec(L + 1);
        prefetch_router(L + 1);
      }
      rotate_b();
      AIMA_TRACE(L, 20, 0);  // down rows in registers (wave 0)
    }
    if (RING) {
      // this layer's down rows and their scale / zero-point words (the
      // lanes of rotate_b's picks)
      const RingSlot& R = ring[L & 1];
      wb[0] = R.b[wave][0][ln];
      wb[1] = R.b[wave][1][ln];
      wb[2] = R.bs[wave][ln & 15];
#pragma unroll
      for (int u = 0; u < 2; ++u) {
        const int r = 4 * u + (ln >> 4);
        sb[u] = R.bgs[wave * 16 + 2 * r + ((ln & 15) >> 3)];
        zb[u] = R.bgz[wave * 4 + (r >> 1)];
      }
      const int r8 = (ln & 15) >> 1;
      sb[2] = R.bgs[kWaves * 16 + wave * 16 + 2 * r8 + (x >> 2)];
      zb[2] = R.bgz[kWaves * 4 + wave * 4 + (r8 >> 1)];
    }
    // ================= phase B_L =================
    {
      const int h0 = j * kRowsB + wave * kWaveRowsB;
      const int cl = ln & 15;
      float dr[2];
#pragma unroll
      for (int u = 0; u < 2; ++u) {
        XChunk xc;
        get_chunk(S.xb_p, S.xb_bias, S.xb_xsum, cl, xc);
        const int row = h0 + 4 * u + (ln >> 4);
        const int gi = row * gB + ((cl * 32) >> glog2);
        dr[u] = segment_sum<16>(lane_dot(wb[u], xc, nib(zb[u], gi), scl(sb[u], gi), magic));
      }
      float ds;
      {
        XChunk xc;
        get_chunk(S.xb_p, S.xb_bias, S.xb_xsum, kI / 32 + (ln & 1), xc);
        const int row = h0 + ((ln & 15) >> 1);
        const int ch = 2 * x + (ln & 1);
        const int gi = row * gB + ((ch * 32) >> glog2);
        ds = segment_sum<2>(lane_dot(wb[2], xc, nib(zb[2], gi), scl(sb[2], gi), magic));
      }
      // lane r < 8 gathers row r: routed sum from lane 16 (r & 3) of unit
      // r >> 2, shared sum from lane 2r
      const float g0 = __shfl(dr[0], (ln & 3) * 16, 64);
      const float g1 = __shfl(dr[1], (ln & 3) * 16, 64);
      const float gs = __shfl(ds, 2 * (ln & 7), 64);
      const int eid = x < k ? S.route_id[L][x] : -1;
      const float c = eid >= 0 ? S.route_w[L][x] : 0.f;
      if (ln < kWaveRowsB) {
        const float dsel = ln < 4 ? g0 : g1;
        float pv = S.sigma * gs;
        if (eid >= 0) pv = c * dsel + pv;
        st_coherent64(&a.pbuf[((size_t)par * kXcds + x) * kH + h0 + ln], pack_f32(pv, epP));
      }
    }
    AIMA_TRACE(L, 8, 0);  // P published (wave 0)
    if (wave == 0) {
      // relay: rows 64j + lane of r_{L+1} = r_L + sum over XCDs of P
      // (each XCD's P rows are contiguous: stores from different XCDs never
      // share a cache line, which measured 15 % faster per token than
      // interleaving the 8 records of a row)
      const uint64_t* src = a.pbuf + (size_t)par * kXcds * kH + j * kRowsB + ln;
      uint64_t v[kXcds];
      uint32_t spins = 0;
      bool have = true;
      while (true) {
        poll8(src, kH * 8, v);
        bool ok = true;
#pragma unroll
        for (int q = 0; q < kXcds; ++q) ok = ok && (uint32_t)(v[q] >> 32) == epP;
        if (__all(ok)) break;
        if (++spins > kSpinLimit) {
          fail_timeout();
          have = false;
          break;
        }
      }
      AIMA_TRACE(L, 9, 0);  // P read
      // (as_f32 takes the word by value: __builtin_bit_cast applied directly
      // to an element of a vector value reads element 0 with this compiler)
      float f = 0.f;
#pragma unroll
      for (int q = 0; q < kXcds; ++q) f += as_f32((uint32_t)v[q]);
      const int h = j * kRowsB + ln;
      const uint16_t rh = (uint16_t)(S.rl[h >> 1] >> ((h & 1) * 16));
      const uint16_t o = f2h_rounded(h2f(rh) + f);
      if (!have) {
        // nothing is published after a timeout
      } else if (L + 1 < a.n_layers) {
        st_local32(&a.rx[((size_t)x * 2 + (par ^ 1)) * kH + h], pack_word(o, epP));
      } else if (x == 0) {
        a.out[h] = o;
      }
      AIMA_TRACE(L, 10, 0);  // r_{L+1} rows stored
    }
  }
  if (a.n_layers == 1 && b == 0 && wave == 0) {
    // one layer: block 0 exits only after every block published P
    const uint32_t epP = base + 1u;
    uint32_t spins = 0;
    for (int h = lane; h < kH; h += 64) {
      uint64_t v[kXcds];
      while (true) {
        poll8(a.pbuf + h, kH * 8, v);
        bool ok = true;
#pragma unroll
        for (int q = 0; q < kXcds; ++q) ok = ok && (uint32_t)(v[q] >> 32) == epP;
        if (ok || ++spins > kSpinLimit) break;
      }
    }
  }
  finish();
}

#ifdef AIMA_DECODE_TRACE
extern "C" int aima_debug_set_decode_trace(uint64_t* dev_buf) {
  return hip_check(hipMemcpyToSymbol(HIP_SYMBOL(g_trace), &dev_buf, sizeof(dev_buf)),
                   "set decode trace");
}
#endif

}  // namespace aima

// ---------------------------------------------------------------------------
// host: resident decode plan
// ---------------------------------------------------------------------------
using namespace aima;

struct aima_moe_decode_plan {
  int device = 0;
  bool ring = false;  // logits-fed 128-group runs take the weight-ring instance
  int n_layers = 0;
  int k = 0;
  int experts = 0;
  int group_log2 = 0;
  int blocks = 0;
  char* mem = nullptr;  // device allocation holding everything below
  PlanLayer* table = nullptr;
  uint32_t* rx = nullptr;
  uint64_t* actx = nullptr;
  uint64_t* pbuf = nullptr;
  uint32_t* route_ids = nullptr;
  uint64_t* route_w = nullptr;
  uint64_t* lgx = nullptr;
  uint32_t* counter = nullptr;
  uint32_t* err = nullptr;
  std::vector<PlanLayer> host;  // the uploaded table
  bool routers = false;         // router rows present in the table
};

namespace {

int persistent_shape_ok(const aima_moe_layer* layers, int n, int k, std::string* why) {
  if (n <= 0 || n > 79) { *why = "n_layers must be in [1, 79]"; return 0; }
  if (k <= 0 || k > kMaxK) { *why = "k must be in [1, 8]"; return 0; }
  for (int l = 0; l < n; ++l) {
    const aima_moe_layer& L = layers[l];
    if (L.hidden != kH || L.inter != kI || L.shared_inter != kI) {
      *why = "the persistent decode is specialized for hidden 2048, inter 512";
      return 0;
    }
    if (L.experts != layers[0].experts || L.group != layers[0].group) {
      *why = "all layers must share experts and group";
      return 0;
    }
    if (L.experts < k || L.experts > 1024) { *why = "experts must be in [k, 1024]"; return 0; }
    if (!(L.group == 32 || L.group == 64 || L.group == 128 || L.group == 256)) {
      *why = "group must be 32, 64, 128 or 256";
      return 0;
    }
    if (!L.gate_up.qweight || !L.gate_up.scale || !L.gate_up.zp || !L.down.qweight ||
        !L.down.scale || !L.down.zp || !L.shared_gate_up.qweight || !L.shared_gate_up.scale ||
        !L.shared_gate_up.zp || !L.shared_down.qweight || !L.shared_down.scale ||
        !L.shared_down.zp || !L.shared_gate_vec || !L.norm_weight) {
      *why = "null tensor pointer";
      return 0;
    }
    if (!split_tensors_ok(L)) {
      *why = "a split up tensor needs qweight, scale and zp";
      return 0;
    }
    if (!aligned(L.gate_up.qweight, 16) || !aligned(L.down.qweight, 16) ||
        !aligned(L.shared_gate_up.qweight, 16) || !aligned(L.shared_down.qweight, 16) ||
        !aligned(L.shared_gate_vec, 16) || !aligned(L.norm_weight, 16)) {
      *why = "qweight, shared_gate_vec and norm_weight must be 16-byte aligned";
      return 0;
    }
    // scales and zero points are read as 32-bit words
    const aima_u4_tensor* ts[] = {&L.gate_up, &L.down, &L.shared_gate_up, &L.shared_down,
                                  &L.up, &L.shared_up};
    for (const aima_u4_tensor* t : ts) {
      if (t->qweight && (!aligned(t->scale, 4) || !aligned(t->zp, 4))) {
        *why = "scale and zp pointers must be 4-byte aligned";
        return 0;
      }
    }
  }
  return 1;
}

// The kernel's table entry of one layer (shapes already validated).
PlanLayer plan_layer(const aima_moe_layer& L) {
  const int64_t G = L.hidden / L.group;  // groups per gate/up row
  const GateUpView r = routed_gate_up(L), s = shared_gate_up(L);
  PlanLayer p{};
  for (int h = 0; h < 2; ++h) {
    const int64_t r0 = r.row(0, h, 0), s0 = s.row(0, h, 0);
    (h ? p.gq1 : p.gq0) = r.q[h] + r0 * (L.hidden / 2);
    (h ? p.gs1 : p.gs0) = r.s[h] + r0 * G;
    (h ? p.gz1 : p.gz0) = r.z[h] + r0 * G / 2;
    (h ? p.sq1 : p.sq0) = s.q[h] + s0 * (L.hidden / 2);
    (h ? p.ss1 : p.ss0) = s.s[h] + s0 * G;
    (h ? p.sz1 : p.sz0) = s.z[h] + s0 * G / 2;
  }
  p.estride_q = (uint32_t)(r.expert_rows * (L.hidden / 2));
  p.estride_s = (uint32_t)(r.expert_rows * G * 2);
  p.estride_z = (uint32_t)(r.expert_rows * G / 2);
  p.dq = L.down.qweight;
  p.ds = L.down.scale;
  p.dz = L.down.zp;
  p.sdq = L.shared_down.qweight;
  p.sds = L.shared_down.scale;
  p.sdz = L.shared_down.zp;
  p.gate_vec = L.shared_gate_vec;
  p.norm = L.norm_weight;
  return p;
}

}  // namespace

extern "C" int aima_moe_decode_plan_create(const aima_moe_layer* layers, int32_t n_layers,
                                           int32_t k, aima_moe_decode_plan** plan) {
  AIMA_REQUIRE(layers && plan, "moe_decode_plan_create: null pointer");
  *plan = nullptr;
  std::string why;
  if (!persistent_shape_ok(layers, n_layers, k, &why)) {
    return fail(AIMA_E_UNSUPPORTED, "moe_decode_plan_create: " + why);
  }
  int dev = 0;
  AIMA_HIP(hipGetDevice(&dev));
  int cus = 0, coop = 0, per_cu = 0;
  AIMA_HIP(hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev));
  AIMA_HIP(hipDeviceGetAttribute(&coop, hipDeviceAttributeCooperativeLaunch, dev));
  per_cu = 1 << 30;
  for (const void* kern : {reinterpret_cast<const void*>(decode_persistent_kernel<false, false>),
                           reinterpret_cast<const void*>(decode_persistent_kernel<true, false>),
                           reinterpret_cast<const void*>(decode_persistent_kernel<false, true>),
                           reinterpret_cast<const void*>(decode_persistent_kernel<true, true>)}) {
    int n = 0;
    AIMA_HIP(hipOccupancyMaxActiveBlocksPerMultiprocessor(&n, kern, kThreads, 0));
    per_cu = std::min(per_cu, n);
  }
  {
    int n = 0;
    AIMA_HIP(hipOccupancyMaxActiveBlocksPerMultiprocessor(
        &n, reinterpret_cast<const void*>(decode_persistent_kernel<true, false, true>),
        kRingThreads, 0));
    per_cu = std::min(per_cu, n);
  }
  const int blocks = kBlocks;  // one block per CU: 8 XCDs x 32 CUs
  (void)coop;
  if (cus != kBlocks || per_cu < 1) {
    return fail(AIMA_E_UNSUPPORTED,
                "moe_decode_plan_create: the persistent decode needs a device of 256 CUs "
                "(8 XCDs x 32) that keeps one 512-thread block per CU resident");
  }
  size_t off = 0;
  auto take = [&](size_t bytes) {
    const size_t at = off;
    off += round_up(bytes, 256);
    return at;
  };
  const size_t o_err = take(kWsHeader);
  const size_t o_table = take(sizeof(PlanLayer) * n_layers);
  const size_t o_rx = take(sizeof(uint32_t) * kXcds * 2 * kH);
  const size_t o_act = take(sizeof(uint64_t) * kXcds * 2 * kActStride);
  const size_t o_p = take(sizeof(uint64_t) * 2 * kH * kXcds);
  const size_t o_rid = take(sizeof(uint32_t) * n_layers * k);
  const size_t o_rw = take(sizeof(uint64_t) * n_layers * k);
  const size_t o_lgx = take(sizeof(uint64_t) * kXcds * 2 * kRouterRows);
  const size_t o_ctr = take(256);
  // each layer's shared-expert down weights, slice-major: XCD x reads K
  // slice x (32 bytes) of every row, which the row-major tensor spreads
  // over a 128-byte line per row (4x the bytes through the L2)
  constexpr size_t kSliceBytes = (size_t)kH * (kI / 2);
  const size_t o_sdq = take(kSliceBytes * n_layers);
  aima_moe_decode_plan* p = new aima_moe_decode_plan();
  p->device = dev;
  // AIMA_DECODE_RING=0 keeps the register-prefetch instance (A/B runs)
  const char* ring_env = std::getenv("AIMA_DECODE_RING");
  p->ring = !(ring_env && ring_env[0] == '0');
  p->n_layers = n_layers;
  p->k = k;
  p->experts = layers[0].experts;
  p->group_log2 = group_log2_of(layers[0].group);
  p->blocks = blocks;
  hipError_t e = hipMalloc(&p->mem, off);
  if (e != hipSuccess) {
    delete p;
    return hip_check(e, "hipMalloc(decode plan)");
  }
  p->err = reinterpret_cast<uint32_t*>(p->mem + o_err);
  p->table = reinterpret_cast<PlanLayer*>(p->mem + o_table);
  p->rx = reinterpret_cast<uint32_t*>(p->mem + o_rx);
  p->actx = reinterpret_cast<uint64_t*>(p->mem + o_act);
  p->pbuf = reinterpret_cast<uint64_t*>(p->mem + o_p);
  p->route_ids = reinterpret_cast<uint32_t*>(p->mem + o_rid);
  p->route_w = reinterpret_cast<uint64_t*>(p->mem + o_rw);
  p->lgx = reinterpret_cast<uint64_t*>(p->mem + o_lgx);
  p->counter = reinterpret_cast<uint32_t*>(p->mem + o_ctr);
  e = hipMemset(p->mem, 0, off);
  if (e == hipSuccess) {
    p->host.resize(n_layers);
    for (int l = 0; l < n_layers && e == hipSuccess; ++l) {
      p->host[l] = plan_layer(layers[l]);
      char* dst = p->mem + o_sdq + kSliceBytes * l;
      for (int xs = 0; xs < kXcds && e == hipSuccess; ++xs) {
        e = hipMemcpy2D(dst + (size_t)xs * kH * 32, 32, layers[l].shared_down.qweight + xs * 32,
                        kI / 2, 32, kH, hipMemcpyDeviceToDevice);
      }
      p->host[l].sdq = reinterpret_cast<const uint8_t*>(dst);
    }
    if (e == hipSuccess) {
      e = hipMemcpy(p->table, p->host.data(), sizeof(PlanLayer) * n_layers,
                    hipMemcpyHostToDevice);
    }
  }
  if (e != hipSuccess) {
    (void)hipFree(p->mem);
    delete p;
    return hip_check(e, "decode plan upload");
  }
  *plan = p;
  return AIMA_OK;
}

namespace {

int plan_launch(aima_moe_decode_plan* plan, PersistArgs& a, bool routed, void* stream) {
  int dev = 0;
  AIMA_HIP(hipGetDevice(&dev));
  AIMA_REQUIRE(dev == plan->device, "moe_decode_plan_run: plan belongs to another device");
  a.layers = plan->table;
  a.n_layers = plan->n_layers;
  a.k = plan->k;
  a.experts = plan->experts;
  a.group_log2 = plan->group_log2;
  a.rx = plan->rx;
  a.actx = plan->actx;
  a.pbuf = plan->pbuf;
  a.route_ids = plan->route_ids;
  a.route_w = plan->route_w;
  a.lgx = plan->lgx;
  a.epoch_counter = plan->counter;
  a.err = plan->err;
  void* args[] = {&a};
  const bool g128 = plan->group_log2 == 7;
  const bool ring = !routed && g128 && plan->ring;
  const void* kern =
      ring ? reinterpret_cast<const void*>(decode_persistent_kernel<true, false, true>)
      : routed ? (g128 ? reinterpret_cast<const void*>(decode_persistent_kernel<true, true>)
                       : reinterpret_cast<const void*>(decode_persistent_kernel<false, true>))
               : (g128 ? reinterpret_cast<const void*>(decode_persistent_kernel<true, false>)
                       : reinterpret_cast<const void*>(decode_persistent_kernel<false, false>));
  // A regular launch: with one block per CU on 256 CUs every block becomes
  // resident (work of other streams only delays placement).  A cooperative
  // launch would guarantee it against concurrent persistent launches too,
  // but measured 18 us slower per launch (the gap between launches).
  AIMA_HIP(hipLaunchKernel(kern, dim3(plan->blocks), dim3(ring ? kRingThreads : kThreads), args,
                           0, (hipStream_t)stream));
  return AIMA_OK;
}

}  // namespace

extern "C" int aima_moe_decode_plan_run(aima_moe_decode_plan* plan, float eps,
                                        const uint16_t* residual_in,
                                        const float* router_logits, const int32_t* ids,
                                        const float* weights, float min_weight_sum,
                                        uint16_t* out, void* stream) {
  AIMA_REQUIRE(plan && residual_in && out, "moe_decode_plan_run: null pointer");
  AIMA_REQUIRE(router_logits || (ids && weights),
               "moe_decode_plan_run: need router logits or ids + weights");
  AIMA_REQUIRE(min_weight_sum > 0.f, "moe_decode_plan_run: minimum weight sum must be positive");
  AIMA_REQUIRE(aligned(residual_in, 16), "moe_decode_plan_run: residual_in must be 16-byte aligned");
  PersistArgs a{};
  a.logits = router_logits;
  a.ids_in = ids;
  a.w_in = weights;
  a.min_weight_sum = min_weight_sum;
  a.eps = eps;
  a.r0 = residual_in;
  a.out = out;
  return plan_launch(plan, a, false, stream);
}

extern "C" int aima_moe_decode_plan_set_routers(aima_moe_decode_plan* plan,
                                                const aima_u4_tensor* routers) {
  AIMA_REQUIRE(plan && routers, "moe_decode_plan_set_routers: null pointer");
  if (plan->experts > kRouterRows) {
    return fail(AIMA_E_UNSUPPORTED,
                "moe_decode_plan_set_routers: the routed plan takes at most 256 experts");
  }
  for (int l = 0; l < plan->n_layers; ++l) {
    const aima_u4_tensor& R = routers[l];
    AIMA_REQUIRE(R.qweight && R.scale && R.zp, "moe_decode_plan_set_routers: null router tensor");
    AIMA_REQUIRE(aligned(R.qweight, 16) && aligned(R.scale, 4) && aligned(R.zp, 4),
                 "moe_decode_plan_set_routers: router qweight must be 16-byte aligned, "
                 "scale and zp 4-byte aligned");
  }
  int dev = 0;
  AIMA_HIP(hipGetDevice(&dev));
  AIMA_REQUIRE(dev == plan->device, "moe_decode_plan_set_routers: plan belongs to another device");
  std::vector<PlanLayer> host = plan->host;
  for (int l = 0; l < plan->n_layers; ++l) {
    host[l].rq = routers[l].qweight;
    host[l].rs = routers[l].scale;
    host[l].rz = routers[l].zp;
  }
  // setup time: no run of this plan may be in flight while the table changes
  AIMA_HIP(hipDeviceSynchronize());
  AIMA_HIP(hipMemcpy(plan->table, host.data(), sizeof(PlanLayer) * plan->n_layers,
                     hipMemcpyHostToDevice));
  plan->host.swap(host);
  plan->routers = true;
  return AIMA_OK;
}

extern "C" int aima_moe_decode_plan_run_routed(aima_moe_decode_plan* plan, float eps,
                                               const uint16_t* residual_in, float min_weight_sum,
                                               int32_t* ids, float* weights, float* logits,
                                               uint16_t* out, void* stream) {
  AIMA_REQUIRE(plan && residual_in && out, "moe_decode_plan_run_routed: null pointer");
  if (!plan->routers) {
    return fail(AIMA_E_INVALID,
                "moe_decode_plan_run_routed: no routers (aima_moe_decode_plan_set_routers)");
  }
  AIMA_REQUIRE(min_weight_sum > 0.f,
               "moe_decode_plan_run_routed: minimum weight sum must be positive");
  AIMA_REQUIRE(aligned(residual_in, 16),
               "moe_decode_plan_run_routed: residual_in must be 16-byte aligned");
  PersistArgs a{};
  a.min_weight_sum = min_weight_sum;
  a.eps = eps;
  a.r0 = residual_in;
  a.out = out;
  a.logits_out = logits;
  a.ids_out = ids;
  a.w_out = weights;
  return plan_launch(plan, a, true, stream);
}

extern "C" int aima_moe_decode_plan_error(aima_moe_decode_plan* plan, uint32_t* error_bits,
                                          void* stream) {
  AIMA_REQUIRE(plan && error_bits, "moe_decode_plan_error: null pointer");
  return aima_workspace_error(plan->err, error_bits, stream);
}

extern "C" int aima_moe_decode_plan_destroy(aima_moe_decode_plan* plan) {
  if (!plan) return AIMA_OK;
  hipError_t e = hipFree(plan->mem);
  delete plan;
  return hip_check(e, "hipFree(decode plan)");
}
