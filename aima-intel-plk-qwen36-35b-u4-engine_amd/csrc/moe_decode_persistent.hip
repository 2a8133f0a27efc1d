// Persistent batch-1 decode of an MoE FFN stack (all layers in one launch).
//
// Launch: one 512-thread block per CU, cooperative (every block resident).
// Wave 0 of each block is the control wave; waves 1..7 compute.
//
// Per layer L the work is the same as the two-launch decode (moe_decode.hip):
//   A_L  rows of the k routed + shared gate/up matrices -> SwiGLU -> act_L
//   B_L  rows of the down matrices, weighted sum, residual -> r_{L+1}
// but no launch or grid barrier separates the phases.  Every value another
// block consumes is published as a self-validating word: {f16 value, u16
// epoch} for the residual, {3 x f16, u16 epoch} records (64-bit, written
// atomically) for the activations, {id, epoch} / {f32, epoch} for the routes.
// A consumer polls the words it needs with device-coherent loads until every
// epoch matches the one expected for this launch and phase, so the wait and
// the data transfer are one round trip.
// Ordering argument: a block can only publish act_{L+1} after seeing all of
// r_{L+1}, i.e. after every block finished B_L (and thus its reads of act_L),
// and likewise for r; with buffers alternating by layer parity a word can
// never be overwritten while a reader still expects it.  Epochs are unique
// per launch, so stale words left by an earlier launch never match: every
// block reads the launch counter when it starts and block 0 advances it when
// it exits, which cannot happen before every block has started (block 0's
// last phase consumes an output of every block).
//
// Everything a block needs that does not depend on other blocks' results of
// the current layer is fetched ahead: all routes once at the start, the next
// layer's norm weight and shared-expert gate vector into LDS during B_L, and
// each wave's weight rows for the next phase right after the previous one.
// So each phase boundary costs only the exchange itself.  The control wave
// turns r_L into the A-phase operands (RMSNorm, per-chunk pairs and sums, the
// shared-expert gate sigmoid, computed by every block for itself) and stages
// act_L; the compute waves build their own B-phase chunk operands.  Every
// poll has a spin limit: on expiry the block records AIMA_DEVERR_TIMEOUT and
// all its waves return, so no wave can wait forever.
#include "common.h"

#include <math.h>

#include <string>

namespace aima {

namespace {

constexpr int kThreads = 512;
constexpr int kComputeWaves = 7;
constexpr int kH = 2048;             // hidden (specialization)
constexpr int kI = 512;              // expert intermediate (specialization)
constexpr int kMaxRowsA = 6;         // gate/up rows per compute wave
constexpr int kMaxUnitsB = 3;        // (slot, 4-row pass) units per compute wave
constexpr int kMaxK = 8;
constexpr int kMaxSlots = kMaxK + 1;
constexpr int kRowsB = 8;            // output rows per block
constexpr uint32_t kSpinLimit = 1u << 22;
constexpr int kMaxLayers = 79;
constexpr int kChunksA = kH / 32;                   // A-phase operand chunks
constexpr int kChunksB = kMaxUnitsB * (kI / 32);    // B-phase chunks per wave
constexpr int kActRecords = kMaxSlots * kI / 3;     // act records per parity buffer
constexpr int kAuxCoherent = 16;                    // sc1: device-coherent load

struct PersistArgs {
  const aima_moe_layer* layers;   // device table [n_layers]
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
  uint32_t* r_buf;                // [2][H]            {f16, epoch}, chunk-interleaved
  uint64_t* act_buf;              // [2][kActRecords]  {3 x f16, epoch}
  uint32_t* route_ids;            // [L][k]            {id, epoch}
  uint64_t* route_w;              // [L][k]            {f32, epoch}
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

__device__ __forceinline__ uint32_t pack_word(uint16_t v, uint32_t epoch) {
  return (uint32_t)v | (epoch << 16);
}
__device__ __forceinline__ uint64_t pack_f32(float v, uint32_t epoch) {
  return (uint64_t)__builtin_bit_cast(uint32_t, v) | ((uint64_t)epoch << 32);
}

// Residual words are stored chunk-interleaved: value h = 32 c + 4 q + j sits
// at word 4 (64 q + c) + j, so the 16-byte load q of lane c returns values
// 4q..4q+3 of chunk c and the eight loads of a lane are coalesced across the
// wave.  Each word validates itself, so a wide load needs no atomicity
// beyond the 32-bit word.
__device__ __forceinline__ int r_pos(int h) {
  return ((((h & 31) >> 2) * 64 + (h >> 5)) << 2) + (h & 3);
}

struct SharedState {
  u32x4 xa_p[4][kChunksA];             // A operands: chunk pairs, word-group major
  float xa_bias[kChunksA];
  float xa_xsum[kChunksA];
  uint32_t xb[kMaxSlots * kI / 2];     // act_L, f16 pairs (slot-major)
  u32x4 xb_p[kComputeWaves][4][kChunksB];  // per compute wave B operands
  float xb_bias[kComputeWaves][kChunksB];
  float xb_xsum[kComputeWaves][kChunksB];
  // RMSNorm weight (f32) and shared gate vector (f16) of the current layer,
  // and the normalized activation x (f16), each stored so that lane c's
  // 16-byte read q returns part q of chunk c (conflict-free LDS reads)
  u32x4 nw_p[8][kChunksA];
  u32x4 gv_p[4][kChunksA];
  u32x4 xw_p[4][kChunksA];
  float rowsum[kComputeWaves * kMaxRowsA];
  float part[kMaxSlots][kRowsB];
  float rown[kRowsB];                  // this block's residual rows (f32 of f16)
  aima_moe_layer table[kMaxLayers];    // the layer table, copied once
  int32_t route_id[kMaxLayers][kMaxK];
  float route_w[kMaxLayers][kMaxK];
  float sigma;
  int abort;
};

// Router top-k for one layer (one wave): f64 softmax over the logits,
// (probability desc, id asc) selection, renormalization by max(sum, min).
// Lane `r` < k returns the rank-r id and weight.  Reductions use DPP inside
// 16-lane rows and readlane across rows (no LDS round trips).
template <int CTRL>
__device__ __forceinline__ int dpp_int(int v) {
  return __builtin_amdgcn_update_dpp(0, v, CTRL, 0xF, 0xF, false);
}
__device__ __forceinline__ bool route_better(float p, int i, float bp, int bi) {
  return p > bp || (p == bp && i < bi);
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

// Orders one wave's LDS writes before its following LDS reads by other lanes
// of the same wave (a wave executes its LDS operations in order; the fences
// keep the compiler from moving the accesses across).
__device__ __forceinline__ void wave_lds_sync() {
  __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
  __builtin_amdgcn_wave_barrier();
  __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
}

#ifdef AIMA_DECODE_TRACE
// Diagnostics build only (never in the product library): phase timestamps of
// every block, 100 MHz real-time clock, g_trace[(L * 256 + block) * 16 + slot].
__device__ uint64_t* g_trace = nullptr;
#define AIMA_TRACE(L, slot, T)                                              \
  do {                                                                      \
    if (trace && threadIdx.x == (T) && b < 256)                             \
      trace[((L) * 256 + b) * 16 + (slot)] = __builtin_amdgcn_s_memrealtime(); \
  } while (0)
#else
#define AIMA_TRACE(L, slot, T) \
  do {                         \
  } while (0)
#endif

}  // namespace

__global__ __launch_bounds__(kThreads, 1) void decode_persistent_kernel(PersistArgs a) {
  __shared__ SharedState S;
  const int lane = threadIdx.x & 63;
  // wave-uniform values in scalar registers, so per-row branches and buffer
  // offsets below are scalar and never merge divergent loads
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int cw = wave - 1;  // compute wave index (valid for wave >= 1)
  const int ct = threadIdx.x - 64;  // compute thread index (valid for wave >= 1)
  const int nb = gridDim.x;
  const int b = blockIdx.x;
  const int k = a.k;
  const int slots = k + 1;
  const int pairs = slots * kI;
  // pairs per block, a multiple of 3 so each block owns whole act records
  const int ppb = ((pairs + nb - 1) / nb + 2) / 3 * 3;
  const int pair0 = b * ppb;
  const int npairs = max(0, min(ppb, pairs - pair0));
  const int h0 = b * kRowsB;
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

  if (threadIdx.x == 0) S.abort = 0;
  {
    const uint32_t* src = reinterpret_cast<const uint32_t*>(a.layers);
    uint32_t* dst = reinterpret_cast<uint32_t*>(S.table);
    const int words = a.n_layers * (int)(sizeof(aima_moe_layer) / 4);
    for (int i = threadIdx.x; i < words; i += kThreads) dst[i] = src[i];
  }
  if (threadIdx.x < kRowsB) S.rown[threadIdx.x] = h2f(a.r0[h0 + threadIdx.x]);
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
  __syncthreads();

  // norm weight (f32) and shared gate vector (f16) of a layer: 768 16-byte
  // pieces, two per compute thread at most, staged through registers
  auto load_vec = [&](int L, u32x4* v) {
    const aima_moe_layer& Ly = S.table[L];
#pragma unroll
    for (int j = 0; j < 2; ++j) {
      const int c = ct + j * (kThreads - 64);
      if (c < kH / 4) {
        v[j] = gload16(Ly.norm_weight + 4 * c);
      } else if (c < kH / 4 + kH / 8) {
        v[j] = gload16(Ly.shared_gate_vec + 8 * (c - kH / 4));
      }
    }
  };
  auto store_vec = [&](const u32x4* v) {
#pragma unroll
    for (int j = 0; j < 2; ++j) {
      const int c = ct + j * (kThreads - 64);
      if (c < kH / 4) {
        S.nw_p[c & 7][c >> 3] = v[j];            // floats 4c.. = chunk c/8, part c%8
      } else if (c < kH / 4 + kH / 8) {
        const int g = c - kH / 4;                // halves 8g.. = chunk g/4, part g%4
        S.gv_p[g & 3][g >> 2] = v[j];
      }
    }
  };
  // route of layer L into LDS (ids range-checked); one wave, lanes < k
  auto put_route = [&](int L, int id, float w) {
    if (lane < k) {
      if (id < 0 || id >= a.experts) {
        atomicOr(a.err, AIMA_DEVERR_EXPERT_RANGE);
        id = -1;
      }
      S.route_id[L][lane] = id;
      S.route_w[L][lane] = w;
    }
  };
  auto local_route = [&](int L, int32_t* id, float* w) {
    if (a.logits) {
      route_layer(a.logits + (int64_t)L * a.experts, a.experts, k, a.min_weight_sum, id, w);
    } else if (lane < k) {
      *id = a.ids_in[L * k + lane];
      *w = a.w_in[L * k + lane];
    }
  };
  // poll the route block L published (returns false on timeout)
  auto poll_route = [&](int L) -> bool {
    uint32_t spins = 0;
    while (true) {
      bool ok = true;
      uint32_t idw = 0;
      uint64_t ww = 0;
      if (lane < k) {
        idw = ld_coherent32(&a.route_ids[L * k + lane]);
        ww = ld_coherent64(&a.route_w[L * k + lane]);
        ok = (idw >> 16) == route_epoch && (uint32_t)(ww >> 32) == route_epoch;
      }
      if (__all(ok)) {
        put_route(L, (int)(idw & 0xffffu), __builtin_bit_cast(float, (uint32_t)ww));
        return true;
      }
      if (++spins > kSpinLimit) return false;
      __builtin_amdgcn_s_sleep(2);
    }
  };

  // ---- prologue --------------------------------------------------------------
  // Every block computes layer 0's route itself (wave 0); block L >= 1
  // publishes layer L's route (wave 2), which is polled one layer ahead.
  if (wave == 0) {
    int32_t id = 0;
    float w = 0.f;
    local_route(0, &id, &w);
    put_route(0, id, w);
  } else {
    u32x4 v[2];
    load_vec(0, v);
    store_vec(v);
    if (wave == 2) {
      for (int L = (b == 0 ? nb : b); L < a.n_layers; L += nb) {
        int32_t id = 0;
        float w = 0.f;
        local_route(L, &id, &w);
        if (lane < k) {
          st_coherent32(&a.route_ids[L * k + lane], pack_word((uint16_t)id, route_epoch));
          st_coherent64(&a.route_w[L * k + lane], pack_f32(w, route_epoch));
        }
      }
    }
  }
  __syncthreads();

  // ---- per-wave prefetch state ----------------------------------------------
  // raw prefetched words: weights, f16 scale bits, zero-point byte + nibble
  // shift; converted only when used so no wait sits between the loads
  u32x4 wa[kMaxRowsA];
  uint32_t sa[kMaxRowsA];
  uint32_t za[kMaxRowsA];
  u32x4 wb[kMaxUnitsB];
  uint32_t sb[kMaxUnitsB];
  uint32_t zb[kMaxUnitsB];
  // The prefetch keeps the aligned 32-bit words holding a lane's f16 scale
  // (index gi) and u4 zero point (nibble gi); select them here.
  auto nib = [](uint32_t word, int gi) { return (word >> ((gi & 7) * 4)) & 0xfu; };
  auto scl = [](uint32_t word, int gi) { return h2f((uint16_t)(word >> ((gi & 1) * 16))); };

  // Weight loads: scalar base (readfirstlane of the table pointer, so it is
  // provably wave-uniform) plus a 32-bit per-lane offset.  Each prefetch is
  // straight-line code: a wave's surplus row slots are clamped onto a row the
  // block loads anyway (a cache hit) and an out-of-range expert id onto
  // expert 0 (its slot is weighted 0 and the error bit is set), so every
  // load is in bounds and issued back to back.
  auto uptr = [](const void* p) {
    const uint64_t v = reinterpret_cast<uint64_t>(p);
    const uint32_t lo = __builtin_amdgcn_readfirstlane((uint32_t)v);
    const uint32_t hi = __builtin_amdgcn_readfirstlane((uint32_t)(v >> 32));
    return reinterpret_cast<const AIMA_GLOBAL uint8_t*>(((uint64_t)hi << 32) | lo);
  };
  auto ld_w = [](const AIMA_GLOBAL uint8_t* base_ptr, uint32_t off) {
    return __builtin_nontemporal_load(
        reinterpret_cast<const AIMA_GLOBAL u32x4*>(base_ptr + off));
  };
  auto ld_u32 = [](const AIMA_GLOBAL uint8_t* base_ptr, uint32_t off) {
    return *reinterpret_cast<const AIMA_GLOBAL uint32_t*>(base_ptr + off);
  };
  // Per-lane offsets are recomputed at each prefetch from opaque copies of
  // the lane and wave index: hoisting them out of the layer loop would keep
  // ~30 more registers live across every phase.
  auto opaque_v = [](int v) {
    asm volatile("" : "+v"(v));
    return v;
  };
  auto opaque_s = [](int v) {
    asm volatile("" : "+s"(v));
    return v;
  };
  const int rowsA = 2 * npairs;  // gate/up rows of this block
  auto prefetch_a = [&](int L) {
    if (rowsA == 0) return;
    const int lane = opaque_v(threadIdx.x & 63);
    const int cw = opaque_s(wave - 1);
    const aima_moe_layer& Ly = S.table[L];
    const uint32_t wbytes = (uint32_t)(2 * kI) * (kH / 2);      // per expert
    const uint32_t sbytes = (uint32_t)(2 * kI) * gA * 2;
    const uint32_t zbytes = (uint32_t)(2 * kI) * gA / 2;
#pragma unroll
    for (int i = 0; i < kMaxRowsA; ++i) {
      const int ri = min(cw + kComputeWaves * i, rowsA - 1);  // row index within the block
      const int pair = pair0 + (ri >> 1);
      const int slot = pair / kI;
      const int j = pair - slot * kI;
      const int row = (ri & 1) ? kI + j : j;
      const int gi = row * gA + ((lane * 32) >> glog2);
      const bool routed = slot < k;
      const uint32_t e =
          (uint32_t)max(0, __builtin_amdgcn_readfirstlane(S.route_id[L][min(slot, k - 1)]));
      const AIMA_GLOBAL uint8_t* w = routed ? uptr(Ly.gate_up.qweight) + (size_t)e * wbytes
                                            : uptr(Ly.shared_gate_up.qweight);
      const AIMA_GLOBAL uint8_t* sp = routed ? uptr(Ly.gate_up.scale) + (size_t)e * sbytes
                                             : uptr(Ly.shared_gate_up.scale);
      const AIMA_GLOBAL uint8_t* zp = routed ? uptr(Ly.gate_up.zp) + (size_t)e * zbytes
                                             : uptr(Ly.shared_gate_up.zp);
      wa[i] = ld_w(w, (uint32_t)row * (kH / 2) + lane * 16);
      sa[i] = ld_u32(sp, (gi * 2) & ~3);
      za[i] = ld_u32(zp, (gi >> 1) & ~3);
    }
  };
  // B units: u = cw + 7 i -> slot = u / 2, pass = u % 2 (4 rows per pass)
  auto prefetch_b = [&](int L) {
    const int lane = opaque_v(threadIdx.x & 63);
    const int cw = opaque_s(wave - 1);
    const aima_moe_layer& Ly = S.table[L];
    const int seg = lane >> 4, cl = lane & 15;
    const uint32_t wbytes = (uint32_t)kH * (kI / 2);
    const uint32_t sbytes = (uint32_t)kH * gB * 2;
    const uint32_t zbytes = (uint32_t)kH * gB / 2;
#pragma unroll
    for (int i = 0; i < kMaxUnitsB; ++i) {
      const int u = cw + kComputeWaves * i;
      const int slot = min(u >> 1, slots - 1);
      const int row = h0 + (u & 1) * 4 + seg;
      const int gi = row * gB + ((cl * 32) >> glog2);
      const bool routed = slot < k;
      const uint32_t e =
          (uint32_t)max(0, __builtin_amdgcn_readfirstlane(S.route_id[L][min(slot, k - 1)]));
      const AIMA_GLOBAL uint8_t* w = routed ? uptr(Ly.down.qweight) + (size_t)e * wbytes
                                            : uptr(Ly.shared_down.qweight);
      const AIMA_GLOBAL uint8_t* sp = routed ? uptr(Ly.down.scale) + (size_t)e * sbytes
                                             : uptr(Ly.shared_down.scale);
      const AIMA_GLOBAL uint8_t* zp = routed ? uptr(Ly.down.zp) + (size_t)e * zbytes
                                             : uptr(Ly.shared_down.zp);
      wb[i] = ld_w(w, (uint32_t)row * (kI / 2) + cl * 16);
      sb[i] = ld_u32(sp, (gi * 2) & ~3);
      zb[i] = ld_u32(zp, (gi >> 1) & ~3);
    }
  };

  if (wave > 0) prefetch_a(0);
  AIMA_TRACE(40, 1, 0);  // prologue done

  // r_{L} polling: eight coalesced 16-byte device-coherent loads per lane
  // (the volatile bit keeps the compiler from merging repeated polls), one
  // batch at a time without pause: measured faster than keeping two batches
  // in flight or sleeping between polls, which add fabric traffic or delay.
  constexpr int kAuxPoll = kAuxCoherent | (int)(1u << 31);
  auto issue_r = [&](const AIMA_GLOBAL uint8_t* src, uint32_t (&rv)[32]) {
    const int lane = opaque_v(threadIdx.x & 63);
    const auto rr = __builtin_amdgcn_make_buffer_rsrc((void*)(uintptr_t)src, 0, kH * 4, 0x00020000);
#pragma unroll
    for (int q = 0; q < 8; ++q) {
      const u32x4 v = __builtin_amdgcn_raw_buffer_load_b128(rr, (q * 64 + lane) * 16, 0, kAuxPoll);
#pragma unroll
      for (int t = 0; t < 4; ++t) rv[4 * q + t] = v[t];
    }
  };
  auto r_ready = [&](const uint32_t (&rv)[32], uint32_t ep) {
    bool ok = true;
#pragma unroll
    for (int q = 0; q < 32; ++q) ok = ok && (rv[q] >> 16) == ep;
    return __all(ok) != 0;
  };
  // act_L polling: 24 records per lane; each batch is staged into LDS as it
  // is checked (a later complete batch overwrites it)
  constexpr int kQ = kActRecords / 64;
  const int nrec = (pairs + 2) / 3;  // valid records
  auto issue_act = [&](const uint64_t* src, uint64_t (&v)[kQ]) {
    const int lane = opaque_v(threadIdx.x & 63);
#pragma unroll
    for (int q = 0; q < kQ; ++q) v[q] = ld_coherent64(src + lane + 64 * q);
  };
  auto stage_act = [&](const uint64_t (&v)[kQ], uint32_t ep) {
    const int lane = opaque_v(threadIdx.x & 63);
    bool ok = true;
    uint8_t* d = reinterpret_cast<uint8_t*>(S.xb);
#pragma unroll
    for (int q = 0; q < kQ; ++q) {
      const int r = lane + 64 * q;
      ok = ok && (r >= nrec || (uint32_t)(v[q] >> 48) == ep);
      // record r = halves 3r..3r+2: an even r starts 4-byte aligned (word +
      // half), an odd r ends 4-byte aligned (half + word)
      const uint32_t lo = (uint32_t)v[q], hi = (uint32_t)(v[q] >> 32);
      const bool even = (r & 1) == 0;
      const uint32_t word = even ? lo : ((lo >> 16) | (hi << 16));
      const uint16_t half = even ? (uint16_t)hi : (uint16_t)lo;
      *reinterpret_cast<uint32_t*>(d + 6 * r + (even ? 0 : 2)) = word;
      *reinterpret_cast<uint16_t*>(d + 6 * r + (even ? 4 : 0)) = half;
    }
    return __all(ok) != 0;
  };

  for (int L = 0; L < a.n_layers; ++L) {
    // an opaque lane index per layer keeps lane-derived addresses from being
    // hoisted out of the loop (they would stay live in registers throughout)
    const int lane = opaque_v(threadIdx.x & 63);
    const uint32_t epA = base + 2u * (uint32_t)L;        // act_L
    const uint32_t epB = base + 2u * (uint32_t)L + 1u;   // r_{L+1}
    const uint32_t epR = base + 2u * (uint32_t)L - 1u;   // r_L (L > 0)

    // ================= phase A_L =================
    if (wave == 0) {
      // r_L chunk `lane` as {f16, epoch} words
      uint32_t rv[32];
      if (L == 0) {
        const AIMA_GLOBAL u32x4* p = (const AIMA_GLOBAL u32x4*)(a.r0 + lane * 32);
#pragma unroll
        for (int q = 0; q < 4; ++q) {
          const u32x4 v = p[q];
#pragma unroll
          for (int t = 0; t < 4; ++t) {
            rv[8 * q + 2 * t] = v[t] & 0xffffu;
            rv[8 * q + 2 * t + 1] = v[t] >> 16;
          }
        }
      } else {
        const AIMA_GLOBAL uint8_t* src = uptr(a.r_buf + ((L - 1) & 1) * kH);
        uint32_t spins = 0;
        while (true) {
          issue_r(src, rv);
          if (r_ready(rv, epR)) break;
          if (++spins > kSpinLimit) {
            fail_timeout();
            break;
          }
        }
      }
      AIMA_TRACE(L, 0, 0);  // r_L polled
      // RMSNorm: x = f16(r * rsqrt(mean(r^2) + eps) * w)
      float ss = 0.f;
#pragma unroll
      for (int q = 0; q < 32; ++q) {
        const float v = h2f((uint16_t)rv[q]);
        ss += v * v;
      }
      ss = segment_sum<64>(ss);
      const float scale = 1.0f / sqrtf(ss / (float)kH + a.eps);
      uint32_t xw[16];
#pragma unroll
      for (int q = 0; q < 8; ++q) {
        const u32x4 nv = S.nw_p[q][lane];
#pragma unroll
        for (int t = 0; t < 4; t += 2) {
          const float n0 = as_f32(nv[t]);
          const float n1 = as_f32(nv[t + 1]);
          const uint16_t x0 = f2h(h2f((uint16_t)rv[4 * q + t]) * scale * n0);
          const uint16_t x1 = f2h(h2f((uint16_t)rv[4 * q + t + 1]) * scale * n1);
          xw[2 * q + t / 2] = (uint32_t)x0 | ((uint32_t)x1 << 16);
        }
      }
#pragma unroll
      for (int q = 0; q < 4; ++q) {
        S.xw_p[q][lane] = u32x4{xw[4 * q], xw[4 * q + 1], xw[4 * q + 2], xw[4 * q + 3]};
      }
      XChunk c;
      make_xchunk(xw, c);
      put_chunk(S.xa_p, S.xa_bias, S.xa_xsum, lane, c);
    }
    __syncthreads();  // #1: A operands ready
    AIMA_TRACE(L, 6, 64);
    if (S.abort) {
      finish();
      return;
    }
    if (wave > 0) {
      XChunk xc;
      get_chunk(S.xa_p, S.xa_bias, S.xa_xsum, lane, xc);
#pragma unroll
      for (int i = 0; i < kMaxRowsA; ++i) {
        const int ri = cw + kComputeWaves * i;
        if ((ri >> 1) < npairs) {
          const int pair = pair0 + (ri >> 1);
          const int row = (ri & 1) ? kI + (pair % kI) : (pair % kI);
          const int gi = row * gA + ((lane * 32) >> glog2);
          const float d =
              segment_sum<64>(u4_chunk_dot(wa[i], xc, nib(za[i], gi), scl(sa[i], gi), magic));
          if (lane == 0) S.rowsum[ri] = d;
        }
      }
      AIMA_TRACE(L, 7, 64);
    } else {
      // shared-expert gate sigma = sigmoid(gate_vec . x), every block for
      // itself, while the compute waves run their dot products
      float g = 0.f;
#pragma unroll
      for (int q = 0; q < 4; ++q) {
        const u32x4 gg = S.gv_p[q][lane];
        const u32x4 xx = S.xw_p[q][lane];
#pragma unroll
        for (int t = 0; t < 4; ++t) {
          const f16x2 gh = as_h2(gg[t]);
          const f16x2 xh = as_h2(xx[t]);
          g += (float)gh.x * (float)xh.x;
          g += (float)gh.y * (float)xh.y;
        }
      }
      g = segment_sum<64>(g);
      if (lane == 0) {
        const double t = g;
        S.sigma = (float)(t >= 0.0 ? 1.0 / (1.0 + exp(-t)) : exp(t) / (1.0 + exp(t)));
      }
    }
    __syncthreads();  // #2: row sums ready
    AIMA_TRACE(L, 1, 64);
    u32x4 vec[2];
    if (wave > 0) {
      // SwiGLU for the block's pairs, published three per {3 x f16, epoch}
      if (3 * ct < npairs) {
        const int p0 = 3 * ct;
        float rs[6];
#pragma unroll
        for (int j = 0; j < 6; ++j) rs[j] = S.rowsum[min(2 * p0 + j, kComputeWaves * kMaxRowsA - 1)];
        uint64_t rec = (uint64_t)epA << 48;
#pragma unroll
        for (int j = 0; j < 3; ++j) {
          const uint16_t h = p0 + j < npairs ? f2h(silu_mul(rs[2 * j], rs[2 * j + 1])) : (uint16_t)0;
          rec |= (uint64_t)h << (16 * j);
        }
        st_coherent64(&a.act_buf[(L & 1) * kActRecords + pair0 / 3 + ct], rec);
      }
      AIMA_TRACE(L, 2, 64);
      // Weight prefetches are issued where the compute waves would otherwise
      // wait: a wave stalls at issue until the memory pipeline accepts its
      // loads, which at the chip's streaming rate takes about a microsecond.
      prefetch_b(L);
      AIMA_TRACE(L, 8, 64);
      if (L + 1 < a.n_layers) {
        load_vec(L + 1, vec);
        // the last compute wave fetches the next layer's route meanwhile
        if (cw == kComputeWaves - 1 && !poll_route(L + 1)) fail_timeout();
      }
    } else {
      const uint64_t* src = a.act_buf + (L & 1) * kActRecords;
      uint64_t va[kQ];
      uint32_t spins = 0;
      while (true) {
        issue_act(src, va);
        if (stage_act(va, epA)) break;
        if (++spins > kSpinLimit) {
          fail_timeout();
          break;
        }
      }
      AIMA_TRACE(L, 3, 0);
    }
    __syncthreads();  // #3: act_L staged
    AIMA_TRACE(L, 12, 64);
    if (S.abort) {
      finish();
      return;
    }
    if (wave > 0) {
      // this wave's B operand chunks: lane t < 48 builds chunk (unit t/16, t%16)
      if (lane < kChunksB) {
        const int u = cw + kComputeWaves * (lane >> 4);
        const int slot = u >> 1;
        if (slot < slots) {
          XChunk c;
          lds_xchunk(S.xb, slot * (kI / 2) + (lane & 15) * 16, c);
          put_chunk(S.xb_p[cw], S.xb_bias[cw], S.xb_xsum[cw], lane, c);
        }
      }
      wave_lds_sync();
      AIMA_TRACE(L, 10, 64);
      const int seg = lane >> 4, cl = lane & 15;
#pragma unroll
      for (int i = 0; i < kMaxUnitsB; ++i) {
        const int u = cw + kComputeWaves * i;
        const int slot = u >> 1;
        if (slot < slots) {
          XChunk xc;
          get_chunk(S.xb_p[cw], S.xb_bias[cw], S.xb_xsum[cw], i * 16 + cl, xc);
          const int row = h0 + (u & 1) * 4 + seg;
          const int gi = row * gB + ((cl * 32) >> glog2);
          const float d =
              segment_sum<16>(u4_chunk_dot(wb[i], xc, nib(zb[i], gi), scl(sb[i], gi), magic));
          if (cl == 0) S.part[slot][(u & 1) * 4 + seg] = d;
        }
      }
      AIMA_TRACE(L, 11, 64);
      if (L + 1 < a.n_layers) store_vec(vec);
    }
    __syncthreads();  // #4: partial sums ready, next layer's vectors staged
    AIMA_TRACE(L, 4, 0);
    if (wave > 0) {
      if (L + 1 < a.n_layers) prefetch_a(L + 1);
      AIMA_TRACE(L, 9, 64);
    } else if (lane < kRowsB) {
      // weighted sum in rank order, then the gated shared expert
      float c[kMaxK], pv[kMaxSlots];
#pragma unroll
      for (int s = 0; s < kMaxK; ++s) {
        c[s] = S.route_id[L][s] < 0 ? 0.f : S.route_w[L][s];
        pv[s] = S.part[s][lane];
      }
      pv[kMaxK] = S.part[kMaxK][lane];
      float f = 0.f;
#pragma unroll
      for (int s = 0; s < kMaxK; ++s) {
        if (s < k) f += c[s] * pv[s];
      }
      float sh = pv[0];
#pragma unroll
      for (int s = 1; s < kMaxSlots; ++s) sh = s == k ? pv[s] : sh;
      f += S.sigma * sh;
      const uint16_t o = f2h(S.rown[lane] + f);
      S.rown[lane] = h2f(o);
      if (L + 1 < a.n_layers) {
        st_coherent32(&a.r_buf[(L & 1) * kH + r_pos(h0 + lane)], pack_word(o, epB));
      } else {
        a.out[h0 + lane] = o;
      }
      AIMA_TRACE(L, 5, 0);  // r_{L+1} rows stored
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
  int n_layers = 0;
  int k = 0;
  int experts = 0;
  int group_log2 = 0;
  int blocks = 0;
  char* mem = nullptr;  // device allocation holding everything below
  aima_moe_layer* table = nullptr;
  uint32_t* r_buf = nullptr;
  uint64_t* act_buf = nullptr;
  uint32_t* route_ids = nullptr;
  uint64_t* route_w = nullptr;
  uint32_t* counter = nullptr;
  uint32_t* err = nullptr;
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
    if (!aligned(L.gate_up.qweight, 16) || !aligned(L.down.qweight, 16) ||
        !aligned(L.shared_gate_up.qweight, 16) || !aligned(L.shared_down.qweight, 16) ||
        !aligned(L.shared_gate_vec, 16) || !aligned(L.norm_weight, 16)) {
      *why = "qweight, shared_gate_vec and norm_weight must be 16-byte aligned";
      return 0;
    }
  }
  return 1;
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
  AIMA_HIP(hipOccupancyMaxActiveBlocksPerMultiprocessor(&per_cu, decode_persistent_kernel,
                                                        kThreads, 0));
  const int blocks = kH / kRowsB;  // 256: one block owns 8 output rows
  if (!coop || (int64_t)cus * per_cu < blocks) {
    return fail(AIMA_E_UNSUPPORTED,
                "moe_decode_plan_create: the device cannot keep 256 blocks of 512 threads "
                "resident for a cooperative launch");
  }
  size_t off = 0;
  auto take = [&](size_t bytes) {
    const size_t at = off;
    off += round_up(bytes, 256);
    return at;
  };
  const size_t o_err = take(kWsHeader);
  const size_t o_table = take(sizeof(aima_moe_layer) * n_layers);
  const size_t o_r = take(sizeof(uint32_t) * 2 * kH);
  const size_t o_act = take(sizeof(uint64_t) * 2 * kMaxSlots * kI / 3);
  const size_t o_rid = take(sizeof(uint32_t) * n_layers * k);
  const size_t o_rw = take(sizeof(uint64_t) * n_layers * k);
  const size_t o_ctr = take(256);
  aima_moe_decode_plan* p = new aima_moe_decode_plan();
  p->device = dev;
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
  p->table = reinterpret_cast<aima_moe_layer*>(p->mem + o_table);
  p->r_buf = reinterpret_cast<uint32_t*>(p->mem + o_r);
  p->act_buf = reinterpret_cast<uint64_t*>(p->mem + o_act);
  p->route_ids = reinterpret_cast<uint32_t*>(p->mem + o_rid);
  p->route_w = reinterpret_cast<uint64_t*>(p->mem + o_rw);
  p->counter = reinterpret_cast<uint32_t*>(p->mem + o_ctr);
  e = hipMemset(p->mem, 0, off);
  if (e == hipSuccess) {
    e = hipMemcpy(p->table, layers, sizeof(aima_moe_layer) * n_layers, hipMemcpyHostToDevice);
  }
  if (e != hipSuccess) {
    (void)hipFree(p->mem);
    delete p;
    return hip_check(e, "decode plan upload");
  }
  *plan = p;
  return AIMA_OK;
}

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
  int dev = 0;
  AIMA_HIP(hipGetDevice(&dev));
  AIMA_REQUIRE(dev == plan->device, "moe_decode_plan_run: plan belongs to another device");
  hipStream_t st = (hipStream_t)stream;
  PersistArgs a{};
  a.layers = plan->table;
  a.n_layers = plan->n_layers;
  a.k = plan->k;
  a.experts = plan->experts;
  a.group_log2 = plan->group_log2;
  a.logits = router_logits;
  a.ids_in = ids;
  a.w_in = weights;
  a.min_weight_sum = min_weight_sum;
  a.eps = eps;
  a.r0 = residual_in;
  a.out = out;
  a.r_buf = plan->r_buf;
  a.act_buf = plan->act_buf;
  a.route_ids = plan->route_ids;
  a.route_w = plan->route_w;
  a.epoch_counter = plan->counter;
  a.err = plan->err;
  void* args[] = {&a};
  AIMA_HIP(hipLaunchCooperativeKernel(reinterpret_cast<const void*>(decode_persistent_kernel),
                                      dim3(plan->blocks), dim3(kThreads), args, 0, st));
  return AIMA_OK;
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
