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
// epoch} for the activations and the residual, {f32, u32 epoch} for router
// weights and the shared gate.  A consumer polls the words it needs with
// device-coherent loads until every epoch matches the one expected for this
// launch and phase, so the wait and the data transfer are one round trip.
// Ordering argument: a block can only publish act_{L+1} after seeing all of
// r_{L+1}, i.e. after every block finished B_L (and thus its reads of act_L),
// and likewise for r; with buffers alternating by layer parity a word can
// never be overwritten while a reader still expects it.  Epochs are unique
// per launch, so stale words left by an earlier launch never match: every
// block reads the launch counter when it starts and block 0 advances it when
// it exits, which cannot happen before every block has started (block 0's
// last phase consumes an output of every block).
//
// The control wave polls and converts the phase inputs into per-chunk dot
// product operands (XChunk, common.h) in LDS; meanwhile the compute waves
// have already issued the loads of their weight rows for that phase, so the
// HBM stream overlaps the cross-CU wait.  Every poll has a spin limit: on
// expiry the block records AIMA_DEVERR_TIMEOUT and all its waves return, so
// no wave can wait forever.
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
  uint32_t* r_buf;                // [2][H]            {f16, epoch}
  uint64_t* act_buf;              // [2][kMaxSlots*I/3] {3 x f16, epoch}
  uint64_t* sigma_buf;            // [2]               {f32, epoch}
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

struct SharedState {
  uint32_t xa[kH / 2];                 // A-phase input x, f16 pairs
  uint32_t xb[kMaxSlots * kI / 2];     // B-phase inputs act_L, f16 pairs (slot-major)
  __device__ uint16_t* xb16() { return reinterpret_cast<uint16_t*>(xb); }
  float rowsum[kComputeWaves * kMaxRowsA];
  float part[kMaxSlots][kRowsB];
  float rown[kRowsB];                  // this block's residual rows (f32 of f16)
  aima_moe_layer table[kMaxLayers];    // the layer table, copied once
  int32_t route_id[2][kMaxK];
  float route_w[2][kMaxK];
  float sigma;
  int abort;
};

// Router top-k for one layer (one wave): f64 softmax over the logits,
// (probability desc, id asc) selection, renormalization by max(sum, min).
__device__ void route_layer(const float* __restrict__ l, int E, int k, float min_sum,
                            int32_t* ids, float* w) {
  const int lane = threadIdx.x & 63;
  float mx = -INFINITY;
  for (int i = lane; i < E; i += 64) mx = fmaxf(mx, l[i]);
#pragma unroll
  for (int off = 32; off > 0; off >>= 1) mx = fmaxf(mx, __shfl_xor(mx, off, 64));
  double sum = 0.0;
  for (int i = lane; i < E; i += 64) sum += exp((double)l[i] - (double)mx);
#pragma unroll
  for (int off = 32; off > 0; off >>= 1) sum += __shfl_xor(sum, off, 64);
  float p[16];
  const int per = (E + 63) / 64;
#pragma unroll
  for (int j = 0; j < 16; ++j) {
    const int i = lane + 64 * j;
    p[j] = (j < per && i < E) ? (float)(exp((double)l[i] - (double)mx) / sum) : -INFINITY;
  }
  float psum = 0.f;
  for (int r = 0; r < k; ++r) {
    float bp = -INFINITY;
    int bi = 0x7fffffff;
#pragma unroll
    for (int j = 0; j < 16; ++j) {
      const int i = lane + 64 * j;
      if (i < E && (p[j] > bp || (p[j] == bp && i < bi))) {
        bp = p[j];
        bi = i;
      }
    }
#pragma unroll
    for (int off = 32; off > 0; off >>= 1) {
      const float op = __shfl_xor(bp, off, 64);
      const int oi = __shfl_xor(bi, off, 64);
      if (op > bp || (op == bp && oi < bi)) {
        bp = op;
        bi = oi;
      }
    }
#pragma unroll
    for (int j = 0; j < 16; ++j) {
      if (lane + 64 * j == bi) p[j] = -INFINITY;
    }
    if (lane == r) {
      ids[0] = bi;
      w[0] = bp;
    }
    psum = (r == 0) ? bp : psum + bp;  // sequential f32 sum in rank order
  }
  const float den = psum > min_sum ? psum : min_sum;
  if (lane < k) w[0] = w[0] / den;
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
// the first and last block, 100 MHz real-time clock.
__device__ uint64_t* g_trace = nullptr;
#define AIMA_TRACE(L, slot)                                                          \
  do {                                                                               \
    if (g_trace && (threadIdx.x == 0 || threadIdx.x == 64) && (b == 0 || b == nb - 1)) \
      g_trace[(b == 0 ? 0 : 4096) + (L) * 32 + (threadIdx.x ? 16 : 0) + (slot)] =      \
          __builtin_amdgcn_s_memrealtime();                                          \
  } while (0)
#define AIMA_TRACE_WAIT_LOADS() asm volatile("s_waitcnt vmcnt(0)" ::: "memory")
#else
#define AIMA_TRACE(L, slot) \
  do {                      \
  } while (0)
#define AIMA_TRACE_WAIT_LOADS() \
  do {                          \
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
  const int nb = gridDim.x;
  const int b = blockIdx.x;
  const int k = a.k;
  const int slots = k + 1;
  const int pairs = slots * kI;
  constexpr int kActStride = kMaxSlots * kI / 3;  // act records per parity buffer
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

  if (threadIdx.x == 0) S.abort = 0;
  {
    const uint32_t* src = reinterpret_cast<const uint32_t*>(a.layers);
    uint32_t* dst = reinterpret_cast<uint32_t*>(S.table);
    const int words = a.n_layers * (int)(sizeof(aima_moe_layer) / 4);
    for (int i = threadIdx.x; i < words; i += kThreads) dst[i] = src[i];
  }
  // block 0 advances the launch counter on every exit path
  auto finish = [&]() {
    if (b == 0 && threadIdx.x == 0) *a.epoch_counter = *a.epoch_counter + 1u;
  };

  // ---- router prologue: block L publishes layer L's top-k ------------------
  for (int L = b; L < a.n_layers; L += nb) {
    if (wave == 0) {
      int32_t id = 0;
      float w = 0.f;
      if (a.logits) {
        route_layer(a.logits + (int64_t)L * a.experts, a.experts, k, a.min_weight_sum, &id, &w);
      } else if (lane < k) {
        id = a.ids_in[L * k + lane];
        w = a.w_in[L * k + lane];
      }
      if (lane < k) {
        st_coherent32(&a.route_ids[L * k + lane], pack_word((uint16_t)id, route_epoch));
        st_coherent64(&a.route_w[L * k + lane], pack_f32(w, route_epoch));
      }
    }
  }
  // own residual rows of r_0
  if (threadIdx.x < kRowsB) S.rown[threadIdx.x] = h2f(a.r0[h0 + threadIdx.x]);

  // control wave: fetch route of layer 0 into LDS
  auto poll_route = [&](int L) -> bool {
    const int buf = L & 1;
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
        if (lane < k) {
          int id = (int)(idw & 0xffffu);
          if (id >= a.experts) {
            atomicOr(a.err, AIMA_DEVERR_EXPERT_RANGE);
            id = -1;
          }
          S.route_id[buf][lane] = id;
          S.route_w[buf][lane] = __builtin_bit_cast(float, (uint32_t)ww);
        }
        return true;
      }
      if (++spins > kSpinLimit) return false;
      __builtin_amdgcn_s_sleep(2);
    }
  };
  if (wave == 0) {
    if (!poll_route(0)) {
      if (lane == 0) {
        atomicOr(a.err, 4u);
        S.abort = 1;
      }
    }
  }
  __syncthreads();
  if (S.abort) {
    finish();
    return;
  }

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

  // Weight loads go through buffer resources (base and byte bound in SGPRs,
  // 32-bit offsets in VGPRs): few registers, and an out-of-range offset reads
  // zero instead of faulting.
  // (table pointers come from LDS; readfirstlane makes them provably
  // wave-uniform so the descriptors live in SGPRs without a waterfall loop)
  auto rsrc = [](const void* base, uint32_t bytes) {
    const uint64_t v = reinterpret_cast<uint64_t>(base);
    const uint32_t lo = __builtin_amdgcn_readfirstlane((uint32_t)v);
    const uint32_t hi = __builtin_amdgcn_readfirstlane((uint32_t)(v >> 32));
    void* u = reinterpret_cast<void*>(((uint64_t)hi << 32) | lo);
    return __builtin_amdgcn_make_buffer_rsrc(u, 0, bytes, 0x00020000);
  };
  constexpr int kAux = 2;  // non-temporal: weights are streamed once
  const int E = a.experts;
  auto prefetch_a = [&](int L) {
    const aima_moe_layer& Ly = S.table[L];
    const int buf = L & 1;
    const uint32_t wbytes = (uint32_t)(2 * kI) * (kH / 2);      // per expert
    const uint32_t sbytes = (uint32_t)(2 * kI) * gA * 2;
    const uint32_t zbytes = (uint32_t)(2 * kI) * gA / 2;
    const auto rw = rsrc(Ly.gate_up.qweight, wbytes * E);
    const auto rs = rsrc(Ly.gate_up.scale, sbytes * E);
    const auto rz = rsrc(Ly.gate_up.zp, zbytes * E);
    const auto qw = rsrc(Ly.shared_gate_up.qweight, wbytes);
    const auto qs = rsrc(Ly.shared_gate_up.scale, sbytes);
    const auto qz = rsrc(Ly.shared_gate_up.zp, zbytes);
#pragma unroll
    for (int i = 0; i < kMaxRowsA; ++i) {
      const int ri = cw + kComputeWaves * i;  // row index within the block
      const int p = ri >> 1;
      wa[i] = u32x4{0u, 0u, 0u, 0u};
      sa[i] = 0u;
      za[i] = 0u;
      if (p < npairs) {
        const int pair = pair0 + p;
        const int slot = pair / kI;
        const int j = pair - slot * kI;
        const int row = (ri & 1) ? kI + j : j;
        const int gi = row * gA + ((lane * 32) >> glog2);
        const uint32_t vw = (uint32_t)row * (kH / 2) + lane * 16;
        if (slot < k) {
          const int e = __builtin_amdgcn_readfirstlane(S.route_id[buf][slot]);
          if (e < 0) continue;
          wa[i] = __builtin_amdgcn_raw_buffer_load_b128(rw, vw, (uint32_t)e * wbytes, kAux);
          sa[i] = __builtin_amdgcn_raw_buffer_load_b32(rs, (gi * 2) & ~3, (uint32_t)e * sbytes, 0);
          za[i] = __builtin_amdgcn_raw_buffer_load_b32(rz, (gi >> 1) & ~3, (uint32_t)e * zbytes, 0);
        } else {
          wa[i] = __builtin_amdgcn_raw_buffer_load_b128(qw, vw, 0, kAux);
          sa[i] = __builtin_amdgcn_raw_buffer_load_b32(qs, (gi * 2) & ~3, 0, 0);
          za[i] = __builtin_amdgcn_raw_buffer_load_b32(qz, (gi >> 1) & ~3, 0, 0);
        }
      }
    }
  };
  // B units: u = cw + 7 i -> slot = u / 2, pass = u % 2 (4 rows per pass)
  auto prefetch_b = [&](int L) {
    const aima_moe_layer& Ly = S.table[L];
    const int buf = L & 1;
    const int seg = lane >> 4, cl = lane & 15;
    const uint32_t wbytes = (uint32_t)kH * (kI / 2);
    const uint32_t sbytes = (uint32_t)kH * gB * 2;
    const uint32_t zbytes = (uint32_t)kH * gB / 2;
    const auto rw = rsrc(Ly.down.qweight, wbytes * E);
    const auto rs = rsrc(Ly.down.scale, sbytes * E);
    const auto rz = rsrc(Ly.down.zp, zbytes * E);
    const auto qw = rsrc(Ly.shared_down.qweight, wbytes);
    const auto qs = rsrc(Ly.shared_down.scale, sbytes);
    const auto qz = rsrc(Ly.shared_down.zp, zbytes);
#pragma unroll
    for (int i = 0; i < kMaxUnitsB; ++i) {
      const int u = cw + kComputeWaves * i;
      const int slot = u >> 1;
      wb[i] = u32x4{0u, 0u, 0u, 0u};
      sb[i] = 0u;
      zb[i] = 0u;
      if (slot < slots) {
        const int row = h0 + (u & 1) * 4 + seg;
        const int gi = row * gB + ((cl * 32) >> glog2);
        const uint32_t vw = (uint32_t)row * (kI / 2) + cl * 16;
        if (slot < k) {
          const int e = __builtin_amdgcn_readfirstlane(S.route_id[buf][slot]);
          if (e < 0) continue;
          wb[i] = __builtin_amdgcn_raw_buffer_load_b128(rw, vw, (uint32_t)e * wbytes, kAux);
          sb[i] = __builtin_amdgcn_raw_buffer_load_b32(rs, (gi * 2) & ~3, (uint32_t)e * sbytes, 0);
          zb[i] = __builtin_amdgcn_raw_buffer_load_b32(rz, (gi >> 1) & ~3, (uint32_t)e * zbytes, 0);
        } else {
          wb[i] = __builtin_amdgcn_raw_buffer_load_b128(qw, vw, 0, kAux);
          sb[i] = __builtin_amdgcn_raw_buffer_load_b32(qs, (gi * 2) & ~3, 0, 0);
          zb[i] = __builtin_amdgcn_raw_buffer_load_b32(qz, (gi >> 1) & ~3, 0, 0);
        }
      }
    }
  };

  if (wave > 0) prefetch_a(0);

  for (int L = 0; L < a.n_layers; ++L) {
    const aima_moe_layer& Ly = S.table[L];
    const int buf = L & 1;
    const uint32_t epA = base + 2u * (uint32_t)L;        // act_L
    const uint32_t epB = base + 2u * (uint32_t)L + 1u;   // r_{L+1}
    const uint32_t epR = base + 2u * (uint32_t)L - 1u;   // r_L (L > 0)

    // ================= phase A_L =================
    if (wave == 0) {
      // poll r_L (lane = chunk of 32 values), then x = f16(r * scale * w)
      // into LDS; the raw words stay packed to keep this path's registers low
      uint64_t rv[16];
      if (L == 0) {
        const AIMA_GLOBAL u32x4* p = (const AIMA_GLOBAL u32x4*)(a.r0 + lane * 32);
#pragma unroll
        for (int q = 0; q < 4; ++q) {
          const u32x4 v = p[q];
#pragma unroll
          for (int t = 0; t < 4; ++t) {
            rv[4 * q + t] = (uint64_t)(v[t] & 0xffffu) | ((uint64_t)(v[t] >> 16) << 32);
          }
        }
      } else {
        const uint64_t* src =
            reinterpret_cast<const uint64_t*>(a.r_buf + ((L - 1) & 1) * kH + lane * 32);
        uint32_t spins = 0;
        while (true) {
#pragma unroll
          for (int q = 0; q < 16; ++q) rv[q] = ld_coherent64(src + q);
          bool ok = true;
#pragma unroll
          for (int q = 0; q < 16; ++q) {
            ok = ok && ((uint32_t)rv[q] >> 16) == epR && ((uint32_t)(rv[q] >> 32) >> 16) == epR;
          }
          if (__all(ok)) break;
          if (++spins > kSpinLimit) {
            if (lane == 0) {
              atomicOr(a.err, 4u);
              S.abort = 1;
            }
            break;
          }
          __builtin_amdgcn_s_sleep(1);
        }
      }
      float ss = 0.f;
#pragma unroll
      for (int q = 0; q < 16; ++q) {
        const float v0 = h2f((uint16_t)rv[q]), v1 = h2f((uint16_t)(rv[q] >> 32));
        ss += v0 * v0;
        ss += v1 * v1;
      }
      ss = segment_sum<64>(ss);
      const float scale = 1.0f / sqrtf(ss / (float)kH + a.eps);
      const AIMA_GLOBAL float* nw = (const AIMA_GLOBAL float*)(Ly.norm_weight + lane * 32);
#pragma unroll
      for (int q = 0; q < 16; ++q) {
        const float n0 = nw[2 * q], n1 = nw[2 * q + 1];
        const float v0 = h2f((uint16_t)rv[q]), v1 = h2f((uint16_t)(rv[q] >> 32));
        S.xa[lane * 16 + q] = f2h(v0 * scale * n0) | ((uint32_t)f2h(v1 * scale * n1) << 16);
      }
      // shared-expert gate: sigma = sigmoid(gate_vec . x) (block 0 publishes)
      if (b == 0) {
        const AIMA_GLOBAL uint32_t* gv =
            (const AIMA_GLOBAL uint32_t*)(Ly.shared_gate_vec + lane * 32);
        float g = 0.f;
#pragma unroll
        for (int q = 0; q < 16; ++q) {
          const f16x2 gg = as_h2(gv[q]);
          const f16x2 xx = as_h2(S.xa[lane * 16 + q]);
          g += (float)gg.x * (float)xx.x;
          g += (float)gg.y * (float)xx.y;
        }
        g = segment_sum<64>(g);
        if (lane == 0) {
          const double t = g;
          const double sg = t >= 0.0 ? 1.0 / (1.0 + exp(-t)) : exp(t) / (1.0 + exp(t));
          st_coherent64(&a.sigma_buf[buf], pack_f32((float)sg, epA));
        }
      }
      // fetch next layer's route into LDS while the compute waves work
      if (L + 1 < a.n_layers && !S.abort) {
        if (!poll_route(L + 1) && lane == 0) {
          atomicOr(a.err, 4u);
          S.abort = 1;
        }
      }
    }
    AIMA_TRACE(L, 0);
    __syncthreads();  // #1: A operands ready
    AIMA_TRACE(L, 1);
    if (S.abort) {
      finish();
      return;
    }
    if (wave > 0) {
      AIMA_TRACE_WAIT_LOADS();
      AIMA_TRACE(L, 10);  // wave 1: prefetched A weights landed
      XChunk xc;
      lds_xchunk(S.xa, lane * 16, xc);
#pragma unroll
      for (int i = 0; i < kMaxRowsA; ++i) {
        const int ri = cw + kComputeWaves * i;
        if ((ri >> 1) < npairs) {
          const int pair = pair0 + (ri >> 1);
          const int row = (ri & 1) ? kI + (pair % kI) : (pair % kI);
          const int gi = row * gA + ((lane * 32) >> glog2);
          const float d = segment_sum<64>(
              u4_chunk_dot(wa[i], xc, nib(za[i], gi), scl(sa[i], gi)));
          if (lane == 0) S.rowsum[ri] = d;
        }
      }
      AIMA_TRACE(L, 11);  // wave 1: A dots done
    }
    __syncthreads();  // #2: row sums ready
    AIMA_TRACE(L, 2);
    if (wave > 0) {
      // SwiGLU for the block's pairs, published three per {3 x f16, epoch}
      const int t = threadIdx.x - 64;
      if (3 * t < npairs) {
        uint64_t rec = (uint64_t)epA << 48;
#pragma unroll
        for (int j = 0; j < 3; ++j) {
          const int p = 3 * t + j;
          const uint16_t h = p < npairs ? f2h(silu_mul(S.rowsum[2 * p], S.rowsum[2 * p + 1]))
                                        : (uint16_t)0;
          rec |= (uint64_t)h << (16 * j);
        }
        st_coherent64(&a.act_buf[buf * kActStride + pair0 / 3 + t], rec);
      }
      prefetch_b(L);
    } else {
      // poll act_L (all slots, fixed-size region so every load is issued in
      // one unrolled batch) and sigma_L; stage the f16 pairs in LDS
      constexpr int kQ = kActStride / 64;   // record loads per lane
      const int nrec = (pairs + 2) / 3;      // valid records
      const uint64_t* src = a.act_buf + buf * kActStride;
      uint32_t spins = 0;
      while (true) {
        uint64_t v[kQ];
#pragma unroll
        for (int q = 0; q < kQ; ++q) v[q] = ld_coherent64(src + lane + 64 * q);
        const uint64_t sv = ld_coherent64(&a.sigma_buf[buf]);
        bool ok = (uint32_t)(sv >> 32) == epA;
#pragma unroll
        for (int q = 0; q < kQ; ++q) {
          ok = ok && (lane + 64 * q >= nrec || (uint32_t)(v[q] >> 48) == epA);
        }
        if (__all(ok)) {
          uint16_t* d = S.xb16();
#pragma unroll
          for (int q = 0; q < kQ; ++q) {
            const int r = lane + 64 * q;
            d[3 * r + 0] = (uint16_t)v[q];
            d[3 * r + 1] = (uint16_t)(v[q] >> 16);
            d[3 * r + 2] = (uint16_t)(v[q] >> 32);
          }
          if (lane == 0) S.sigma = __builtin_bit_cast(float, (uint32_t)sv);
          break;
        }
        if (++spins > kSpinLimit) {
          if (lane == 0) {
            atomicOr(a.err, 4u);
            S.abort = 1;
          }
          break;
        }
        __builtin_amdgcn_s_sleep(1);
      }
    }
    AIMA_TRACE(L, 3);
    __syncthreads();  // #3: B operands ready
    AIMA_TRACE(L, 4);
    if (S.abort) {
      finish();
      return;
    }
    if (wave > 0) {
      AIMA_TRACE_WAIT_LOADS();
      AIMA_TRACE(L, 12);  // wave 1: prefetched B weights landed
      const int seg = lane >> 4, cl = lane & 15;
#pragma unroll
      for (int i = 0; i < kMaxUnitsB; ++i) {
        const int u = cw + kComputeWaves * i;
        const int slot = u >> 1;
        if (slot < slots) {
          XChunk xc;
          lds_xchunk(S.xb, slot * (kI / 2) + cl * 16, xc);
          const int row = h0 + (u & 1) * 4 + seg;
          const int gi = row * gB + ((cl * 32) >> glog2);
          const float d = segment_sum<16>(
              u4_chunk_dot(wb[i], xc, nib(zb[i], gi), scl(sb[i], gi)));
          if (cl == 0) S.part[slot][(u & 1) * 4 + seg] = d;
        }
      }
    }
    __syncthreads();  // #4: partial sums ready
    AIMA_TRACE(L, 5);
    if (wave > 0) {
      if (L + 1 < a.n_layers) prefetch_a(L + 1);
    } else if (lane < kRowsB) {
      float f = 0.f;
      for (int s = 0; s < k; ++s) {
        const float c = S.route_id[buf][s] < 0 ? 0.f : S.route_w[buf][s];
        f += c * S.part[s][lane];
      }
      f += S.sigma * S.part[k][lane];
      const uint16_t o = f2h(S.rown[lane] + f);
      S.rown[lane] = h2f(o);
      if (L + 1 < a.n_layers) {
        st_coherent32(&a.r_buf[(L & 1) * kH + h0 + lane], pack_word(o, epB));
      } else {
        a.out[h0 + lane] = o;
      }
    }
  }
  AIMA_TRACE(a.n_layers, 0);
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
  uint64_t* sigma_buf = nullptr;
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
  const size_t o_sigma = take(sizeof(uint64_t) * 2);
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
  p->sigma_buf = reinterpret_cast<uint64_t*>(p->mem + o_sigma);
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
  a.sigma_buf = plan->sigma_buf;
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
