// Batch-1 MoE FFN decode on gfx950: two bandwidth-bound launches per layer.
//
// Phase A (gate/up + SwiGLU): the k routed experts and the shared expert form
// (k+1)*I row pairs (gate row j, up row I+j).  Each wave streams two pairs
// (4 rows of H/2 bytes) with 128-bit loads, reduces each row across its lane
// segment and applies silu(gate)*up in registers; the activation is stored as
// f16 [k+1][I].  Block 0 also evaluates the shared expert's scalar gate
// sigmoid(gate_vec . h), with all its threads (row_dot_f16: one wave alone
// made block 0 the last to finish).
//
// Phase B (down + aggregate + residual): each block owns 8 output rows.  Its
// eight waves split the k+1 down matrices (slot s -> wave s % 8) and issue
// all their weight loads before any compute; each lane accumulates
// w_s * (row . act_s) over its slots, and the eight partial sums plus the
// residual are added in a fixed order: no atomics, deterministic.
#include "common.h"

#include <math.h>

#include <mutex>
#include <unordered_map>

namespace aima {

constexpr int kPairsPerWave = 2;
constexpr int kDownRowsPerBlock = 8;
constexpr int kDownThreads = 512;      // 8 waves, wave w owns slots w, w + 8, w + 16
constexpr int kDownSlotsPerWave = 3;   // slots per wave per batch of 24

constexpr int kStackMaxExperts = 1024;  // router logits room in the stack workspace

struct DecodeWs {
  uint32_t* err;
  uint16_t* act;   // [(k+1)][I] f16
  float* sigma;    // shared-expert gate
  uint16_t* h;     // [H] normalized input (stack only)
  uint16_t* r[2];  // [H] residual ping-pong (stack only)
  float* logits;   // [<= 1024] router logits (stack only)
};

static size_t decode_ws_bytes(int64_t hidden, int64_t inter, int k, bool stack) {
  size_t b = kWsHeader;
  b += round_up((size_t)(k + 1) * inter * 2, 256);
  b += 256;
  if (stack) b += 3 * round_up((size_t)hidden * 2, 256) + kStackMaxExperts * 4;
  return b;
}

static DecodeWs decode_ws(void* ws, int64_t hidden, int64_t inter, int k, bool stack) {
  DecodeWs w{};
  char* p = static_cast<char*>(ws);
  w.err = reinterpret_cast<uint32_t*>(p);
  p += kWsHeader;
  w.act = reinterpret_cast<uint16_t*>(p);
  p += round_up((size_t)(k + 1) * inter * 2, 256);
  w.sigma = reinterpret_cast<float*>(p);
  p += 256;
  if (stack) {
    w.h = reinterpret_cast<uint16_t*>(p);
    p += round_up((size_t)hidden * 2, 256);
    w.r[0] = reinterpret_cast<uint16_t*>(p);
    p += round_up((size_t)hidden * 2, 256);
    w.r[1] = reinterpret_cast<uint16_t*>(p);
    p += round_up((size_t)hidden * 2, 256);
    w.logits = reinterpret_cast<float*>(p);
  }
  return w;
}

template <int KCH>
struct Geom {
  static constexpr int NC = KCH > 64 ? KCH / 64 : 1;
  static constexpr int SEG = KCH > 64 ? 64 : KCH;
  static constexpr int RPI = 64 / SEG;
  static constexpr int K = KCH * 32;
};

template <int KCH>
__device__ __forceinline__ void load_chunks(const uint16_t* __restrict__ x, int cl,
                                            XChunk (&xc)[Geom<KCH>::NC]) {
  using G = Geom<KCH>;
#pragma unroll
  for (int i = 0; i < G::NC; ++i) {
    const int c = cl + i * G::SEG;
    const u32x4* p = reinterpret_cast<const u32x4*>(x + (int64_t)c * 32);
    uint32_t w[16];
#pragma unroll
    for (int q = 0; q < 4; ++q) {
      const u32x4 v = p[q];
      w[4 * q + 0] = v[0];
      w[4 * q + 1] = v[1];
      w[4 * q + 2] = v[2];
      w[4 * q + 3] = v[3];
    }
    make_xchunk(w, xc[i]);
  }
}

// ---------------------------------------------------------------------------
// phase A
// ---------------------------------------------------------------------------
// Routing from the layer's router logits (RPER > 0, the routed stack): every
// block selects the top-k itself (router_select_wave, wave 0) before it
// needs its expert id, and block 0 writes the selection to ids_out / w_out
// for the down kernel and the caller.  This replaces a separate selection
// launch; the ids and weights are those of aima_router_topk.
struct RouteIn {
  const float* logits;  // [experts] (RPER > 0)
  float min_weight_sum;
  int32_t* ids_out;     // [k]
  float* w_out;         // [k]
};

template <int KCH, int RPER>
__global__ __launch_bounds__(256) void decode_gateup_kernel(
    const uint16_t* __restrict__ x, aima_moe_layer L, const int32_t* __restrict__ ids_in,
    int k, uint32_t* __restrict__ err, uint16_t* __restrict__ act,
    float* __restrict__ sigma, float* __restrict__ gu_trace, float* __restrict__ gate_logit,
    RouteIn route) {
  using G = Geom<KCH>;
  constexpr int NR = 2 * kPairsPerWave;          // rows per wave
  constexpr int PASSES = (NR + G::RPI - 1) / G::RPI;
  constexpr int BP = 4 * kPairsPerWave;          // pairs per block (one slot, consecutive)
  constexpr int kMaxGroups = G::K / 32;
  // the block's scales and zero points: gate rows j0.. and up rows I+j0..,
  // each a contiguous run, staged through LDS (one element per thread)
  __shared__ __attribute__((aligned(16))) uint16_t s_lds[2 * BP * kMaxGroups];
  __shared__ __attribute__((aligned(16))) uint8_t z_lds[2][BP * kMaxGroups / 2];
  const int lane = threadIdx.x & 63;
  const int wave = threadIdx.x >> 6;
  const int seg = lane / G::SEG;
  const int cl = lane % G::SEG;
  const int64_t I = L.inter;
  const int groups = G::K / L.group;
  const int64_t total_pairs = (int64_t)(k + 1) * I;
  const int64_t bpair0 = (int64_t)blockIdx.x * BP;
  const int64_t pair0 = bpair0 + wave * kPairsPerWave;
  const uint32_t magic = u4_magic();

  const int32_t* ids = ids_in;
  if constexpr (RPER > 0) {
    __shared__ int32_t s_ids[16];
    if (wave == 0) {
      int pick;
      float w, p;
      router_select_wave<RPER>(route.logits, L.experts, k, route.min_weight_sum, pick, w, p);
      if (lane < k) {
        s_ids[lane] = pick;
        if (blockIdx.x == 0) {
          route.ids_out[lane] = pick;
          route.w_out[lane] = w;
        }
      }
    }
    __syncthreads();
    ids = s_ids;
  }
  // the block's slot (inter is a multiple of BP: every block lies in one slot)
  const int64_t slot = bpair0 / I;
  const int64_t j0 = bpair0 - slot * I;
  // the block's gate run (h = 0) and up run (h = 1): rows j0 .. j0 + BP - 1
  // of the expert's gate and up projections, either boundary form
  const uint8_t* qw[2];
  const uint16_t* sc[2];
  const uint8_t* zp[2];
  bool valid = bpair0 < total_pairs;
  {
    int64_t ee = 0;
    if (slot < k) {
      const int32_t e = valid ? ids[slot] : 0;
      if (valid && (e < 0 || e >= L.experts)) {
        if (j0 == 0 && threadIdx.x == 0) atomicOr(err, AIMA_DEVERR_EXPERT_RANGE);
        valid = false;
      }
      ee = valid ? e : 0;
    }
    const GateUpView V = slot < k ? routed_gate_up(L) : shared_gate_up(L);
#pragma unroll
    for (int h = 0; h < 2; ++h) {
      const int64_t r0 = V.row(ee, h, j0);
      qw[h] = V.q[h] + r0 * (G::K / 2);
      sc[h] = V.s[h] + r0 * groups;
      zp[h] = V.z[h] + ((r0 * groups) >> 1);  // r0 * groups is even (j0 % 8 == 0)
    }
  }
  // Load order: the block's scale and zero-point runs (32-bit words where
  // aligned), the activations, then the weights, nothing waited for in
  // between: loads complete in order, so staging the runs in LDS and
  // building the activation operands wait only for the small early loads
  // while the weights stream.  An invalid block loads expert 0's rows (in
  // bounds) and discards them.
  const int n = BP * groups;  // scales per run (zero points: n / 2 bytes)
  const int tid = threadIdx.x;
  const bool words = ((reinterpret_cast<uintptr_t>(sc[0]) | reinterpret_cast<uintptr_t>(sc[1]) |
                       reinterpret_cast<uintptr_t>(zp[0]) | reinterpret_cast<uintptr_t>(zp[1])) &
                      3u) == 0;
  constexpr int kSW = (BP * kMaxGroups + 255) / 256;       // scale words of both runs
  constexpr int kZW = (BP * kMaxGroups / 4 + 255) / 256;   // zero-point words of both runs
  uint32_t sw[kSW], zw[kZW];
#pragma unroll
  for (int j = 0; j < kSW; ++j) {
    const int d = tid + 256 * j, h = d >= n / 2;
    sw[j] = (words && d < n) ? reinterpret_cast<const uint32_t*>(sc[h])[d - h * (n / 2)] : 0u;
  }
#pragma unroll
  for (int j = 0; j < kZW; ++j) {
    const int d = tid + 256 * j, h = d >= n / 8;
    zw[j] = (words && d < n / 4) ? reinterpret_cast<const uint32_t*>(zp[h])[d - h * (n / 8)] : 0u;
  }
  u32x4 xr[G::NC][4];
#pragma unroll
  for (int i = 0; i < G::NC; ++i) {
    const u32x4* p = reinterpret_cast<const u32x4*>(x + (int64_t)(cl + i * G::SEG) * 32);
#pragma unroll
    for (int q = 0; q < 4; ++q) xr[i][q] = p[q];
  }
  u32x4 w[PASSES][G::NC];
#pragma unroll
  for (int ps = 0; ps < PASSES; ++ps) {
    const int ri = ps * G::RPI + seg;  // row index in this wave's list
    const int64_t row = ri < NR ? wave * kPairsPerWave + ri / 2 : 0;  // within the block's run
#pragma unroll
    for (int i = 0; i < G::NC; ++i) {
      const int c = cl + i * G::SEG;
      w[ps][i] = load16_nt(qw[ri & 1] + row * (G::K / 2) + (int64_t)c * 16);
    }
  }
  if (words) {
#pragma unroll
    for (int j = 0; j < kSW; ++j) {
      const int d = tid + 256 * j;
      if (d < n) reinterpret_cast<uint32_t*>(s_lds)[d] = sw[j];
    }
#pragma unroll
    for (int j = 0; j < kZW; ++j) {
      const int d = tid + 256 * j, h = d >= n / 8;
      if (d < n / 4) reinterpret_cast<uint32_t*>(z_lds[h])[d - h * (n / 8)] = zw[j];
    }
  } else {
    for (int t = tid; t < 2 * n; t += 256) {
      const int up = t >= n;
      s_lds[t] = sc[up][t - up * n];
    }
    for (int t = tid; t < n; t += 256) {
      const int up = t >= n / 2;
      z_lds[up][t - up * (n / 2)] = zp[up][t - up * (n / 2)];
    }
  }
  XChunk xc[G::NC];
#pragma unroll
  for (int i = 0; i < G::NC; ++i) {
    uint32_t xw[16];
#pragma unroll
    for (int q = 0; q < 4; ++q) {
      xw[4 * q + 0] = xr[i][q][0];
      xw[4 * q + 1] = xr[i][q][1];
      xw[4 * q + 2] = xr[i][q][2];
      xw[4 * q + 3] = xr[i][q][3];
    }
    make_xchunk(xw, xc[i]);
  }
  __syncthreads();
  float s[PASSES][G::NC];
  uint32_t z[PASSES][G::NC];
  bool ok[PASSES];
#pragma unroll
  for (int ps = 0; ps < PASSES; ++ps) {
    const int ri = ps * G::RPI + seg;
    const int up = ri & 1;
    const int lr = wave * kPairsPerWave + ri / 2;  // row within the block's run
    ok[ps] = valid && ri < NR;
#pragma unroll
    for (int i = 0; i < G::NC; ++i) {
      const int c = cl + i * G::SEG;
      const int gi = lr * groups + ((c * 32) / L.group);
      s[ps][i] = ok[ps] ? h2f(s_lds[up * BP * groups + gi]) : 0.f;
      z[ps][i] = ok[ps] ? (uint32_t)(z_lds[up][gi >> 1] >> ((gi & 1) * 4)) & 0xfu : 0u;
    }
  }
  float v[PASSES];
#pragma unroll
  for (int ps = 0; ps < PASSES; ++ps) {
    float acc = 0.f;
#pragma unroll
    for (int i = 0; i < G::NC; ++i) acc += u4_chunk_dot(w[ps][i], xc[i], z[ps][i], s[ps][i], magic);
    const float t = segment_sum<G::SEG>(acc);  // all lanes active here
    v[ps] = ok[ps] ? t : 0.f;
  }
  // Gather the NR row sums: row ri lives in segment (ri % RPI) of pass ri / RPI.
  float rows[NR];
#pragma unroll
  for (int ri = 0; ri < NR; ++ri) rows[ri] = __shfl(v[ri / G::RPI], (ri % G::RPI) * G::SEG, 64);
  if (lane < kPairsPerWave) {
    const int64_t pair = pair0 + lane;
    if (valid && pair < total_pairs) {
      float g = 0.f, u = 0.f;
#pragma unroll
      for (int p = 0; p < kPairsPerWave; ++p) {
        if (p == lane) {
          g = rows[2 * p];
          u = rows[2 * p + 1];
        }
      }
      act[pair] = f2h(silu_mul(g, u));
      if (gu_trace) {  // the layer trace: gate and up rows, slot-major
        gu_trace[slot * 2 * I + (pair - slot * I)] = g;
        gu_trace[slot * 2 * I + I + (pair - slot * I)] = u;
      }
    }
  }
  if (blockIdx.x == 0) {
    __shared__ float red[4];
    const double t = row_dot_f16(L.shared_gate_vec, x, L.hidden, red);
    if (threadIdx.x == 0) {
      const double r = t >= 0.0 ? 1.0 / (1.0 + exp(-t)) : exp(t) / (1.0 + exp(t));
      *sigma = (float)r;
      if (gate_logit) *gate_logit = (float)t;
    }
  }
}

// ---------------------------------------------------------------------------
// phase B
// ---------------------------------------------------------------------------
// down_trace (the layer trace, else null): each slot's unweighted down row
// sums, [(k+1)][H].
template <int KCH>
__global__ __launch_bounds__(kDownThreads) void decode_down_kernel(
    aima_moe_layer L, const int32_t* __restrict__ ids, const float* __restrict__ rw, int k,
    const uint16_t* __restrict__ act, const float* __restrict__ sigma,
    const uint16_t* __restrict__ residual, uint16_t* __restrict__ out,
    float* __restrict__ down_trace) {
  using G = Geom<KCH>;
  constexpr int PASSES = (kDownRowsPerBlock + G::RPI - 1) / G::RPI;
  constexpr int NW = kDownThreads / 64;
  __shared__ float part[NW][PASSES * G::RPI];
  const int lane = threadIdx.x & 63;
  const int wave = threadIdx.x >> 6;
  const int seg = lane / G::SEG;
  const int cl = lane % G::SEG;
  const int64_t H = L.hidden;
  const int64_t I = L.inter;
  const int64_t groups = G::K / L.group;
  const int64_t h0 = (int64_t)blockIdx.x * kDownRowsPerBlock;
  const uint32_t magic = u4_magic();

  float acc[PASSES];
#pragma unroll
  for (int ps = 0; ps < PASSES; ++ps) acc[ps] = 0.f;
  // in each batch of NW * kDownSlotsPerWave slots, wave w owns slots
  // base + w + q NW (<= k) and issues all their weight loads before any
  // compute; k + 1 <= 24 takes one batch
  for (int base = 0; base <= k; base += NW * kDownSlotsPerWave) {
    u32x4 w[kDownSlotsPerWave][PASSES][G::NC];
    float s[kDownSlotsPerWave][PASSES][G::NC];
    uint32_t z[kDownSlotsPerWave][PASSES][G::NC];
    float coef[kDownSlotsPerWave];
#pragma unroll
    for (int q = 0; q < kDownSlotsPerWave; ++q) {
      const int slot = base + wave + q * NW;
      const uint8_t* qw = L.shared_down.qweight;
      const uint16_t* sc = L.shared_down.scale;
      const uint8_t* zp = L.shared_down.zp;
      bool live = slot <= k;
      coef[q] = 0.f;
      if (live && slot < k) {
        const int32_t e = ids[slot];
        if (e < 0 || e >= L.experts) {
          live = false;  // flagged by phase A
        } else {
          qw = L.down.qweight + (int64_t)e * H * (G::K / 2);
          sc = L.down.scale + (int64_t)e * H * groups;
          zp = L.down.zp + (int64_t)e * (H * groups / 2);
          coef[q] = rw[slot];
        }
      } else if (live) {
        coef[q] = *sigma;
      }
#pragma unroll
      for (int ps = 0; ps < PASSES; ++ps) {
        const int64_t row = h0 + ps * G::RPI + seg;
#pragma unroll
        for (int i = 0; i < G::NC; ++i) {
          const int c = cl + i * G::SEG;
          if (live && ps * G::RPI + seg < kDownRowsPerBlock && row < H) {
            w[q][ps][i] = load16_nt(qw + row * (G::K / 2) + (int64_t)c * 16);
            const int64_t gi = row * groups + ((int64_t)c * 32) / L.group;
            s[q][ps][i] = h2f(sc[gi]);
            z[q][ps][i] = u4_code(zp, gi);
          } else {
            w[q][ps][i] = u32x4{0u, 0u, 0u, 0u};
            s[q][ps][i] = 0.f;
            z[q][ps][i] = 0u;
          }
        }
      }
    }
#pragma unroll
    for (int q = 0; q < kDownSlotsPerWave; ++q) {
      const int slot = base + wave + q * NW;
      if (slot > k) break;
      XChunk xc[G::NC];
      load_chunks<KCH>(act + (int64_t)slot * I, cl, xc);
#pragma unroll
      for (int ps = 0; ps < PASSES; ++ps) {
        float d = 0.f;
#pragma unroll
        for (int i = 0; i < G::NC; ++i)
          d += u4_chunk_dot(w[q][ps][i], xc[i], z[q][ps][i], s[q][ps][i], magic);
        acc[ps] += coef[q] * d;
        if (down_trace) {
          const float t = segment_sum<G::SEG>(d);
          const int64_t row = h0 + ps * G::RPI + seg;
          if (cl == 0 && ps * G::RPI + seg < kDownRowsPerBlock && row < H)
            down_trace[(int64_t)slot * H + row] = t;
        }
      }
    }
  }
#pragma unroll
  for (int ps = 0; ps < PASSES; ++ps) {
    const float t = segment_sum<G::SEG>(acc[ps]);
    if (cl == 0) part[wave][ps * G::RPI + seg] = t;
  }
  __syncthreads();
  if (threadIdx.x < kDownRowsPerBlock) {
    const int64_t row = h0 + threadIdx.x;
    if (row < H) {
      float f = part[0][threadIdx.x];
#pragma unroll
      for (int ww = 1; ww < NW; ++ww) f += part[ww][threadIdx.x];
      const float r = residual ? h2f(residual[row]) : 0.f;
      out[row] = f2h(r + f);
    }
  }
}

// ---------------------------------------------------------------------------
// host side
// ---------------------------------------------------------------------------
static int check_layer(const aima_moe_layer* L, int k, bool need_norm) {
  AIMA_REQUIRE(L != nullptr, "moe: null layer");
  AIMA_REQUIRE(L->gate_up.qweight && L->gate_up.scale && L->gate_up.zp,
               "moe: null routed gate/up tensor");
  AIMA_REQUIRE(L->down.qweight && L->down.scale && L->down.zp, "moe: null routed down tensor");
  AIMA_REQUIRE(L->shared_gate_up.qweight && L->shared_gate_up.scale && L->shared_gate_up.zp,
               "moe: null shared gate/up tensor");
  AIMA_REQUIRE(L->shared_down.qweight && L->shared_down.scale && L->shared_down.zp,
               "moe: null shared down tensor");
  AIMA_REQUIRE(L->shared_gate_vec != nullptr, "moe: null shared gate vector");
  AIMA_REQUIRE(!need_norm || L->norm_weight != nullptr, "moe: null norm weight");
  AIMA_REQUIRE(L->experts > 0 && k > 0 && k <= L->experts, "moe: need 0 < k <= experts");
  AIMA_REQUIRE(L->shared_inter == L->inter, "moe: shared_inter must equal inter");
  AIMA_REQUIRE(L->group == 32 || L->group == 64 || L->group == 128 || L->group == 256,
               "moe: group must be 32, 64, 128 or 256");
  AIMA_REQUIRE(L->hidden % L->group == 0 && L->inter % L->group == 0,
               "moe: hidden and inter must be multiples of group");
  AIMA_REQUIRE(aligned(L->gate_up.qweight, 16) && aligned(L->down.qweight, 16) &&
                   aligned(L->shared_gate_up.qweight, 16) && aligned(L->shared_down.qweight, 16),
               "moe: qweight pointers must be 16-byte aligned");
  AIMA_REQUIRE(split_tensors_ok(*L),
               "moe: a split up tensor needs qweight, scale and zp (qweight 16-byte aligned)");
  return AIMA_OK;
}

static bool decode_shape_ok(const aima_moe_layer* L) {
  const int64_t hk = L->hidden / 32, ik = L->inter / 32;
  return L->hidden % 32 == 0 && L->inter % 32 == 0 && (hk == 16 || hk == 32 || hk == 64 ||
         hk == 128) && (ik == 4 || ik == 8 || ik == 16 || ik == 32 || ik == 64);
}

// Trace buffers of aima_moe_ffn_layer_trace (all null on the product path).
struct DecodeTrace {
  float* gate_up;     // [(k+1)][2I]
  float* gate_logit;  // [1]
  float* down;        // [(k+1)][H]
};

template <int KCH, int RPER>
static void launch_gateup_r(const uint16_t* x, const aima_moe_layer& L, const int32_t* ids, int k,
                            const DecodeWs& w, const DecodeTrace& tr, const RouteIn& route,
                            hipStream_t st) {
  const int64_t pairs = (int64_t)(k + 1) * L.inter;
  const int64_t waves = (pairs + kPairsPerWave - 1) / kPairsPerWave;
  const int64_t blocks = (waves + 3) / 4;
  hipLaunchKernelGGL((decode_gateup_kernel<KCH, RPER>), dim3((unsigned)blocks), dim3(256), 0, st,
                     x, L, ids, k, w.err, w.act, w.sigma, tr.gate_up, tr.gate_logit, route);
}

// route.logits null: the ids are given; else the selection per block, with
// the logits per lane (experts / 64 rounded up to a power of two) as the
// template argument.
template <int KCH>
static void launch_gateup(const uint16_t* x, const aima_moe_layer& L, const int32_t* ids, int k,
                          const DecodeWs& w, const DecodeTrace& tr, hipStream_t st,
                          const RouteIn& route = RouteIn{}) {
  if (!route.logits) {
    launch_gateup_r<KCH, 0>(x, L, ids, k, w, tr, route, st);
  } else if (L.experts <= 64) {
    launch_gateup_r<KCH, 1>(x, L, ids, k, w, tr, route, st);
  } else if (L.experts <= 128) {
    launch_gateup_r<KCH, 2>(x, L, ids, k, w, tr, route, st);
  } else if (L.experts <= 256) {
    launch_gateup_r<KCH, 4>(x, L, ids, k, w, tr, route, st);
  } else if (L.experts <= 512) {
    launch_gateup_r<KCH, 8>(x, L, ids, k, w, tr, route, st);
  } else {
    launch_gateup_r<KCH, 16>(x, L, ids, k, w, tr, route, st);
  }
}

template <int KCH>
static void launch_down(const aima_moe_layer& L, const int32_t* ids, const float* rw, int k,
                        const DecodeWs& w, const uint16_t* residual, uint16_t* out,
                        const DecodeTrace& tr, hipStream_t st) {
  const int64_t blocks = (L.hidden + kDownRowsPerBlock - 1) / kDownRowsPerBlock;
  hipLaunchKernelGGL((decode_down_kernel<KCH>), dim3((unsigned)blocks), dim3(kDownThreads), 0, st, L,
                     ids, rw, k, w.act, w.sigma, residual, out, tr.down);
}

// route.logits set: the gate/up kernel selects the route from the logits
// and writes it to ids / rw (route.ids_out == ids, route.w_out == rw), which
// the down kernel then reads.
static int decode_layer(const aima_moe_layer& L, const uint16_t* x, const uint16_t* residual,
                        const int32_t* ids, const float* rw, int k, uint16_t* out,
                        const DecodeWs& w, hipStream_t st, const DecodeTrace& tr = DecodeTrace{},
                        const RouteIn& route = RouteIn{}) {
  switch (L.hidden / 32) {
    case 16: launch_gateup<16>(x, L, ids, k, w, tr, st, route); break;
    case 32: launch_gateup<32>(x, L, ids, k, w, tr, st, route); break;
    case 64: launch_gateup<64>(x, L, ids, k, w, tr, st, route); break;
    case 128: launch_gateup<128>(x, L, ids, k, w, tr, st, route); break;
    default: return fail(AIMA_E_UNSUPPORTED, "moe decode: unsupported hidden size");
  }
  int rc = launch_check("moe decode gate/up");
  if (rc != AIMA_OK) return rc;
  switch (L.inter / 32) {
    case 4: launch_down<4>(L, ids, rw, k, w, residual, out, tr, st); break;
    case 8: launch_down<8>(L, ids, rw, k, w, residual, out, tr, st); break;
    case 16: launch_down<16>(L, ids, rw, k, w, residual, out, tr, st); break;
    case 32: launch_down<32>(L, ids, rw, k, w, residual, out, tr, st); break;
    case 64: launch_down<64>(L, ids, rw, k, w, residual, out, tr, st); break;
    default: return fail(AIMA_E_UNSUPPORTED, "moe decode: unsupported intermediate size");
  }
  return launch_check("moe decode down");
}

// The layer trace's sums, one thread per output row: the weighted routed
// rows and their rank-order sum (apply_expert_weights, aggregate_experts),
// the gated shared row and the FFN output.  down: [(k+1)][H] unweighted.
__global__ __launch_bounds__(256) void trace_combine_kernel(
    const float* __restrict__ down, const float* __restrict__ rw, const float* __restrict__ sigma,
    int k, int64_t H, float* __restrict__ weighted, float* __restrict__ moe_out,
    float* __restrict__ shared_gated, float* __restrict__ ffn_out) {
  // separately rounded products and sums (no contraction into fused
  // multiply-adds), as the reference's separate passes compute them
#pragma clang fp contract(off)
  const int64_t h = (int64_t)blockIdx.x * 256 + threadIdx.x;
  if (h >= H) return;
  float m = 0.f;
  for (int r = 0; r < k; ++r) {
    const float v = down[(int64_t)r * H + h] * rw[r];
    weighted[(int64_t)r * H + h] = v;
    m += v;
  }
  const float g = down[(int64_t)k * H + h] * *sigma;
  moe_out[h] = m;
  shared_gated[h] = g;
  ffn_out[h] = m + g;
}

static size_t trace_ws_bytes(const aima_moe_layer& L, int k) {
  return decode_ws_bytes(L.hidden, L.inter, k, false) +
         round_up((size_t)(k + 1) * 2 * L.inter * 4, 256) +
         round_up((size_t)(k + 1) * L.hidden * 4, 256);
}

int rmsnorm_launch(const uint16_t* x, const float* weight, int64_t rows, int64_t hidden,
                   float eps, uint16_t* out, hipStream_t st);
int u4_matvec_dispatch(const uint16_t* x, const uint8_t* qw, const uint16_t* scale,
                       const uint8_t* zp, int64_t n, int64_t k, int glog2, void* y,
                       int out_f32, hipStream_t st);
int router_topk_launch(const float* logits, int64_t tokens, int experts, int k,
                       float min_weight_sum, int32_t* ids, float* weights, hipStream_t st,
                       float* probs = nullptr);
int group_log2_of(int group);

}  // namespace aima

using namespace aima;

extern "C" int aima_moe_decode_workspace_size(const aima_moe_layer* layer, int32_t k,
                                              size_t* bytes) {
  AIMA_REQUIRE(layer && bytes, "moe_decode_workspace_size: null pointer");
  AIMA_REQUIRE(k > 0, "moe_decode_workspace_size: k must be positive");
  *bytes = decode_ws_bytes(layer->hidden, layer->inter, k, true);
  return AIMA_OK;
}

extern "C" int aima_moe_ffn_layer_trace_workspace_size(const aima_moe_layer* layer, int32_t k,
                                                       size_t* bytes) {
  AIMA_REQUIRE(layer && bytes, "moe_ffn_layer_trace_workspace_size: null pointer");
  AIMA_REQUIRE(k > 0, "moe_ffn_layer_trace_workspace_size: k must be positive");
  *bytes = trace_ws_bytes(*layer, k);
  return AIMA_OK;
}

extern "C" int aima_moe_ffn_layer_trace(const aima_moe_layer* layer, const aima_u4_tensor* router,
                                        const uint16_t* residual, float eps, int32_t k,
                                        float min_weight_sum, const aima_ffn_trace* t,
                                        void* workspace, size_t workspace_bytes, void* stream) {
  int rc = check_layer(layer, k, true);
  if (rc != AIMA_OK) return rc;
  const aima_moe_layer& L = *layer;
  AIMA_REQUIRE(router && router->qweight && router->scale && router->zp && residual && t,
               "moe_ffn_layer_trace: null pointer");
  AIMA_REQUIRE(t->ffn_norm && t->router_logits && t->expert_ids && t->router_weights &&
                   t->normalized_weights && t->selected_gate_up && t->selected_swiglu &&
                   t->selected_down && t->weighted_selected_down && t->moe_out &&
                   t->shared_gate && t->shared_gate_sigmoid && t->shared_gate_up &&
                   t->shared_swiglu && t->shared_down && t->shared_gated && t->ffn_out &&
                   t->residual,
               "moe_ffn_layer_trace: every trace buffer is required");
  AIMA_REQUIRE(L.experts <= 1024 && k <= 16, "moe_ffn_layer_trace: experts <= 1024, k <= 16");
  AIMA_REQUIRE(min_weight_sum > 0.f, "moe_ffn_layer_trace: minimum weight sum must be positive");
  AIMA_REQUIRE(aligned(residual, 16) && aligned(t->ffn_norm, 16) && aligned(router->qweight, 16),
               "moe_ffn_layer_trace: residual, ffn_norm and router qweight must be 16-byte "
               "aligned");
  if (!decode_shape_ok(layer)) {
    return fail(AIMA_E_UNSUPPORTED, "moe_ffn_layer_trace: hidden/32 must be 16..128 and inter/32 4..64 (powers of two)");
  }
  if (!workspace || workspace_bytes < trace_ws_bytes(L, k)) {
    return fail(AIMA_E_WORKSPACE, "moe_ffn_layer_trace: workspace missing or too small");
  }
  AIMA_REQUIRE(aligned(workspace, 256), "moe_ffn_layer_trace: workspace must be 256-byte aligned");
  const hipStream_t st = (hipStream_t)stream;
  const int64_t H = L.hidden, I = L.inter;
  const DecodeWs w = decode_ws(workspace, H, I, k, false);
  char* p = static_cast<char*>(workspace) + decode_ws_bytes(H, I, k, false);
  DecodeTrace tr;
  tr.gate_up = reinterpret_cast<float*>(p);
  tr.down = reinterpret_cast<float*>(p + round_up((size_t)(k + 1) * 2 * I * 4, 256));
  tr.gate_logit = t->shared_gate;
  // ffn_norm, router logits and selection, then the decode kernels
  rc = rmsnorm_launch(residual, L.norm_weight, 1, H, eps, t->ffn_norm, st);
  if (rc != AIMA_OK) return rc;
  rc = u4_matvec_dispatch(t->ffn_norm, router->qweight, router->scale, router->zp, L.experts, H,
                          group_log2_of(L.group), t->router_logits, 1, st);
  if (rc != AIMA_OK) return rc;
  rc = router_topk_launch(t->router_logits, 1, L.experts, k, min_weight_sum, t->expert_ids,
                          t->normalized_weights, st, t->router_weights);
  if (rc != AIMA_OK) return rc;
  rc = decode_layer(L, t->ffn_norm, residual, t->expert_ids, t->normalized_weights, k,
                    t->residual, w, st, tr);
  if (rc != AIMA_OK) return rc;
  // the kernels' own intermediates, split into routed and shared parts
  const size_t gu = (size_t)2 * I * 4, hf = (size_t)H * 4;
  AIMA_HIP(hipMemcpyAsync(t->selected_gate_up, tr.gate_up, k * gu, hipMemcpyDeviceToDevice, st));
  AIMA_HIP(hipMemcpyAsync(t->shared_gate_up, reinterpret_cast<char*>(tr.gate_up) + k * gu, gu,
                          hipMemcpyDeviceToDevice, st));
  AIMA_HIP(hipMemcpyAsync(t->selected_swiglu, w.act, (size_t)k * I * 2, hipMemcpyDeviceToDevice,
                          st));
  AIMA_HIP(hipMemcpyAsync(t->shared_swiglu, w.act + (size_t)k * I, (size_t)I * 2,
                          hipMemcpyDeviceToDevice, st));
  AIMA_HIP(hipMemcpyAsync(t->shared_gate_sigmoid, w.sigma, 4, hipMemcpyDeviceToDevice, st));
  AIMA_HIP(hipMemcpyAsync(t->selected_down, tr.down, k * hf, hipMemcpyDeviceToDevice, st));
  AIMA_HIP(hipMemcpyAsync(t->shared_down, reinterpret_cast<char*>(tr.down) + k * hf, hf,
                          hipMemcpyDeviceToDevice, st));
  hipLaunchKernelGGL(trace_combine_kernel, dim3((unsigned)((H + 255) / 256)), dim3(256), 0, st,
                     tr.down, t->normalized_weights, w.sigma, k, H, t->weighted_selected_down,
                     t->moe_out, t->shared_gated, t->ffn_out);
  return launch_check("moe_ffn_layer_trace");
}

extern "C" int aima_moe_ffn_decode(const aima_moe_layer* layer, const uint16_t* x,
                                   const uint16_t* residual, const int32_t* ids,
                                   const float* weights, int32_t k, uint16_t* out,
                                   void* workspace, size_t workspace_bytes, void* stream) {
  int rc = check_layer(layer, k, false);
  if (rc != AIMA_OK) return rc;
  AIMA_REQUIRE(x && ids && weights && out, "moe_ffn_decode: null pointer");
  AIMA_REQUIRE(aligned(x, 16), "moe_ffn_decode: x must be 16-byte aligned");
  if (!decode_shape_ok(layer)) {
    return fail(AIMA_E_UNSUPPORTED, "moe_ffn_decode: hidden/32 must be 16..128 and inter/32 4..64 (powers of two)");
  }
  if (!workspace || workspace_bytes < decode_ws_bytes(layer->hidden, layer->inter, k, false)) {
    return fail(AIMA_E_WORKSPACE, "moe_ffn_decode: workspace missing or too small");
  }
  AIMA_REQUIRE(aligned(workspace, 256), "moe_ffn_decode: workspace must be 256-byte aligned");
  const DecodeWs w = decode_ws(workspace, layer->hidden, layer->inter, k, false);
  return decode_layer(*layer, x, residual, ids, weights, k, out, w, (hipStream_t)stream);
}

extern "C" int aima_moe_decode_gate_up(const aima_moe_layer* layer, const uint16_t* x,
                                       const int32_t* ids, int32_t k, uint16_t* act,
                                       float* shared_sigma, uint32_t* error_word,
                                       void* stream) {
  int rc = check_layer(layer, k, false);
  if (rc != AIMA_OK) return rc;
  AIMA_REQUIRE(x && ids && act && shared_sigma && error_word, "moe_decode_gate_up: null pointer");
  AIMA_REQUIRE(aligned(x, 16), "moe_decode_gate_up: x must be 16-byte aligned");
  if (!decode_shape_ok(layer)) {
    return fail(AIMA_E_UNSUPPORTED, "moe_decode_gate_up: unsupported hidden/inter");
  }
  DecodeWs w{};
  w.err = error_word;
  w.act = act;
  w.sigma = shared_sigma;
  hipStream_t st = (hipStream_t)stream;
  switch (layer->hidden / 32) {
    case 16: launch_gateup<16>(x, *layer, ids, k, w, DecodeTrace{}, st); break;
    case 32: launch_gateup<32>(x, *layer, ids, k, w, DecodeTrace{}, st); break;
    case 64: launch_gateup<64>(x, *layer, ids, k, w, DecodeTrace{}, st); break;
    case 128: launch_gateup<128>(x, *layer, ids, k, w, DecodeTrace{}, st); break;
    default: return fail(AIMA_E_UNSUPPORTED, "moe decode: unsupported hidden size");
  }
  return launch_check("moe decode gate/up");
}

extern "C" int aima_moe_decode_down(const aima_moe_layer* layer, const uint16_t* act,
                                    const float* shared_sigma, const int32_t* ids,
                                    const float* weights, int32_t k, const uint16_t* residual,
                                    uint16_t* out, void* stream) {
  int rc = check_layer(layer, k, false);
  if (rc != AIMA_OK) return rc;
  AIMA_REQUIRE(act && shared_sigma && ids && weights && out, "moe_decode_down: null pointer");
  AIMA_REQUIRE(aligned(act, 16), "moe_decode_down: act must be 16-byte aligned");
  if (!decode_shape_ok(layer)) {
    return fail(AIMA_E_UNSUPPORTED, "moe_decode_down: unsupported hidden/inter");
  }
  DecodeWs w{};
  w.act = const_cast<uint16_t*>(act);
  w.sigma = const_cast<float*>(shared_sigma);
  hipStream_t st = (hipStream_t)stream;
  switch (layer->inter / 32) {
    case 4: launch_down<4>(*layer, ids, weights, k, w, residual, out, DecodeTrace{}, st); break;
    case 8: launch_down<8>(*layer, ids, weights, k, w, residual, out, DecodeTrace{}, st); break;
    case 16: launch_down<16>(*layer, ids, weights, k, w, residual, out, DecodeTrace{}, st); break;
    case 32: launch_down<32>(*layer, ids, weights, k, w, residual, out, DecodeTrace{}, st); break;
    case 64: launch_down<64>(*layer, ids, weights, k, w, residual, out, DecodeTrace{}, st); break;
    default: return fail(AIMA_E_UNSUPPORTED, "moe decode: unsupported intermediate size");
  }
  return launch_check("moe decode down");
}

extern "C" int aima_moe_stack_decode(const aima_moe_layer* layers, int32_t n_layers, float eps,
                                     const uint16_t* residual_in, const int32_t* ids,
                                     const float* weights, int32_t k, uint16_t* out,
                                     void* workspace, size_t workspace_bytes, void* stream) {
  AIMA_REQUIRE(layers && n_layers > 0, "moe_stack_decode: need at least one layer");
  AIMA_REQUIRE(residual_in && ids && weights && out, "moe_stack_decode: null pointer");
  for (int32_t l = 0; l < n_layers; ++l) {
    int rc = check_layer(&layers[l], k, true);
    if (rc != AIMA_OK) return rc;
    AIMA_REQUIRE(layers[l].hidden == layers[0].hidden && layers[l].inter == layers[0].inter,
                 "moe_stack_decode: all layers must share hidden and inter");
  }
  if (!decode_shape_ok(&layers[0])) {
    return fail(AIMA_E_UNSUPPORTED, "moe_stack_decode: unsupported hidden/inter");
  }
  const size_t need = decode_ws_bytes(layers[0].hidden, layers[0].inter, k, true);
  if (!workspace || workspace_bytes < need) {
    return fail(AIMA_E_WORKSPACE, "moe_stack_decode: workspace missing or too small");
  }
  AIMA_REQUIRE(aligned(workspace, 256), "moe_stack_decode: workspace must be 256-byte aligned");
  const DecodeWs w = decode_ws(workspace, layers[0].hidden, layers[0].inter, k, true);
  hipStream_t st = (hipStream_t)stream;
  const uint16_t* r = residual_in;
  for (int32_t l = 0; l < n_layers; ++l) {
    const aima_moe_layer& L = layers[l];
    int rc = rmsnorm_launch(r, L.norm_weight, 1, L.hidden, eps, w.h, st);
    if (rc != AIMA_OK) return rc;
    uint16_t* dst = (l == n_layers - 1) ? out : w.r[l & 1];
    rc = decode_layer(L, w.h, r, ids + (int64_t)l * k, weights + (int64_t)l * k, k, dst, w, st);
    if (rc != AIMA_OK) return rc;
    r = dst;
  }
  return AIMA_OK;
}

// Argument checks of the routed stack decode (both entry points).
static int check_routed_stack(const aima_moe_layer* layers, const aima_u4_tensor* routers,
                              int32_t n_layers, const uint16_t* residual_in, int32_t k,
                              float min_weight_sum, int32_t* ids, float* weights,
                              uint16_t* out) {
  AIMA_REQUIRE(layers && routers && n_layers > 0, "moe_stack_decode_routed: need layers");
  AIMA_REQUIRE(residual_in && ids && weights && out, "moe_stack_decode_routed: null pointer");
  AIMA_REQUIRE(min_weight_sum > 0.f, "moe_stack_decode_routed: minimum weight sum must be positive");
  for (int32_t l = 0; l < n_layers; ++l) {
    int rc = check_layer(&layers[l], k, true);
    if (rc != AIMA_OK) return rc;
    AIMA_REQUIRE(layers[l].hidden == layers[0].hidden && layers[l].inter == layers[0].inter,
                 "moe_stack_decode_routed: all layers must share hidden and inter");
    AIMA_REQUIRE(routers[l].qweight && routers[l].scale && routers[l].zp,
                 "moe_stack_decode_routed: null router tensor");
    AIMA_REQUIRE(aligned(routers[l].qweight, 16), "moe_stack_decode_routed: router qweight alignment");
    AIMA_REQUIRE(layers[l].experts <= kStackMaxExperts && k <= 16,
                 "moe_stack_decode_routed: experts <= 1024 and k <= 16");
    AIMA_REQUIRE(group_log2_of(layers[l].group) > 0,
                 "moe_stack_decode_routed: group must be 32, 64, 128 or 256");
  }
  if (!decode_shape_ok(&layers[0])) {
    return fail(AIMA_E_UNSUPPORTED, "moe_stack_decode_routed: unsupported hidden/inter");
  }
  return AIMA_OK;
}

// The routed stack decode's launches on workspace w (its error word is w.err).
static int routed_stack_run(const aima_moe_layer* layers, const aima_u4_tensor* routers,
                            int32_t n_layers, float eps, const uint16_t* residual_in, int32_t k,
                            float min_weight_sum, int32_t* ids, float* weights, uint16_t* out,
                            const DecodeWs& w, hipStream_t st) {
  const uint16_t* r = residual_in;
  for (int32_t l = 0; l < n_layers; ++l) {
    const aima_moe_layer& L = layers[l];
    int rc = rmsnorm_launch(r, L.norm_weight, 1, L.hidden, eps, w.h, st);
    if (rc != AIMA_OK) return rc;
    // routing from this layer's normalized input (gguf_loader.cpp:5708-5711)
    rc = u4_matvec_dispatch(w.h, routers[l].qweight, routers[l].scale, routers[l].zp, L.experts,
                            L.hidden, group_log2_of(L.group), w.logits, 1, st);
    if (rc != AIMA_OK) return rc;
    int32_t* ids_l = ids + (int64_t)l * k;
    float* w_l = weights + (int64_t)l * k;
    uint16_t* dst = (l == n_layers - 1) ? out : w.r[l & 1];
    // the selection runs inside the gate/up kernel (no separate launch)
    RouteIn route;
    route.logits = w.logits;
    route.min_weight_sum = min_weight_sum;
    route.ids_out = ids_l;
    route.w_out = w_l;
    rc = decode_layer(L, w.h, r, ids_l, w_l, k, dst, w, st, DecodeTrace{}, route);
    if (rc != AIMA_OK) return rc;
    r = dst;
  }
  return AIMA_OK;
}

extern "C" int aima_moe_stack_decode_routed(const aima_moe_layer* layers,
                                            const aima_u4_tensor* routers, int32_t n_layers,
                                            float eps, const uint16_t* residual_in, int32_t k,
                                            float min_weight_sum, int32_t* ids, float* weights,
                                            uint16_t* out, void* workspace,
                                            size_t workspace_bytes, void* stream) {
  int rc = check_routed_stack(layers, routers, n_layers, residual_in, k, min_weight_sum, ids,
                              weights, out);
  if (rc != AIMA_OK) return rc;
  const size_t need = decode_ws_bytes(layers[0].hidden, layers[0].inter, k, true);
  if (!workspace || workspace_bytes < need) {
    return fail(AIMA_E_WORKSPACE, "moe_stack_decode_routed: workspace missing or too small");
  }
  AIMA_REQUIRE(aligned(workspace, 256), "moe_stack_decode_routed: workspace must be 256-byte aligned");
  const DecodeWs w = decode_ws(workspace, layers[0].hidden, layers[0].inter, k, true);
  return routed_stack_run(layers, routers, n_layers, eps, residual_in, k, min_weight_sum, ids,
                          weights, out, w, (hipStream_t)stream);
}

// ---------------------------------------------------------------------------
// Allocation-free routed stack decode: the workspace is a fixed device array
// of this library (one copy per GPU, kept until the process ends) instead of
// caller memory.  Host code never uses the array's name as an address: the
// device address comes from hipGetSymbolAddress, once per device, with that
// device current.
// ---------------------------------------------------------------------------
namespace {

constexpr size_t kNoAllocScratchBytes = 128 * 1024;
static __device__ __align__(256) uint8_t scratch[kNoAllocScratchBytes];

std::mutex g_scratch_mu;
std::unordered_map<int, void*> g_scratch_ptr;  // device ordinal -> address of `scratch`

int scratch_address(void** ptr) {
  int dev = 0;
  AIMA_HIP(hipGetDevice(&dev));
  std::lock_guard<std::mutex> lock(g_scratch_mu);
  auto it = g_scratch_ptr.find(dev);
  if (it == g_scratch_ptr.end()) {
    void* p = nullptr;
    AIMA_HIP(hipGetSymbolAddress(&p, HIP_SYMBOL(scratch)));
    it = g_scratch_ptr.emplace(dev, p).first;
  }
  *ptr = it->second;
  return AIMA_OK;
}

}  // namespace

extern "C" int aima_moe_stack_decode_routed_noalloc(const aima_moe_layer* layers,
                                                    const aima_u4_tensor* routers,
                                                    int32_t n_layers, float eps,
                                                    const uint16_t* residual_in, int32_t k,
                                                    float min_weight_sum, int32_t* ids,
                                                    float* weights, uint16_t* out,
                                                    uint32_t* error_word, void* stream) {
  int rc = check_routed_stack(layers, routers, n_layers, residual_in, k, min_weight_sum, ids,
                              weights, out);
  if (rc != AIMA_OK) return rc;
  AIMA_REQUIRE(error_word != nullptr, "moe_stack_decode_routed_noalloc: null error word");
  const size_t need = decode_ws_bytes(layers[0].hidden, layers[0].inter, k, true);
  if (need > kNoAllocScratchBytes) {
    return fail(AIMA_E_UNSUPPORTED,
                "moe_stack_decode_routed_noalloc: this shape needs " + std::to_string(need) +
                    " scratch bytes, more than the fixed " +
                    std::to_string(kNoAllocScratchBytes) + " (use aima_moe_stack_decode_routed)");
  }
  void* base = nullptr;
  rc = scratch_address(&base);
  if (rc != AIMA_OK) return rc;
  DecodeWs w = decode_ws(base, layers[0].hidden, layers[0].inter, k, true);
  w.err = error_word;  // device errors go to the caller's word, never cleared here
  return routed_stack_run(layers, routers, n_layers, eps, residual_in, k, min_weight_sum, ids,
                          weights, out, w, (hipStream_t)stream);
}
