// C-ABI shim over the reference engine's CPU ops -- TEST INFRASTRUCTURE ONLY.
//
// Built by oracle/Makefile together with the reference's own
// engine/src/gguf_loader.cpp (compiled where it lies under /root/reference,
// never copied) into oracle/_ref/libiq36_ref.so.  The tests use it to pin the
// C restatement in u4moe_oracle.c bit-for-bit against the reference code.
//
// The only non-trivial piece is a GGUF v3 writer for F32 tensors so that the
// reference's run_qwen36_moe_ffn_layer (gguf_loader.cpp:5654-5782) can be run
// on exactly-dequantized U4 weights.  GGUF dims are listed innermost first, so
// a row-major [E][R][K] array is written with dims {K, R, E}
// (engine/tests/self_test.cpp:129-151 writes its expert fixture the same way).
#include <cstdint>
#include <cstdio>
#include <cstring>
#include <exception>
#include <fstream>
#include <string>
#include <vector>

#include "intel_qwen36/gguf_loader.hpp"

namespace {

thread_local std::string g_last_error;

int fail(const std::exception& e) {
  g_last_error = e.what();
  return -1;
}

std::vector<float> vec(const float* p, std::int64_t n) {
  return std::vector<float>(p, p + n);
}

void copy_out(const std::vector<float>& v, float* out) {
  if (out) std::memcpy(out, v.data(), v.size() * sizeof(float));
}

// One GGUF tensor: dims innermost first, ggml type (0 = F32, 12 = Q4_K) and
// its raw payload.
struct F32Tensor {
  std::string name;
  std::vector<std::uint64_t> dims;
  const float* data;
  std::uint64_t count;
  std::uint32_t type = 0;
  const void* raw = nullptr;   // payload for non-F32 types
  std::uint64_t raw_bytes = 0;
  std::uint64_t nbytes() const { return type == 0 ? count * 4 : raw_bytes; }
  const char* bytes() const {
    return type == 0 ? reinterpret_cast<const char*>(data) : static_cast<const char*>(raw);
  }
};

void put_u32(std::ofstream& out, std::uint32_t v) {
  out.write(reinterpret_cast<const char*>(&v), 4);
}
void put_u64(std::ofstream& out, std::uint64_t v) {
  out.write(reinterpret_cast<const char*>(&v), 8);
}
void put_str(std::ofstream& out, const std::string& s) {
  put_u64(out, s.size());
  out.write(s.data(), static_cast<std::streamsize>(s.size()));
}

void write_gguf_f32(const std::string& path,
                    const std::vector<F32Tensor>& tensors) {
  constexpr std::uint64_t kAlign = 32;
  std::ofstream out(path, std::ios::binary | std::ios::trunc);
  if (!out) throw std::runtime_error("cannot create GGUF file " + path);
  out.write("GGUF", 4);
  put_u32(out, 3);                 // version
  put_u64(out, tensors.size());    // tensor count
  put_u64(out, 2);                 // metadata count
  put_str(out, "general.architecture");
  put_u32(out, 8);                 // string
  put_str(out, "qwen35moe");
  put_str(out, "general.alignment");
  put_u32(out, 4);                 // uint32
  put_u32(out, static_cast<std::uint32_t>(kAlign));
  std::uint64_t offset = 0;
  std::vector<std::uint64_t> offsets;
  for (const auto& t : tensors) {
    put_str(out, t.name);
    put_u32(out, static_cast<std::uint32_t>(t.dims.size()));
    for (auto d : t.dims) put_u64(out, d);
    put_u32(out, t.type);          // ggml type
    put_u64(out, offset);
    offsets.push_back(offset);
    offset += (t.nbytes() + kAlign - 1) / kAlign * kAlign;
  }
  auto pos = static_cast<std::uint64_t>(out.tellp());
  for (; pos % kAlign != 0; ++pos) out.put('\0');
  for (const auto& t : tensors) {
    out.write(t.bytes(), static_cast<std::streamsize>(t.nbytes()));
    for (std::uint64_t b = t.nbytes(); b % kAlign != 0; ++b) out.put('\0');
  }
  if (!out) throw std::runtime_error("GGUF write failed");
}

}  // namespace

extern "C" {

const char* ref_last_error() { return g_last_error.c_str(); }

float ref_sigmoid_scalar(float v) { return iq36::sigmoid_scalar(v); }

int ref_softmax(const float* in, std::int64_t n, float* out) {
  try {
    copy_out(iq36::softmax(vec(in, n)), out);
    return 0;
  } catch (const std::exception& e) {
    return fail(e);
  }
}

int ref_top_k(const float* v, std::int64_t n, std::int64_t k, std::int32_t* out) {
  try {
    auto r = iq36::top_k_indices(vec(v, n), static_cast<int>(k));
    std::memcpy(out, r.data(), r.size() * sizeof(std::int32_t));
    return 0;
  } catch (const std::exception& e) {
    return fail(e);
  }
}

int ref_normalize_weights(const float* w, std::int64_t k, float min_sum, float* out) {
  try {
    copy_out(iq36::normalize_weights(vec(w, k), min_sum), out);
    return 0;
  } catch (const std::exception& e) {
    return fail(e);
  }
}

int ref_select_router_topk(const float* logits, std::int64_t n, std::int64_t k,
                           float min_sum, std::int32_t* ids, float* weights,
                           float* normalized) {
  try {
    auto s = iq36::select_router_topk(vec(logits, n), static_cast<int>(k), min_sum);
    std::memcpy(ids, s.expert_ids.data(), s.expert_ids.size() * sizeof(std::int32_t));
    copy_out(s.weights, weights);
    copy_out(s.normalized_weights, normalized);
    return 0;
  } catch (const std::exception& e) {
    return fail(e);
  }
}

int ref_swiglu_pair(const float* g, const float* u, std::int64_t n, float* out) {
  try {
    copy_out(iq36::apply_swiglu_pair(vec(g, n), vec(u, n)), out);
    return 0;
  } catch (const std::exception& e) {
    return fail(e);
  }
}

int ref_swiglu_from_gate_up(const float* gu, std::int64_t inter,
                            std::int64_t experts, float* out) {
  try {
    copy_out(iq36::apply_swiglu_from_gate_up(vec(gu, 2 * inter * experts),
                                             inter, experts),
             out);
    return 0;
  } catch (const std::exception& e) {
    return fail(e);
  }
}

int ref_apply_expert_weights(const float* down, const float* w,
                             std::int64_t experts, std::int64_t hidden, float* out) {
  try {
    copy_out(iq36::apply_expert_weights(vec(down, experts * hidden),
                                        vec(w, experts), hidden),
             out);
    return 0;
  } catch (const std::exception& e) {
    return fail(e);
  }
}

int ref_aggregate_experts(const float* weighted, std::int64_t experts,
                          std::int64_t hidden, float* out) {
  try {
    copy_out(iq36::aggregate_experts(vec(weighted, experts * hidden), experts, hidden),
             out);
    return 0;
  } catch (const std::exception& e) {
    return fail(e);
  }
}

int ref_rms_norm(const float* x, const float* w, std::int64_t n, float eps, float* out) {
  try {
    copy_out(iq36::apply_rms_norm(vec(x, n), vec(w, n), eps), out);
    return 0;
  } catch (const std::exception& e) {
    return fail(e);
  }
}

// F32 matvec through the reference's GGUF path: W is row-major [rows][k].
int ref_matvec_f32(const char* path, const float* w, std::int64_t rows,
                   std::int64_t k, const float* x, float* y) {
  try {
    write_gguf_f32(path, {{"unit.matrix", {static_cast<std::uint64_t>(k),
                                           static_cast<std::uint64_t>(rows)},
                           w, static_cast<std::uint64_t>(rows * k)}});
    auto index = iq36::parse_gguf_model_index(path);
    copy_out(iq36::matvec_tensor(path, index, "unit.matrix", vec(x, k)), y);
    std::remove(path);
    return 0;
  } catch (const std::exception& e) {
    std::remove(path);
    return fail(e);
  }
}

// One MoE FFN layer through run_qwen36_moe_ffn_layer on F32 tensors.
//   gate_up   [E][2I][H]  rows 0..I-1 gate, I..2I-1 up
//   down      [E][H][I]
//   sh_gate_up[2IS][H]    rows 0..IS-1 gate, IS..2IS-1 up
//   sh_down   [H][IS]
//   router    [E][H]      (ffn_gate_inp)
//   sh_gate   [H]         (ffn_gate_inp_shexp, one row)
//   norm_w    [H]         (post_attention_norm.weight)
int ref_moe_ffn_layer_f32(const char* path, std::int64_t H, std::int64_t I,
                          std::int64_t IS, std::int64_t E, const float* gate_up,
                          const float* down, const float* sh_gate_up,
                          const float* sh_down, const float* router,
                          const float* sh_gate, const float* norm_w,
                          const float* residual, float eps, float* ffn_norm,
                          float* router_logits, std::int32_t* ids,
                          float* normalized_weights, float* selected_gate_up,
                          float* selected_swiglu, float* selected_down,
                          float* moe_out, float* shared_gate_sigmoid,
                          float* shared_down, float* ffn_out,
                          float* residual_out) {
  try {
    using u64 = std::uint64_t;
    const u64 h = H, i = I, is = IS, e = E;
    std::vector<F32Tensor> t = {
        {"blk.0.ffn_gate_up_exps.weight", {h, 2 * i, e}, gate_up, e * 2 * i * h},
        {"blk.0.ffn_down_exps.weight", {i, h, e}, down, e * h * i},
        {"blk.0.ffn_gate_shexp.weight", {h, is}, sh_gate_up, is * h},
        {"blk.0.ffn_up_shexp.weight", {h, is}, sh_gate_up + is * h, is * h},
        {"blk.0.ffn_down_shexp.weight", {is, h}, sh_down, h * is},
        {"blk.0.ffn_gate_inp.weight", {h, e}, router, e * h},
        {"blk.0.ffn_gate_inp_shexp.weight", {h}, sh_gate, h},
        {"blk.0.post_attention_norm.weight", {h}, norm_w, h},
    };
    write_gguf_f32(path, t);
    auto index = iq36::parse_gguf_model_index(path);
    auto r = iq36::run_qwen36_moe_ffn_layer(path, index, 0, vec(residual, H), eps);
    std::remove(path);
    copy_out(r.ffn_norm, ffn_norm);
    copy_out(r.router_logits, router_logits);
    if (ids) {
      std::memcpy(ids, r.router.expert_ids.data(),
                  r.router.expert_ids.size() * sizeof(std::int32_t));
    }
    copy_out(r.router.normalized_weights, normalized_weights);
    copy_out(r.selected_gate_up, selected_gate_up);
    copy_out(r.selected_swiglu, selected_swiglu);
    copy_out(r.selected_down, selected_down);
    copy_out(r.moe_out, moe_out);
    copy_out(r.shared_gate_sigmoid, shared_gate_sigmoid);
    copy_out(r.shared_down, shared_down);
    copy_out(r.ffn_out, ffn_out);
    copy_out(r.residual, residual_out);
    return 0;
  } catch (const std::exception& e) {
    std::remove(path);
    return fail(e);
  }
}

// Q4_K rows decoded by the reference: a GGUF file with one Q4_K tensor
// [rows][cols] (raw 144-byte super-blocks, row-major) read back row by row
// through decode_tensor_row (gguf_loader.cpp:3245), which decodes each block
// with decode_q4_k_block (gguf_loader.cpp:1011-1040).
int ref_decode_q4k_rows(const char* path, const std::uint8_t* blocks, std::int64_t rows,
                        std::int64_t cols, float* out) {
  try {
    F32Tensor t{"blk.0.ffn_down_exps.weight",
                {static_cast<std::uint64_t>(cols), static_cast<std::uint64_t>(rows)},
                nullptr, static_cast<std::uint64_t>(rows * cols)};
    t.type = 12;
    t.raw = blocks;
    t.raw_bytes = static_cast<std::uint64_t>(rows * (cols / 256) * 144);
    write_gguf_f32(path, {t});
    auto index = iq36::parse_gguf_model_index(path);
    for (std::int64_t r = 0; r < rows; ++r) {
      const auto v = iq36::decode_tensor_row(path, index, t.name, static_cast<std::uint64_t>(r));
      if (static_cast<std::int64_t>(v.size()) != cols) throw std::runtime_error("row size");
      std::memcpy(out + r * cols, v.data(), sizeof(float) * static_cast<std::size_t>(cols));
    }
    std::remove(path);
    return 0;
  } catch (const std::exception& e) {
    std::remove(path);
    return fail(e);
  }
}

}  // extern "C"
