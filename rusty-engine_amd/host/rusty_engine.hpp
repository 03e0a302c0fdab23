// C++ host-side mirror of rusty-engine's quantized-matrix interface, over librehip's C ABI.
//
// Callers written against the reference keep their shape:
//   QMat::from_bytes(ggml_type, bytes, m, n)   src/qmat.rs:52-59 (uploads and repacks once)
//   q.matvec(x) -> y[m]                        src/qmat.rs:80
//   q.matmul(x, rows) -> Y[rows x m]           src/qmat.rs:169
//   q.rows(), q.cols()                         src/qmat.rs:62-73
//   top_k / top_k_sigmoid / route / silu       src/moe.rs:44-125 (host router)
//   moe_layer_forward(..., shared)             src/moe.rs:360-388, experts on the GPU, optional shared expert
//   combine(routed, weights, shared)           src/moe.rs:306-345
//   MmapModel::open(path), header(), tensor_bytes(name)   src/loader.rs:25-130, src/gguf.rs:120-170
//   QMat::from_model(model, name, m, n)        src/qmat.rs:310-330 (bytes go to the GPU from the map)
//   Q8Activation::from_f32(x), q.matvec_i8 / matmul_i8   src/kernel.rs:70-166 (int8 activations)
// Failures surface as EngineError (src/core.rs:56-68) thrown with librehip's message; the
// reference panics on unknown types at call time, this layer throws at construction.
#pragma once

#include <algorithm>
#include <cmath>
#include <cstdint>
#include <memory>
#include <numeric>
#include <stdexcept>
#include <string>
#include <utility>
#include <vector>
#include <cfloat>
#include <optional>

#include "../../include/rehip.h"

namespace rusty_engine {

struct EngineError : std::runtime_error {
  int code;
  EngineError(int c, const std::string& m) : std::runtime_error(m), code(c) {}
};

inline void check(int rc) {
  if (rc != RE_OK) throw EngineError(rc, re_last_error());
}

enum class Precision { Bf16Mfma = RE_MODE_BF16, F32Strict = RE_MODE_F32 };

// ---- GGUF model files (src/gguf.rs, src/loader.rs) -----------------------------------------
// One row of the tensor-info table (gguf.rs TensorEntry).
struct TensorEntry {
  std::string name;
  std::vector<uint64_t> dims;
  uint32_t ggml_type = 0;
  uint64_t offset = 0;
  uint64_t numel() const {
    uint64_t n = 1;
    for (uint64_t d : dims) n *= d;
    return n;
  }
};

// The parsed header (GgufFile, gguf.rs:126-170): version, metadata accessors, tensor table.
class GgufHeader {
 public:
  explicit GgufHeader(const re_gguf* g) : g_(g) {
    const size_t nt = re_gguf_tensor_count(g);
    tensors.reserve(nt);
    for (size_t i = 0; i < nt; ++i) {
      const char* name = nullptr;
      uint32_t type = 0, nd = 0;
      uint64_t dims[8], off = 0;
      check(re_gguf_tensor_info(g, i, &name, &type, &nd, dims, &off));
      tensors.push_back(TensorEntry{name, std::vector<uint64_t>(dims, dims + nd), type, off});
    }
  }
  uint32_t version() const { return re_gguf_version(g_); }
  size_t n_kv() const { return re_gguf_kv_count(g_); }
  uint64_t alignment() const { return re_gguf_alignment(g_); }
  size_t data_offset() const { return re_gguf_data_offset(g_); }
  // metadata by key; EngineError when absent or of another kind
  int64_t get_int(const std::string& key) const {
    int64_t v = 0;
    check(re_gguf_get_int(g_, key.c_str(), &v));
    return v;
  }
  double get_float(const std::string& key) const {
    double v = 0;
    check(re_gguf_get_float(g_, key.c_str(), &v));
    return v;
  }
  std::string get_str(const std::string& key) const {
    const char* p = nullptr;
    size_t n = 0;
    check(re_gguf_get_str(g_, key.c_str(), &p, &n));
    return std::string(p, n);
  }
  std::vector<TensorEntry> tensors;

 private:
  const re_gguf* g_;
};

// A GGUF file mapped read-only (MmapModel, loader.rs:25-130). Tensor bytes are views into the
// mapping and stay valid while the model lives.
class MmapModel {
 public:
  static MmapModel open(const std::string& path) {
    re_gguf* g = nullptr;
    check(re_gguf_open(path.c_str(), &g));
    return MmapModel(g);
  }
  const GgufHeader& header() const { return *header_; }
  size_t data_start() const { return re_gguf_data_start(g_.get()); }
  // [data_start + offset, + nbytes) of a named tensor (loader.rs:95-101)
  std::pair<const uint8_t*, size_t> tensor_bytes(const std::string& name) const {
    size_t i = 0;
    check(re_gguf_find_tensor(g_.get(), name.c_str(), &i));
    const uint8_t* p = nullptr;
    size_t n = 0;
    check(re_gguf_tensor_data(g_.get(), i, &p, &n));
    return {p, n};
  }
  const re_gguf* raw() const { return g_.get(); }

 private:
  explicit MmapModel(re_gguf* g) : g_(g, re_gguf_close), header_(std::make_shared<GgufHeader>(g)) {}
  std::shared_ptr<re_gguf> g_;
  std::shared_ptr<GgufHeader> header_;
};

// ---- int8 activations (src/kernel.rs:70-166) ------------------------------------------------
// One activation row quantized per 32 values: f32 scale d = max|x| / 127 and i8 values
// round(x / d) (Q8Activation::from_f32, kernel.rs:88-105), computed on the GPU, bit-identical.
struct Q8Activation {
  std::vector<float> scales;
  std::vector<int8_t> qs;
  static Q8Activation from_f32(const std::vector<float>& x) {
    if (x.size() % 32) throw EngineError(RE_ERR_SIZE, "Q8Activation::from_f32: length must be a multiple of 32");
    Q8Activation a;
    a.scales.resize(x.size() / 32);
    a.qs.resize(x.size());
    if (!x.empty()) check(re_quantize_q8_act(x.data(), 1, x.size(), a.scales.data(), a.qs.data()));
    return a;
  }
  size_t blocks() const { return scales.size(); }
};

// A GPU-resident weight matrix W[m x n] (qmat.rs:30-42): quant blocks, or F32/F16/BF16 elements.
class QMat {
 public:
  // QMat::from_f32 (qmat.rs:45-49): a row-major f32 matrix; products in f32
  static QMat from_f32(const std::vector<float>& data, size_t m, size_t n) {
    if (data.size() != m * n) throw EngineError(RE_ERR_SIZE, "QMat::from_f32: shape mismatch");
    re_qmat* h = nullptr;
    check(re_qmat_create(0, reinterpret_cast<const uint8_t*>(data.data()), data.size() * sizeof(float), m, n, &h));
    return QMat(h);
  }

  // tensor `name` of a mapped model, dims [n, m]; EngineError when missing or out of bounds
  static QMat from_model(const MmapModel& model, const std::string& name, size_t m, size_t n) {
    re_qmat* h = nullptr;
    check(re_qmat_from_gguf(model.raw(), name.c_str(), m, n, &h));
    return QMat(h);
  }

  static QMat from_bytes(uint32_t ggml_type, const std::vector<uint8_t>& bytes, size_t m, size_t n) {
    re_qmat* h = nullptr;
    check(re_qmat_create(ggml_type, bytes.data(), bytes.size(), m, n, &h));
    return QMat(h);
  }

  size_t rows() const { return re_qmat_rows(h_.get()); }
  size_t cols() const { return re_qmat_cols(h_.get()); }
  uint32_t ggml_type() const { return re_qmat_type(h_.get()); }

  // W[m x n] * x[n] -> out[m]; f32 accumulation on the GPU
  std::vector<float> matvec(const std::vector<float>& x) const {
    if (x.size() != cols()) throw EngineError(RE_ERR_SIZE, "matvec: input width mismatch");
    std::vector<float> y(rows());
    check(re_qmat_matvec(h_.get(), x.data(), y.data()));
    return y;
  }

  // W[m x n] * X[rows x n] -> Out[rows x m] (row-major, out[row*m + r])
  std::vector<float> matmul(const std::vector<float>& x, size_t nrows,
                            Precision prec = Precision::Bf16Mfma) const {
    if (x.size() != nrows * cols()) throw EngineError(RE_ERR_SIZE, "matmul: X rows x n mismatch");
    std::vector<float> y(nrows * rows());
    check(re_qmat_matmul(h_.get(), x.data(), nrows, y.data(), static_cast<int>(prec)));
    return y;
  }

  // matvec_q8_0_i8 / matmul_q8_0_i8 (kernel.rs:145-166): Q8_0 weights times quantized rows,
  // bit-identical to the reference's integer dot
  std::vector<float> matvec_i8(const Q8Activation& x) const { return matmul_i8(std::vector<Q8Activation>{x}); }
  std::vector<float> matmul_i8(const std::vector<Q8Activation>& xs) const {
    const size_t n = cols(), nrows = xs.size();
    std::vector<float> sc, y(nrows * rows());
    std::vector<int8_t> qs;
    sc.reserve(nrows * n / 32);
    qs.reserve(nrows * n);
    for (const auto& a : xs) {
      if (a.qs.size() != n || a.scales.size() != n / 32)
        throw EngineError(RE_ERR_SIZE, "matmul_i8: activation length mismatch");
      sc.insert(sc.end(), a.scales.begin(), a.scales.end());
      qs.insert(qs.end(), a.qs.begin(), a.qs.end());
    }
    if (nrows) check(re_qmat_matmul_i8(h_.get(), sc.data(), qs.data(), nrows, y.data()));
    return y;
  }

  re_qmat* raw() const { return h_.get(); }

 private:
  explicit QMat(re_qmat* h) : h_(h, re_qmat_destroy) {}
  std::shared_ptr<re_qmat> h_;
};

// ---- router (src/moe.rs:11-125) -------------------------------------------------------------
struct ExpertScore {
  size_t id;
  float weight;
};

enum class Gate { Softmax, Sigmoid };

struct RouterConfig {
  Gate gate = Gate::Softmax;
  size_t top_k = 2;
};

inline float sigmoid(float x) { return 1.0f / (1.0f + std::exp(-x)); }
inline float silu(float x) { return x * sigmoid(x); }

inline void softmax_in_place(std::vector<float>& v) {
  float mx = -INFINITY;
  for (float a : v) mx = std::fmax(mx, a);
  for (float& a : v) a = std::exp(a - mx);
  float sum = -0.0f;
  for (float a : v) sum = sum + a;
  if (sum != 0.0f)
    for (float& a : v) a /= sum;
}

// indices by score, descending, ties in ascending index order (a stable sort)
inline std::vector<size_t> order_desc(const std::vector<float>& s) {
  std::vector<size_t> idx(s.size());
  std::iota(idx.begin(), idx.end(), 0);
  std::stable_sort(idx.begin(), idx.end(), [&](size_t a, size_t b) { return s[a] > s[b]; });
  return idx;
}

// keep the k best, weights = softmax over the chosen scores (moe.rs:75-93)
inline std::vector<ExpertScore> top_k(const std::vector<float>& scores, size_t k) {
  if (scores.empty()) return {};
  k = std::min(k, scores.size());
  const auto idx = order_desc(scores);
  std::vector<float> w(k);
  for (size_t i = 0; i < k; ++i) w[i] = scores[idx[i]];
  softmax_in_place(w);
  std::vector<ExpertScore> out(k);
  for (size_t i = 0; i < k; ++i) out[i] = {idx[i], w[i]};
  return out;
}

// per-expert sigmoid, keep k, renormalize over the chosen (moe.rs:97-117)
inline std::vector<ExpertScore> top_k_sigmoid(const std::vector<float>& scores, size_t k) {
  if (scores.empty()) return {};
  std::vector<float> sig(scores.size());
  for (size_t i = 0; i < scores.size(); ++i) sig[i] = sigmoid(scores[i]);
  k = std::min(k, sig.size());
  const auto idx = order_desc(sig);
  float wsum = -0.0f;
  for (size_t i = 0; i < k; ++i) wsum = wsum + sig[idx[i]];
  std::vector<ExpertScore> out(k);
  for (size_t i = 0; i < k; ++i) out[i] = {idx[i], wsum == 0.0f ? 0.0f : sig[idx[i]] / wsum};
  return out;
}

inline std::vector<ExpertScore> route(const std::vector<float>& logits, RouterConfig cfg) {
  return cfg.gate == Gate::Softmax ? top_k(logits, cfg.top_k) : top_k_sigmoid(logits, cfg.top_k);
}

// Bias-corrected group routing (moe.rs:126-268): scores sigmoid(logit + bias[i]) (missing bias
// entries count as 0), n_groups contiguous groups (group i * ng / n), only the top_k_group best
// groups eligible (nullopt: every group), the top_k best eligible experts renormalised over their
// scores. noaux_tc scores a group by its two best members, route_group by the sum of all.
inline std::vector<ExpertScore> route_groups(const std::vector<float>& logits, const std::vector<float>& bias,
                                             size_t n_groups, size_t top_k, std::optional<size_t> top_k_group,
                                             bool top2) {
  const size_t n = logits.size();
  if (n == 0) return {};
  std::vector<float> ex(n);
  for (size_t i = 0; i < n; ++i) ex[i] = sigmoid(logits[i] + (i < bias.size() ? bias[i] : 0.0f));
  const size_t ng = std::min(std::max<size_t>(n_groups, 1), n);
  std::vector<float> gscore(ng, 0.0f), t1(ng, -FLT_MAX), t2(ng, -FLT_MAX);
  for (size_t i = 0; i < n; ++i) {
    const size_t g = i * ng / n;
    if (!top2) {
      gscore[g] += ex[i];
    } else if (ex[i] >= t1[g]) {
      t2[g] = t1[g];
      t1[g] = ex[i];
    } else if (ex[i] > t2[g]) {
      t2[g] = ex[i];
    }
  }
  if (top2)
    for (size_t g = 0; g < ng; ++g) gscore[g] = t1[g] + (t2[g] == -FLT_MAX ? 0.0f : t2[g]);
  std::vector<bool> allowed(ng, !top_k_group.has_value());
  if (top_k_group) {
    const auto order = order_desc(gscore);
    for (size_t j = 0; j < std::min(*top_k_group, ng); ++j) allowed[order[j]] = true;
  }
  std::vector<size_t> cand;
  for (size_t i = 0; i < n; ++i)
    if (allowed[i * ng / n]) cand.push_back(i);
  std::stable_sort(cand.begin(), cand.end(), [&](size_t a, size_t b) { return ex[a] > ex[b]; });
  const size_t k = std::min(top_k, cand.size());
  float wsum = 0.0f;
  for (size_t j = 0; j < k; ++j) wsum += ex[cand[j]];
  std::vector<ExpertScore> out(k);
  for (size_t j = 0; j < k; ++j) out[j] = {cand[j], wsum == 0.0f ? 0.0f : ex[cand[j]] / wsum};
  return out;
}

inline std::vector<ExpertScore> route_group(const std::vector<float>& logits, const std::vector<float>& bias,
                                            size_t n_groups, size_t top_k, std::optional<size_t> top_k_group) {
  return route_groups(logits, bias, n_groups, top_k, top_k_group, false);
}

inline std::vector<ExpertScore> route_noaux_tc(const std::vector<float>& logits, const std::vector<float>& bias,
                                               size_t n_groups, size_t top_k, std::optional<size_t> top_k_group) {
  return route_groups(logits, bias, n_groups, top_k, top_k_group, true);
}

// ---- MoE experts on the GPU --------------------------------------------------------------------
// Expert tensors as GGUF stores them: gate/up [n_experts][inter][hidden], down
// [n_experts][hidden][inter], each row a run of blocks.
class MoeExperts {
 public:
  MoeExperts(uint32_t gate_t, const std::vector<uint8_t>& gate, uint32_t up_t, const std::vector<uint8_t>& up,
             uint32_t down_t, const std::vector<uint8_t>& down, size_t n_experts, size_t hidden, size_t inter)
      : n_experts_(n_experts), hidden_(hidden), inter_(inter) {
    re_moe* h = nullptr;
    check(re_moe_create(gate_t, gate.data(), gate.size(), up_t, up.data(), up.size(), down_t, down.data(),
                        down.size(), n_experts, hidden, inter, &h));
    h_.reset(h, re_moe_destroy);
  }

  size_t n_experts() const { return n_experts_; }
  size_t hidden() const { return hidden_; }
  size_t inter() const { return inter_; }
  bool has_shared() const { return has_shared_; }

  // The shared expert (moe.rs:380-385): a dense SwiGLU FFN (gate/up inter x hidden, down hidden x
  // inter) whose output every forward call adds after the routed sum, in the same GPU call.
  void set_shared(uint32_t gate_t, const std::vector<uint8_t>& gate, uint32_t up_t, const std::vector<uint8_t>& up,
                  uint32_t down_t, const std::vector<uint8_t>& down, size_t inter) {
    check(re_moe_set_shared(h_.get(), gate_t, gate.data(), gate.size(), up_t, up.data(), up.size(), down_t,
                            down.data(), down.size(), inter));
    has_shared_ = true;
  }
  void clear_shared() {
    check(re_moe_set_shared(h_.get(), 0, nullptr, 0, 0, nullptr, 0, 0, nullptr, 0, 0));
    has_shared_ = false;
  }

  // tokens x hidden activations, tokens x k routing -> tokens x hidden
  std::vector<float> forward(const std::vector<float>& x, size_t tokens, size_t k, const std::vector<uint32_t>& ids,
                             const std::vector<float>& weights, Precision prec = Precision::Bf16Mfma) const {
    if (x.size() != tokens * hidden_ || ids.size() != tokens * k || weights.size() != tokens * k)
      throw EngineError(RE_ERR_SIZE, "moe forward: shape mismatch");
    std::vector<float> out(tokens * hidden_);
    check(re_moe_forward(h_.get(), x.data(), tokens, k, ids.data(), weights.data(), out.data(),
                         static_cast<int>(prec)));
    return out;
  }

 private:
  std::shared_ptr<re_moe> h_;
  size_t n_experts_, hidden_, inter_;
  bool has_shared_ = false;
};

// One MoE FFN layer on `tokens` hidden vectors (moe.rs:360-388): router logits on the host
// (router_w is n_experts x hidden f32, `matvec` of moe.rs:271-277), route, then the routed
// experts' SwiGLU FFNs and the weighted combine in routing order on the GPU.
// combine (moe.rs:306-345): out = sum over k, in order, of routed[k] * weights[k], then + shared
// verbatim; the reference's shape errors
inline std::vector<float> combine(const std::vector<std::vector<float>>& routed, const std::vector<float>& weights,
                                  const std::vector<float>* shared = nullptr) {
  if (routed.size() != weights.size())
    throw EngineError(RE_ERR_SIZE, "combine: " + std::to_string(routed.size()) + " outputs vs " +
                                       std::to_string(weights.size()) + " weights");
  const size_t dim = !routed.empty() ? routed[0].size() : (shared ? shared->size() : 0);
  for (const auto& r : routed)
    if (r.size() != dim) throw EngineError(RE_ERR_SIZE, "combine: ragged routed outputs");
  if (shared && shared->size() != dim)
    throw EngineError(RE_ERR_SIZE,
                      "combine: shared dim " + std::to_string(shared->size()) + " != " + std::to_string(dim));
  std::vector<float> out(dim, 0.0f);
  for (size_t k = 0; k < routed.size(); ++k)
    for (size_t i = 0; i < dim; ++i) out[i] += routed[k][i] * weights[k];
  if (shared)
    for (size_t i = 0; i < dim; ++i) out[i] += (*shared)[i];
  return out;
}

// The shared expert (moe.rs:380-385) is either set on `experts` (MoeExperts::set_shared: added in
// the same GPU call) or passed as `shared`, a one-expert MoeExperts whose FFN output is added
// verbatim after the routed sum.
inline std::vector<float> moe_layer_forward(const std::vector<float>& hidden, size_t tokens,
                                            const std::vector<float>& router_w, const MoeExperts& experts,
                                            RouterConfig cfg, Precision prec = Precision::Bf16Mfma,
                                            const MoeExperts* shared = nullptr) {
  const size_t d = experts.hidden(), e = experts.n_experts();
  if (hidden.size() != tokens * d || router_w.size() != e * d)
    throw EngineError(RE_ERR_SIZE, "moe_layer_forward: shape mismatch");
  const size_t k = std::min(cfg.top_k, e);
  std::vector<uint32_t> ids(tokens * k);
  std::vector<float> w(tokens * k);
  std::vector<float> logits(e);
  for (size_t t = 0; t < tokens; ++t) {
    for (size_t r = 0; r < e; ++r) {
      float s = -0.0f;
      for (size_t c = 0; c < d; ++c) s = s + router_w[r * d + c] * hidden[t * d + c];
      logits[r] = s;
    }
    const auto chosen = route(logits, cfg);
    for (size_t j = 0; j < k; ++j) {
      ids[t * k + j] = static_cast<uint32_t>(chosen[j].id);
      w[t * k + j] = chosen[j].weight;
    }
  }
  std::vector<float> out = experts.forward(hidden, tokens, k, ids, w, prec);
  if (shared) {
    if (shared->n_experts() != 1 || shared->hidden() != d)
      throw EngineError(RE_ERR_SIZE, "moe_layer_forward: the shared expert must be one expert of the same width");
    // weight 1 through the routed combine gives the expert's output itself (0 + 1 * v)
    const std::vector<float> so =
        shared->forward(hidden, tokens, 1, std::vector<uint32_t>(tokens, 0), std::vector<float>(tokens, 1.0f), prec);
    for (size_t i = 0; i < out.size(); ++i) out[i] += so[i];
  }
  return out;
}

}  // namespace rusty_engine
