// C++ parity tests of the host-side mirror (rusty_engine.hpp) on the GPU, written like the
// reference's own unit tests (src/qmat.rs:333-399, src/kernel.rs:2080-2584, src/moe.rs:624-801,
// src/gguf.rs:1063-1312).
// The CPU oracle (oracle/oracle.h) is the checker. Exit status 0 = all passed.
#include <cmath>
#include <cstdio>
#include <cstring>
#include <random>
#include <vector>

#include "../../oracle/oracle.h"
#include "../../rusty-engine_amd/host/rusty_engine.hpp"

using namespace rusty_engine;

static int g_failed = 0;
#define CHECK(cond, ...)                                   \
  do {                                                     \
    if (!(cond)) {                                         \
      std::printf("  FAIL %s:%d: ", __FILE__, __LINE__);   \
      std::printf(__VA_ARGS__);                            \
      std::printf("\n");                                   \
      ++g_failed;                                          \
    }                                                      \
  } while (0)

// qmat.rs:370-381 fixture: Q8_0 blocks, d = 1, i8 ((bi*31 + j*7) % 251) - 125
static std::vector<uint8_t> q8_blocks(size_t m, size_t n) {
  std::vector<uint8_t> a(m * n / 32 * 34);
  for (size_t bi = 0; bi < m * n / 32; ++bi) {
    a[bi * 34] = 0x00;
    a[bi * 34 + 1] = 0x3C;
    for (int j = 0; j < 32; ++j) a[bi * 34 + 2 + j] = (uint8_t)(int8_t)(((bi * 31 + j * 7) % 251) - 125);
  }
  return a;
}

static std::vector<uint8_t> random_blocks(std::mt19937& g, uint32_t t, size_t m, size_t n) {
  size_t qk = 0, bb = 0;
  orc_block_info(t, &qk, &bb);
  const size_t nb = m * ((n + qk - 1) / qk);
  std::vector<uint8_t> a(nb * bb);
  for (auto& v : a) v = (uint8_t)(g() & 0xFF);
  std::normal_distribution<float> nd(0.f, 1.f);
  for (size_t b = 0; b < nb; ++b) {
    uint8_t* blk = &a[b * bb];
    const uint16_t d = orc_f32_to_f16(std::fabs(nd(g)) * (qk == 32 ? 0.01f : 0.001f));
    const size_t off = t == ORC_Q6_K ? 208 : 0;
    blk[off] = d & 0xFF;
    blk[off + 1] = d >> 8;
    if (t == ORC_Q4_K || t == ORC_Q5_K) { blk[2] = d & 0xFF; blk[3] = d >> 8; }
  }
  return a;
}

static std::vector<float> randn(std::mt19937& g, size_t n) {
  std::normal_distribution<float> nd(0.f, 1.f);
  std::vector<float> v(n);
  for (auto& x : v) x = nd(g);
  return v;
}

// |got - want| <= 2^-10 * sum|w x| per output
static bool within_f32_bound(uint32_t t, const std::vector<uint8_t>& w, size_t m, size_t n,
                             const std::vector<float>& x, size_t rows, const std::vector<float>& got,
                             const std::vector<float>& want) {
  std::vector<double> absd(rows * m);
  orc_qmat_absdot(t, w.data(), w.size(), m, n, x.data(), rows, absd.data());
  for (size_t i = 0; i < rows * m; ++i)
    if (std::fabs((double)got[i] - (double)want[i]) > std::ldexp(absd[i], -10)) return false;
  return true;
}

static void test_matmul_matches_rowwise_matvec() {  // qmat.rs:357-367
  std::printf("matmul_matches_rowwise_matvec\n");
  const size_t m = 64, n = 4096, rows = 8;
  const auto w = q8_blocks(m, n);
  const auto q = QMat::from_bytes(ORC_Q8_0, w, m, n);
  CHECK(q.rows() == m && q.cols() == n, "rows/cols");
  std::vector<float> x(rows * n);
  for (size_t i = 0; i < x.size(); ++i) x[i] = (float)i * 0.0007f - 1.5f;
  const auto got = q.matmul(x, rows, Precision::F32Strict);
  std::vector<float> rowwise;
  for (size_t r = 0; r < rows; ++r) {
    const auto y = q.matvec(std::vector<float>(x.begin() + r * n, x.begin() + (r + 1) * n));
    rowwise.insert(rowwise.end(), y.begin(), y.end());
  }
  CHECK(within_f32_bound(ORC_Q8_0, w, m, n, x, rows, got, rowwise), "matmul vs rowwise matvec");
}

static void test_matvec_is_deterministic() {  // qmat.rs:385-391 (bit-identical whatever the split)
  std::printf("matvec_is_deterministic_and_matches_serial_oracle\n");
  const size_t m = 64, n = 4096;
  const auto w = q8_blocks(m, n);
  const auto q = QMat::from_bytes(ORC_Q8_0, w, m, n);
  std::vector<float> x(n);
  for (size_t i = 0; i < n; ++i) x[i] = (float)i * 0.001f - 2.0f;
  const auto a = q.matvec(x), b = q.matvec(x);
  CHECK(std::memcmp(a.data(), b.data(), a.size() * 4) == 0, "two calls differ");
  std::vector<float> want(m);
  orc_matvec(ORC_Q8_0, w.data(), m, n, x.data(), want.data());
  CHECK(within_f32_bound(ORC_Q8_0, w, m, n, x, 1, a, want), "matvec vs oracle");
}

static void test_every_type_against_oracle() {
  std::printf("qmat_every_type_matvec_and_matmul_against_oracle\n");
  std::mt19937 g(42);
  const uint32_t types[] = {ORC_Q4_0, ORC_Q5_0, ORC_Q8_0, ORC_Q4_K, ORC_Q5_K, ORC_Q6_K};
  for (uint32_t t : types) {
    const size_t m = 200, n = 896, rows = 37;
    const auto w = random_blocks(g, t, m, n);
    const auto x = randn(g, rows * n);
    const auto q = QMat::from_bytes(t, w, m, n);
    std::vector<float> want(rows * m);
    orc_qmat_matmul(t, w.data(), w.size(), m, n, x.data(), rows, want.data());
    const auto got32 = q.matmul(x, rows, Precision::F32Strict);
    CHECK(within_f32_bound(t, w, m, n, x, rows, got32, want), "type %u f32 matmul", t);
    const auto got16 = q.matmul(x, rows, Precision::Bf16Mfma);
    double num = 0, den = 0;
    for (size_t i = 0; i < want.size(); ++i) {
      num += ((double)got16[i] - want[i]) * ((double)got16[i] - want[i]);
      den += (double)want[i] * want[i];
    }
    CHECK(std::sqrt(num / den) <= 1e-2, "type %u bf16 matmul rel %g", t, std::sqrt(num / den));
    const auto y = q.matvec(std::vector<float>(x.begin(), x.begin() + n));
    CHECK(within_f32_bound(t, w, m, n, std::vector<float>(x.begin(), x.begin() + n), 1, y,
                           std::vector<float>(want.begin(), want.begin() + m)),
          "type %u matvec", t);
  }
}

static void test_from_f32_matches_plain_matvec() {  // qmat.rs:337-345
  std::printf("from_f32_matches_plain_matvec\n");
  std::vector<float> data(12);
  for (int i = 0; i < 12; ++i) data[i] = (float)i * 0.25f - 1.0f;
  const QMat qm = QMat::from_f32(data, 3, 4);
  const std::vector<float> x = {1.0f, -2.0f, 0.5f, 3.0f};
  std::vector<float> want(3);
  for (int r = 0; r < 3; ++r) {           // moe::matvec: sequential sum from -0.0 (moe.rs:271-277)
    float acc = -0.0f;
    for (int k = 0; k < 4; ++k) acc += data[r * 4 + k] * x[k];
    want[r] = acc;
  }
  CHECK(qm.matvec(x) == want, "f32 weights: exact sums match the plain matvec");
  CHECK(qm.rows() == 3 && qm.cols() == 4 && qm.ggml_type() == 0, "shape and type");
}

static void test_unknown_type_is_an_error() {  // kernel.rs:2006, 2027 panic -> EngineError
  std::printf("unknown_type_is_an_error\n");
  bool threw = false;
  try {
    (void)QMat::from_bytes(99, std::vector<uint8_t>(34), 1, 32);
  } catch (const EngineError& e) {
    threw = e.code == RE_ERR_TYPE;
  }
  CHECK(threw, "no EngineError for type 99");
}

static void test_group_routers_match_oracle() {  // moe.rs:675-720, then random logits vs the oracle
  std::printf("group_routers_match_oracle\n");
  const std::vector<float> l8 = {5.0f, 2.0f, -9.0f, -9.0f, 0.0f, 0.0f, 0.0f, 0.0f};
  CHECK(route_noaux_tc(l8, {}, 2, 1, 1)[0].id == 0, "noaux_tc picks the dominant pair");
  const auto lite = route_group(l8, {}, 2, 1, 1);
  CHECK(lite[0].id >= 4 && lite[0].id <= 7, "route_group picks the larger sum");
  CHECK(route_noaux_tc({}, {}, 2, 1, 1).empty(), "empty input");
  std::mt19937 rng(91);
  std::normal_distribution<float> nd;
  for (int trial = 0; trial < 50; ++trial) {
    std::vector<float> logits(128), bias(100);
    for (auto& v : logits) v = std::round(nd(rng) * 2.0f) / 2.0f;
    for (auto& v : bias) v = nd(rng) * 0.25f;
    for (int top2 = 0; top2 < 2; ++top2) {
      const auto mine = top2 ? route_noaux_tc(logits, bias, 8, 8, 4) : route_group(logits, bias, 8, 8, 4);
      uint32_t ids[8];
      float w[8];
      const size_t n = (top2 ? orc_route_noaux_tc : orc_route_group)(logits.data(), logits.size(), bias.data(),
                                                                     bias.size(), 8, 8, 4, ids, w);
      CHECK(n == mine.size(), "group route count");
      for (size_t j = 0; j < n; ++j) CHECK(mine[j].id == ids[j] && mine[j].weight == w[j], "group route vs oracle");
    }
  }
}

static void test_router_matches_oracle() {  // moe.rs:631-662
  std::printf("router_top_k_matches_oracle\n");
  auto s = top_k({0.1f, 0.9f, 0.2f, 0.8f}, 2);
  CHECK(s.size() == 2 && s[0].id == 1 && s[1].id == 3, "top_k ids");
  CHECK(std::fabs(s[0].weight + s[1].weight - 1.0f) < 1e-5f, "top_k weights sum");
  CHECK(top_k({0.5f, 0.4f}, 8).size() == 2, "clamp k");
  auto sg = top_k_sigmoid({1.0f, 5.0f, 2.0f, 4.0f}, 2);
  CHECK(sg[0].id == 1 && sg[1].id == 3, "top_k_sigmoid ids");
  std::mt19937 g(5);
  for (int rep = 0; rep < 50; ++rep) {
    const auto logits = randn(g, 128);
    const auto mine = top_k(logits, 8);
    uint32_t ids[8];
    float w[8];
    orc_top_k(logits.data(), logits.size(), 8, ids, w);
    for (int j = 0; j < 8; ++j)
      CHECK(mine[j].id == ids[j] && mine[j].weight == w[j], "router differs at %d", j);
  }
}

// 32 x 32 Q8_0 matrix, d = 1, quant `q` on the diagonal
static std::vector<uint8_t> q8_identity(int q) {
  std::vector<uint8_t> a(32 * 34, 0);
  for (int r = 0; r < 32; ++r) {
    a[r * 34] = 0x00;
    a[r * 34 + 1] = 0x3C;
    a[r * 34 + 2 + r] = (uint8_t)(int8_t)q;
  }
  return a;
}

static void test_moe_layer_routes_to_best_expert() {  // moe.rs:784-796
  std::printf("moe_layer_routes_to_best_expert\n");
  auto ident = q8_identity(1), dbl = q8_identity(2);
  std::vector<uint8_t> gate = ident, down = ident;
  gate.insert(gate.end(), ident.begin(), ident.end());
  down.insert(down.end(), dbl.begin(), dbl.end());
  MoeExperts ex(ORC_Q8_0, gate, ORC_Q8_0, gate, ORC_Q8_0, down, 2, 32, 32);
  std::vector<float> router_w(2 * 32, 0.0f);
  router_w[32] = 10.0f;  // expert 1 scores 10 on hidden[0]
  std::vector<float> h(32, 0.0f);
  h[0] = 1.0f;
  for (Precision p : {Precision::F32Strict, Precision::Bf16Mfma}) {
    const auto out = moe_layer_forward(h, 1, router_w, ex, RouterConfig{Gate::Softmax, 1}, p);
    CHECK(std::fabs(out[0] - 2.0f * silu(1.0f)) < 1e-2f, "out[0] = %g", out[0]);
    float rest = 0;
    for (int i = 1; i < 32; ++i) rest += std::fabs(out[i]);
    CHECK(rest < 1e-5f, "off-diagonal %g", rest);
  }
}

static void test_moe_layer_adds_shared_expert() {  // moe.rs:788-801
  std::printf("moe_layer_adds_shared_expert\n");
  auto ident = q8_identity(1);
  std::vector<uint8_t> two = ident;
  two.insert(two.end(), ident.begin(), ident.end());
  MoeExperts ex(ORC_Q8_0, two, ORC_Q8_0, two, ORC_Q8_0, two, 2, 32, 32);
  MoeExperts shared(ORC_Q8_0, ident, ORC_Q8_0, ident, ORC_Q8_0, ident, 1, 32, 32);
  std::vector<float> router_w(2 * 32, 0.0f);
  router_w[0] = 10.0f;  // expert 0 wins (sigmoid, top-1: weight 1)
  std::vector<float> h(32, 0.0f);
  h[0] = 1.0f;
  for (Precision p : {Precision::F32Strict, Precision::Bf16Mfma}) {
    const auto out = moe_layer_forward(h, 1, router_w, ex, RouterConfig{Gate::Sigmoid, 1}, p, &shared);
    CHECK(std::fabs(out[0] - 2.0f * silu(1.0f)) < 1e-2f, "out[0] = %g", out[0]);
    float rest = 0;
    for (int i = 1; i < 32; ++i) rest += std::fabs(out[i]);
    CHECK(rest < 1e-5f, "off-diagonal %g", rest);
  }
  // the same shared expert set on the experts: added inside the GPU call, same values
  ex.set_shared(ORC_Q8_0, ident, ORC_Q8_0, ident, ORC_Q8_0, ident, 32);
  for (Precision p : {Precision::F32Strict, Precision::Bf16Mfma}) {
    const auto a = moe_layer_forward(h, 1, router_w, ex, RouterConfig{Gate::Sigmoid, 1}, p);
    CHECK(std::fabs(a[0] - 2.0f * silu(1.0f)) < 1e-2f, "set_shared out[0] = %g", a[0]);
    float rest = 0;
    for (int i = 1; i < 32; ++i) rest += std::fabs(a[i]);
    CHECK(rest < 1e-5f, "set_shared off-diagonal %g", rest);
  }
  ex.clear_shared();
  const auto none = moe_layer_forward(h, 1, router_w, ex, RouterConfig{Gate::Sigmoid, 1}, Precision::F32Strict);
  CHECK(std::fabs(none[0] - silu(1.0f)) < 1e-5f, "cleared shared: out[0] = %g", none[0]);
}

static void test_combine_routed_plus_shared() {  // moe.rs:749-765
  std::printf("combine_routed_plus_shared\n");
  const std::vector<std::vector<float>> routed = {{1.0f, 2.0f}, {3.0f, 4.0f}};
  const std::vector<float> w = {0.5f, 0.5f}, sh = {1.0f, 1.0f};
  CHECK(combine(routed, w, &sh) == std::vector<float>({3.0f, 4.0f}), "0.5*[1,2] + 0.5*[3,4] + [1,1]");
  CHECK(combine(routed, w) == std::vector<float>({2.0f, 3.0f}), "no shared expert");
  bool threw = false;
  try { (void)combine({{1.0f, 2.0f}}, {0.5f, 0.5f}); } catch (const EngineError& e) {
    threw = std::string(e.what()) == "combine: 1 outputs vs 2 weights";
  }
  CHECK(threw, "outputs vs weights count");
  threw = false;
  try { (void)combine({{1.0f}, {2.0f, 3.0f}}, {0.5f, 0.5f}); } catch (const EngineError& e) {
    threw = std::string(e.what()) == "combine: ragged routed outputs";
  }
  CHECK(threw, "ragged outputs");
}

// ---- GGUF (gguf.rs:1063-1312, loader.rs:245-270) --------------------------------------------
static void put_u32(std::vector<uint8_t>& b, uint32_t v) { for (int i = 0; i < 4; ++i) b.push_back((v >> (8 * i)) & 0xFF); }
static void put_u64(std::vector<uint8_t>& b, uint64_t v) { for (int i = 0; i < 8; ++i) b.push_back((v >> (8 * i)) & 0xFF); }
static void put_str(std::vector<uint8_t>& b, const std::string& s) {
  put_u64(b, s.size());
  b.insert(b.end(), s.begin(), s.end());
}

static std::string write_file(const std::string& name, const std::vector<uint8_t>& bytes) {
  const std::string path = std::string("/tmp/") + name;
  FILE* f = std::fopen(path.c_str(), "wb");
  std::fwrite(bytes.data(), 1, bytes.size(), f);
  std::fclose(f);
  return path;
}

static void test_gguf_header_fixture() {  // gguf.rs:1085-1145, synth_gguf
  std::printf("gguf_parses_header_kv_and_tensor_info\n");
  std::vector<uint8_t> b = {'G', 'G', 'U', 'F'};
  put_u32(b, 3);
  put_u64(b, 1);
  put_u64(b, 3);
  put_str(b, "general.architecture");
  put_u32(b, 8);
  put_str(b, "qwen2moe");
  put_str(b, "general.block_count");
  put_u32(b, 4);
  put_u32(b, 48);
  put_str(b, "tokenizer.ggml.tokens");
  put_u32(b, 9);
  put_u32(b, 8);
  put_u64(b, 2);
  put_str(b, "a");
  put_str(b, "b");
  put_str(b, "blk.0.ffn_gate_exps.weight");
  put_u32(b, 3);
  put_u64(b, 2048);
  put_u64(b, 512);
  put_u64(b, 64);
  put_u32(b, 12);
  put_u64(b, 0);
  const auto m = MmapModel::open(write_file("re_fixture.gguf", b));
  const auto& h = m.header();
  CHECK(h.version() == 3 && h.tensors.size() == 1 && h.n_kv() == 3, "counts");
  CHECK(h.data_offset() == b.size(), "data offset %zu", h.data_offset());
  CHECK(h.get_str("general.architecture") == "qwen2moe", "architecture");
  CHECK(h.get_int("general.block_count") == 48, "block count");
  CHECK(h.alignment() == 32, "default alignment");
  const auto& t = h.tensors[0];
  CHECK(t.name == "blk.0.ffn_gate_exps.weight" && t.dims == std::vector<uint64_t>({2048, 512, 64}) &&
            t.ggml_type == 12 && t.offset == 0,
        "tensor entry");
  bool threw = false;
  try {
    m.tensor_bytes("blk.0.ffn_gate_exps.weight");     // header only: the bytes are past the end
  } catch (const EngineError& e) {
    threw = e.code == RE_ERR_SIZE;
  }
  CHECK(threw, "tensor bytes out of bounds");
  std::vector<uint8_t> bad = b;
  bad[4] = 1;                                            // version 1
  threw = false;
  try {
    MmapModel::open(write_file("re_bad.gguf", bad));
  } catch (const EngineError& e) {
    threw = std::string(e.what()).find("unsupported GGUF version 1") != std::string::npos;
  }
  CHECK(threw, "version 1 rejected");
}

static void test_qmat_from_model_equals_from_bytes() {  // qmat.rs:310-330
  std::printf("qmat_from_model_equals_from_bytes\n");
  std::mt19937 g(5);
  const size_t m = 200, n = 512;
  const auto w = random_blocks(g, ORC_Q4_K, m, n);
  std::vector<uint8_t> b = {'G', 'G', 'U', 'F'};
  put_u32(b, 3);
  put_u64(b, 1);
  put_u64(b, 0);
  put_str(b, "blk.0.ffn_up.weight");
  put_u32(b, 2);
  put_u64(b, n);
  put_u64(b, m);
  put_u32(b, ORC_Q4_K);
  put_u64(b, 0);
  while (b.size() % 32) b.push_back(0);
  b.insert(b.end(), w.begin(), w.end());
  const auto model = MmapModel::open(write_file("re_model.gguf", b));
  const auto bytes = model.tensor_bytes("blk.0.ffn_up.weight");
  CHECK(bytes.second == w.size() && std::memcmp(bytes.first, w.data(), w.size()) == 0, "mapped bytes");
  const QMat a = QMat::from_model(model, "blk.0.ffn_up.weight", m, n), c = QMat::from_bytes(ORC_Q4_K, w, m, n);
  const auto x = randn(g, n);
  CHECK(a.matvec(x) == c.matvec(x), "from_model and from_bytes give the same bits");
  bool threw = false;
  try {
    QMat::from_model(model, "nope", m, n);
  } catch (const EngineError& e) {
    threw = std::string(e.what()) == "QMat: tensor 'nope' missing";
  }
  CHECK(threw, "missing tensor message");
}

// ---- int8 activations (kernel.rs:2210-2326) ---------------------------------------------------
static void test_q8_activation_and_i8_matmul() {
  std::printf("q8_activation_and_i8_matmul_match_oracle\n");
  std::mt19937 g(9);
  const size_t m = 300, n = 1024, rows = 3;
  const auto w = random_blocks(g, ORC_Q8_0, m, n);
  const QMat q = QMat::from_bytes(ORC_Q8_0, w, m, n);
  std::vector<Q8Activation> xs;
  for (size_t r = 0; r < rows; ++r) {
    auto x = randn(g, n);
    for (size_t i = 0; i < n; ++i) x[i] *= (float)(r + 1) * 3.0f;
    const Q8Activation a = Q8Activation::from_f32(x);
    std::vector<float> sc(n / 32);
    std::vector<int8_t> qs(n);
    orc_quantize_q8_act(x.data(), n, sc.data(), qs.data());
    CHECK(std::memcmp(sc.data(), a.scales.data(), sc.size() * 4) == 0 && qs == a.qs, "quantize row %zu", r);
    xs.push_back(a);
  }
  const auto y = q.matmul_i8(xs);
  for (size_t r = 0; r < rows; ++r) {
    std::vector<float> want(m);
    orc_matmul_q8_0_i8(w.data(), m, n, xs[r].scales.data(), xs[r].qs.data(), 1, want.data());
    CHECK(std::memcmp(want.data(), y.data() + r * m, m * 4) == 0, "i8 matmul row %zu bit-identical", r);
  }
  CHECK(q.matvec_i8(xs[1]) == std::vector<float>(y.begin() + m, y.begin() + 2 * m), "matvec_i8 == matmul_i8 row");
}

int main() {
  try {
    check(re_init());
    test_unknown_type_is_an_error();
    test_matmul_matches_rowwise_matvec();
    test_matvec_is_deterministic();
    test_every_type_against_oracle();
    test_group_routers_match_oracle();
    test_router_matches_oracle();
    test_moe_layer_routes_to_best_expert();
    test_moe_layer_adds_shared_expert();
    test_combine_routed_plus_shared();
    test_gguf_header_fixture();
    test_qmat_from_model_equals_from_bytes();
    test_from_f32_matches_plain_matvec();
    test_q8_activation_and_i8_matmul();
  } catch (const EngineError& e) {
    std::printf("EngineError %d: %s\n", e.code, e.what());
    return 2;
  }
  std::printf(g_failed ? "FAILED (%d)\n" : "ALL PASSED\n", g_failed);
  return g_failed ? 1 : 0;
}
