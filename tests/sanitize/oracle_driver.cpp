// Runs the CPU oracle (oracle/urb_oracle.cpp) over tiny layers of every composition and weight
// format, at two thread counts, plus its element and router entry points on edge inputs.
// Built with -fsanitize=address,undefined by tests/test_sanitizers.py; exits non-zero when the
// two thread counts disagree (the sanitizers abort on their own findings).
#include <cmath>
#include <cstdio>
#include <cstring>
#include <vector>

#include "../../oracle/urb_oracle.h"

static uint64_t rng_state = 0x9E3779B97F4A7C15ull;
static uint64_t next() {
  rng_state ^= rng_state << 13;
  rng_state ^= rng_state >> 7;
  rng_state ^= rng_state << 17;
  return rng_state;
}
static float normal() {
  double s = 0;
  for (int i = 0; i < 12; ++i) s += (next() >> 11) * (1.0 / 9007199254740992.0);
  return (float)(s - 6.0);
}
static uint16_t bf16(float v) {
  uint32_t b;
  std::memcpy(&b, &v, 4);
  return (uint16_t)((b + 0x7fff + ((b >> 16) & 1)) >> 16);
}

struct Mat {
  std::vector<uint8_t> data, scales;
};
static Mat make(int fmt, size_t rows, size_t cols, float sd) {
  Mat m;
  if (fmt == URBO_FMT_BF16) {
    m.data.resize(rows * cols * 2);
    for (size_t i = 0; i < rows * cols; ++i) {
      const uint16_t v = bf16(sd * normal());
      std::memcpy(&m.data[2 * i], &v, 2);
    }
    return m;
  }
  m.data.resize(fmt == URBO_FMT_MXFP4 ? rows * cols / 2 : rows * cols);
  for (auto& b : m.data) {
    b = (uint8_t)next();
    if (fmt == URBO_FMT_MXFP8 && (b & 0x7f) == 0x7f) b ^= 1;  // no E4M3 NaN
  }
  m.scales.resize(rows * cols / 32);
  for (auto& s : m.scales) s = (uint8_t)(119 + next() % 7);
  return m;
}

struct Layer {
  urbo_layer l{};
  std::vector<Mat> mats, shared;
  std::vector<urbo_matrix> em, sm;
  std::vector<uint16_t> router, gate;
  std::vector<float> bias;
  std::vector<int64_t> hash;
};

static void build(Layer& L, int comp, int fmt, int router, bool with_shared, bool hashed) {
  const uint32_t H = 64, E = 8, I = 32, K = 3;
  urbo_layer& l = L.l;
  l.hidden = H;
  l.n_experts = E;
  l.top_k = K;
  l.intermediate = I;
  l.shared_intermediate = with_shared ? I : 0;
  l.expert_format = fmt;
  l.shared_format = comp == URBO_COMPOSE_QWEN36 || comp == URBO_COMPOSE_GLM ? URBO_FMT_BF16 : fmt;
  l.router = router;
  l.composition = comp;
  l.n_group = router == URBO_ROUTER_SIGMOID_NOAUX_TC ? 2 : 1;
  l.topk_group = router == URBO_ROUTER_SIGMOID_NOAUX_TC ? 2 : 1;
  l.normalize = 1;
  l.routed_scaling_factor = 1.5f;
  l.swiglu_limit = 7.0f;
  L.router.resize(E * H);
  for (auto& r : L.router) r = bf16(0.1f * normal());
  l.router_weight = L.router.data();
  L.bias.resize(E);
  for (auto& b : L.bias) b = 0.01f * normal();
  l.correction_bias = router == URBO_ROUTER_SOFTMAX_TOPK ? nullptr : L.bias.data();
  const size_t dims[3][2] = {{I, H}, {I, H}, {H, I}};
  for (uint32_t e = 0; e < E; ++e)
    for (int m = 0; m < 3; ++m) L.mats.push_back(make(fmt, dims[m][0], dims[m][1], 0.05f));
  for (auto& m : L.mats) L.em.push_back({m.data.data(), m.scales.empty() ? nullptr : m.scales.data()});
  l.experts = L.em.data();
  if (with_shared) {
    for (int m = 0; m < 3; ++m) L.shared.push_back(make(l.shared_format, dims[m][0], dims[m][1], 0.05f));
    for (auto& m : L.shared)
      L.sm.push_back({m.data.data(), m.scales.empty() ? nullptr : m.scales.data()});
    l.shared = L.sm.data();
    if (comp == URBO_COMPOSE_QWEN36) {
      L.gate.resize(H);
      for (auto& g : L.gate) g = bf16(0.1f * normal());
      l.shared_expert_gate = L.gate.data();
    }
  }
  if (hashed) {
    const uint32_t vocab = 11;
    for (uint32_t v = 0; v < vocab; ++v)
      for (uint32_t j = 0; j < K; ++j) L.hash.push_back((v + 3 * j) % E);
    l.hash_experts = L.hash.data();
    l.hash_vocab = vocab;
  }
}

static int run(int comp, int fmt, int router, bool with_shared, bool hashed) {
  Layer L;
  build(L, comp, fmt, router, with_shared, hashed);
  const uint32_t T = 5, H = L.l.hidden, E = L.l.n_experts, K = L.l.top_k;
  std::vector<float> x(T * H);
  for (auto& v : x) v = normal();
  std::vector<uint32_t> tok(T);
  for (uint32_t t = 0; t < T; ++t) tok[t] = (7 * t) % 11;
  std::vector<float> y1(T * H), y2(T * H), w1(T * K), w2(T * K), g1(T * E), g2(T * E);
  std::vector<int32_t> i1(T * K), i2(T * K);
  int s1, s2;
  if (hashed) {
    s1 = urbo_moe_forward_tokens(&L.l, x.data(), tok.data(), T, y1.data(), i1.data(), w1.data(),
                                 g1.data(), 1);
    s2 = urbo_moe_forward_tokens(&L.l, x.data(), tok.data(), T, y2.data(), i2.data(), w2.data(),
                                 g2.data(), 3);
    tok[2] = 99;  // beyond the table: an error, not an out-of-bounds read
    if (urbo_moe_forward_tokens(&L.l, x.data(), tok.data(), T, y2.data(), i2.data(), w2.data(),
                                nullptr, 2) == URBO_OK)
      return 1;
  } else {
    s1 = urbo_moe_forward(&L.l, x.data(), T, y1.data(), i1.data(), w1.data(), g1.data(), 1);
    s2 = urbo_moe_forward(&L.l, x.data(), T, y2.data(), i2.data(), w2.data(), g2.data(), 3);
  }
  if (s1 != s2) return 1;
  if (s1 == URBO_OK && (std::memcmp(y1.data(), y2.data(), y1.size() * 4) ||
                        std::memcmp(i1.data(), i2.data(), i1.size() * 4)))
    return 1;
  std::printf("comp %d fmt %d router %d shared %d hash %d: status %d\n", comp, fmt, router,
              (int)with_shared, (int)hashed, s1);
  return 0;
}

int main() {
  int bad = 0;
  bad |= run(URBO_COMPOSE_QWEN36, URBO_FMT_BF16, URBO_ROUTER_SOFTMAX_TOPK, false, false);
  bad |= run(URBO_COMPOSE_QWEN36, URBO_FMT_BF16, URBO_ROUTER_SOFTMAX_TOPK, true, false);
  for (int fmt : {URBO_FMT_BF16, URBO_FMT_MXFP4, URBO_FMT_MXFP8})
    for (int router : {URBO_ROUTER_SOFTMAX_TOPK, URBO_ROUTER_SIGMOID_NOAUX_TC})
      bad |= run(URBO_COMPOSE_GLM, fmt, router, fmt != URBO_FMT_MXFP8, false);
  for (int comp : {URBO_COMPOSE_HY4, URBO_COMPOSE_DSV41, URBO_COMPOSE_DSV4})
    for (int fmt : {URBO_FMT_MXFP4, URBO_FMT_MXFP8})
      bad |= run(comp, fmt, comp == URBO_COMPOSE_HY4 ? URBO_ROUTER_SOFTMAX_TOPK
                                                    : URBO_ROUTER_SQRT_SOFTPLUS, true, false);
  bad |= run(URBO_COMPOSE_DSV4, URBO_FMT_MXFP4, URBO_ROUTER_SQRT_SOFTPLUS, true, true);
  // element and router entry points on edge inputs
  std::vector<float> v = {0.0f, -0.0f, 1e-30f, 3.0e38f, 448.0f, 449.0f, -1e-6f, 5.0f};
  for (size_t i = 0; i < 32; ++i) v.push_back(0.001f * (float)i);
  bad |= urbo_simulate_e4m3_activation(v.data(), 32, 32) != URBO_OK;
  float o;
  for (uint32_t code = 0; code < 256; ++code) {
    (void)urbo_decode_e8m0((uint8_t)code, &o);
    (void)urbo_decode_e4m3fn((uint8_t)code);
    (void)urbo_decode_e2m1((uint8_t)(code & 15));
  }
  std::vector<float> logits = {0.5f, 0.5f, -1.0f, 2.0f, NAN, 0.0f};
  int32_t ids[3];
  float w[3], sel[3];
  bad |= urbo_route_softmax_top_k(logits.data(), 6, 3, ids, w) == URBO_OK;  // NaN: an error
  logits[4] = 1.0f;
  bad |= urbo_route_softmax_top_k(logits.data(), 6, 3, ids, w) != URBO_OK;
  bad |= urbo_route_noaux_tc(logits.data(), nullptr, 6, 3, 2, 1, 1, 1.0f, ids, w, sel) !=
         URBO_OK;
  bad |= urbo_route_noaux_tc(logits.data(), nullptr, 6, 3, 4, 1, 1, 1.0f, ids, w, sel) ==
         URBO_OK;  // 6 experts do not split into 4 groups
  if (bad) {
    std::fprintf(stderr, "oracle driver: a check failed\n");
    return 1;
  }
  std::printf("oracle driver ok\n");
  return 0;
}
