// Exercises every entry point of the residency policy (urbilateria_amd/csrc/urb_residency.cpp)
// on a deterministic pseudo-random schedule, including out-of-range layers, NULL arguments,
// failing loads and the clock corner of finish_grouped_accesses.  Built with
// -fsanitize=address,undefined by tests/test_sanitizers.py; exits non-zero on a broken
// invariant (the sanitizers abort on their own findings).
#include <algorithm>
#include <cstdio>
#include <cstdlib>
#include <set>
#include <vector>

#include "../../include/urb_residency.h"

static uint64_t rng_state = 0x243F6A8885A308D3ull;
static uint64_t next() {
  rng_state ^= rng_state << 13;
  rng_state ^= rng_state >> 7;
  rng_state ^= rng_state << 17;
  return rng_state;
}

static int fail_every = 0;
static uint64_t loads = 0;
static int load(void*, uint32_t, uint64_t key, uint64_t* value, uint64_t* bytes, uint64_t* read) {
  ++loads;
  if (fail_every && loads % fail_every == 0) return 9;
  *value = key * 16 + 1;
  *bytes = 100 + key;
  *read = 100 + key;
  return 0;
}

#define CHECK(c)                                                   \
  do {                                                             \
    if (!(c)) {                                                    \
      std::fprintf(stderr, "check failed line %d: %s\n", __LINE__, #c); \
      return 1;                                                    \
    }                                                              \
  } while (0)

static int check_layer(urb_lru* c, uint32_t layer) {
  std::vector<uint64_t> k(64), u(64), v(64);
  const size_t n = urb_lru_entries(c, layer, k.data(), u.data(), v.data());
  CHECK(n <= urb_lru_layer_capacity(c, layer));
  std::set<uint64_t> keys(k.begin(), k.begin() + n);
  CHECK(keys.size() == n);
  for (size_t i = 0; i < n; ++i) CHECK(v[i] == k[i] * 16 + 1);
  return 0;
}

int main() {
  const uint32_t caps[3] = {4, 0, 6};
  urb_lru* c = nullptr;
  CHECK(urb_lru_create(3, caps, &c) == URB_OK && c);
  CHECK(urb_lru_create(2, nullptr, &c) == URB_ERR_ARGUMENT);
  urb_lru_telemetry t{};
  uint64_t value = 0, evicted = 0;
  int has = 0;
  for (int round = 0; round < 4000; ++round) {
    const uint32_t layer = (uint32_t)(next() % 4);  // layer 3 does not exist
    const uint64_t key = next() % 10;
    fail_every = round % 7 == 0 ? 3 : 0;
    const int op = (int)(next() % 12);
    if (op < 5) {
      const int st = urb_lru_access(c, &t, layer, key, load, nullptr, &value, &evicted, &has);
      if (layer >= 3) CHECK(st == URB_ERR_ARGUMENT);
    } else if (op == 5) {
      std::vector<uint64_t> keys(1 + next() % 8), order(keys.size());
      for (auto& kk : keys) kk = next() % 10;
      urb_lru_plan* p = urb_lru_grouped_access_plan(c, layer, keys.data(), keys.size());
      if (layer >= 3) CHECK(p == nullptr);
      if (p) {
        const size_t m = urb_lru_plan_order(p, order.data());
        CHECK(m <= keys.size());
        for (size_t i = 0; i < m; ++i)
          (void)urb_lru_access_grouped(c, &t, p, order[i], load, nullptr, &value, &evicted, &has);
        urb_lru_finish_grouped_plan(c, p);
        urb_lru_plan_destroy(p);
      }
    } else if (op == 6) {
      std::vector<uint64_t> keys(1 + next() % 8), order(keys.size());
      for (auto& kk : keys) kk = next() % 10;
      size_t m = 0;
      if (urb_lru_grouped_access_order(c, layer, keys.data(), keys.size(), order.data(), &m)) {
        for (size_t i = 0; i < m; ++i)
          (void)urb_lru_access(c, &t, layer, order[i], load, nullptr, &value, &evicted, &has);
        urb_lru_finish_grouped_accesses(c, layer, keys.data(), keys.size(), m);
      }
      // more groups than clock ticks: refused, nothing changes
      const uint64_t clock = urb_lru_clock(c);
      if (clock < UINT64_MAX - 5) {
        urb_lru_finish_grouped_accesses(c, layer, keys.data(), keys.size(), (size_t)clock + 5);
        CHECK(urb_lru_clock(c) == clock);
      }
    } else if (op == 7) {
      std::vector<uint64_t> keys, out(8);
      for (uint64_t kk = next() % 10; keys.size() < 1 + next() % 6; kk = (kk + 3) % 10)
        if (std::find(keys.begin(), keys.end(), kk) == keys.end()) keys.push_back(kk);
      size_t m = 0;
      (void)urb_lru_prepare_ordered_batch(c, &t, layer, keys.data(), keys.size(), out.data(), &m);
      CHECK(m <= out.size());
    } else if (op == 8) {
      const uint32_t steady = urb_lru_lend_unused_capacity(c, layer, (uint32_t)(next() % 9));
      std::vector<uint64_t> out(64);
      if (layer < 3) urb_lru_restore_layer_capacity(c, &t, layer, steady, out.data());
    } else if (op == 9) {
      std::vector<uint64_t> out(64);
      if (next() % 8 == 0) (void)urb_lru_drain_layer(c, &t, layer, out.data());
      uint64_t e = 0, b = 0;
      urb_lru_residency(c, layer, &e, &b);
      if (layer >= 3) CHECK(e == 0 && b == 0);
    } else if (op == 10) {
      uint64_t keys[3] = {next() % 10, next() % 10, next() % 10};
      (void)urb_lru_can_insert_without_eviction(c, layer, keys, 3);
      (void)urb_lru_projected_misses(c, layer, keys, 3);
      (void)urb_lru_contains(c, layer, keys[0]);
      (void)urb_lru_peek(c, layer, keys[1], &value);
      (void)urb_lru_layer_is_empty(c, layer);
    } else {
      if (next() % 50 == 0) urb_lru_set_clock(c, UINT64_MAX - next() % 4);  // saturation
    }
    for (uint32_t l = 0; l < 3; ++l)
      if (check_layer(c, l)) return 1;
  }
  // NULL handles and arguments are refused, not dereferenced
  CHECK(urb_lru_access(nullptr, &t, 0, 1, load, nullptr, &value, &evicted, &has) ==
        URB_ERR_ARGUMENT);
  CHECK(urb_lru_access(c, nullptr, 0, 1, load, nullptr, &value, &evicted, &has) ==
        URB_ERR_ARGUMENT);
  CHECK(urb_lru_layer_capacity(nullptr, 0) == 0);
  CHECK(urb_lru_grouped_access_plan(c, 0, nullptr, 3) == nullptr);
  urb_lru_destroy(c);
  std::printf("lru driver ok: %llu loads, %llu hits, %llu misses\n", (unsigned long long)loads,
              (unsigned long long)t.hits, (unsigned long long)t.misses);
  return 0;
}
