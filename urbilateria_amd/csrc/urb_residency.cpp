// urb_residency.cpp -- the HBM expert-residency policy (include/urb_residency.h): the
// deterministic per-layer LRU of LayerLruCache (src/runtime/cache.rs:66-519), host code.
//
// Entries of a layer live in a vector in insertion order (removal keeps the order of the rest),
// so every "first minimum", drain order and oldest-first trim is the reference's.  Victims are
// the entry with the smallest (last_used, key); keys are unique per layer, so there are no ties.
#include "../../include/urb_residency.h"

#include <algorithm>
#include <cstdint>
#include <limits>
#include <utility>
#include <vector>

namespace {

constexpr uint64_t kMax = std::numeric_limits<uint64_t>::max();
inline uint64_t sat_add(uint64_t a, uint64_t b) { return a > kMax - b ? kMax : a + b; }
inline uint64_t sat_sub(uint64_t a, uint64_t b) { return a < b ? 0 : a - b; }

struct Entry {
  uint64_t key, last_used, bytes, value;
};

using Keyed = std::pair<uint64_t, uint64_t>;  // (key, last_used)

// Position of the (last_used, key) minimum among entries passing `keep`, or -1.
template <class V, class F>
long victim(const V& entries, F keep) {
  long best = -1;
  for (size_t i = 0; i < entries.size(); ++i) {
    if (!keep(entries[i])) continue;
    if (best < 0) {
      best = (long)i;
      continue;
    }
    const auto& b = entries[(size_t)best];
    const auto& e = entries[i];
    if (std::make_pair(e.last_used, e.key) < std::make_pair(b.last_used, b.key)) best = (long)i;
  }
  return best;
}

// Keys in last-use order: reverse, keep first occurrences, reverse again (cache.rs:238-245).
std::vector<uint64_t> last_use_order(const uint64_t* keys, size_t n) {
  std::vector<uint64_t> out;
  for (size_t i = n; i-- > 0;)
    if (std::find(out.begin(), out.end(), keys[i]) == out.end()) out.push_back(keys[i]);
  std::reverse(out.begin(), out.end());
  return out;
}

}  // namespace

struct urb_lru {
  std::vector<std::vector<Entry>> layers;
  std::vector<uint32_t> capacities;
  uint64_t budget = 0;
  uint64_t clock = 0;

  // Layer indices come from the caller: every entry point checks them before indexing (the
  // reference indexes its Vec and panics; here an out-of-range layer is refused).
  bool has(uint32_t layer) const { return layer < layers.size(); }

  bool contains(uint32_t layer, uint64_t key) const {
    if (!has(layer)) return false;
    for (const Entry& e : layers[layer])
      if (e.key == key) return true;
    return false;
  }

  // projected_accesses (cache.rs:373-401): the serial replay's final (key, last_used) entries
  // and its miss count.
  std::pair<std::vector<Keyed>, size_t> projected(uint32_t layer, const uint64_t* keys,
                                                  size_t n) const {
    const size_t cap = capacities[layer];
    if (cap == 0) return {{}, n};
    struct Sim {
      uint64_t key, last_used;
    };
    std::vector<Sim> sim;
    for (const Entry& e : layers[layer]) sim.push_back({e.key, e.last_used});
    uint64_t c = clock;
    size_t misses = 0;
    for (size_t i = 0; i < n; ++i) {
      c = sat_add(c, 1);
      auto it = std::find_if(sim.begin(), sim.end(), [&](const Sim& s) { return s.key == keys[i]; });
      if (it != sim.end()) {
        it->last_used = c;
        continue;
      }
      ++misses;
      if (sim.size() == cap) sim.erase(sim.begin() + victim(sim, [](const Sim&) { return true; }));
      sim.push_back({keys[i], c});
    }
    std::vector<Keyed> out;
    for (const Sim& s : sim) out.push_back({s.key, s.last_used});
    return {out, misses};
  }

  void evicted_account(urb_lru_telemetry* t, const Entry& e) {
    t->evictions = sat_add(t->evictions, 1);
    t->resident_experts = sat_sub(t->resident_experts, 1);
    t->resident_bytes = sat_sub(t->resident_bytes, e.bytes);
  }
};

struct urb_lru_plan {
  uint32_t layer;
  std::vector<uint64_t> order;
  std::vector<Keyed> retained;  // sorted by key
  uint64_t initial_clock, final_clock;

  bool retains(uint64_t key) const {
    auto it = std::lower_bound(retained.begin(), retained.end(), Keyed{key, 0},
                               [](const Keyed& a, const Keyed& b) { return a.first < b.first; });
    return it != retained.end() && it->first == key;
  }
  uint64_t retained_use(uint64_t key) const {
    auto it = std::lower_bound(retained.begin(), retained.end(), Keyed{key, 0},
                               [](const Keyed& a, const Keyed& b) { return a.first < b.first; });
    return it->second;
  }
};

extern "C" {

urb_status urb_lru_create(uint32_t layers, const uint32_t* capacities, urb_lru** out) {
  if (!out || (layers && !capacities)) return URB_ERR_ARGUMENT;
  urb_lru* c = new urb_lru;
  c->layers.resize(layers);
  c->capacities.assign(capacities, capacities + layers);
  for (uint32_t cap : c->capacities) c->budget += cap;
  *out = c;
  return URB_OK;
}

void urb_lru_destroy(urb_lru* lru) { delete lru; }

int urb_lru_access(urb_lru* c, urb_lru_telemetry* t, uint32_t layer, uint64_t key,
                   urb_lru_load_fn load, void* user, uint64_t* value, uint64_t* evicted,
                   int* has_evicted) {
  if (!c || !t || !value || !evicted || !has_evicted || !load || !c->has(layer))
    return URB_ERR_ARGUMENT;
  *has_evicted = 0;
  c->clock = sat_add(c->clock, 1);
  auto& entries = c->layers[layer];
  for (Entry& e : entries)
    if (e.key == key) {
      t->hits = sat_add(t->hits, 1);
      e.last_used = c->clock;
      *value = e.value;
      return 0;
    }
  t->misses = sat_add(t->misses, 1);
  const size_t cap = c->capacities[layer];
  uint64_t v = 0, bytes = 0, read = 0;
  if (cap == 0) {
    const int st = load(user, layer, key, &v, &bytes, &read);
    if (st) return st;
    t->bytes_read = sat_add(t->bytes_read, read);
    *value = v;
    *evicted = v;  // transient: the caller keeps it only for this access
    *has_evicted = 1;
    return 0;
  }
  if (entries.size() == cap) {
    const long p = victim(entries, [](const Entry&) { return true; });
    const Entry e = entries[(size_t)p];
    entries.erase(entries.begin() + p);
    c->evicted_account(t, e);
    *evicted = e.value;
    *has_evicted = 1;
  }
  const int st = load(user, layer, key, &v, &bytes, &read);
  if (st) return st;
  t->bytes_read = sat_add(t->bytes_read, read);
  t->resident_experts = sat_add(t->resident_experts, 1);
  t->resident_bytes = sat_add(t->resident_bytes, bytes);
  entries.push_back({key, c->clock, bytes, v});
  *value = v;
  return 0;
}

int urb_lru_contains(const urb_lru* c, uint32_t layer, uint64_t key) {
  return c && c->contains(layer, key) ? 1 : 0;
}

int urb_lru_peek(const urb_lru* c, uint32_t layer, uint64_t key, uint64_t* value) {
  if (!c || !value || !c->has(layer)) return 0;
  for (const Entry& e : c->layers[layer])
    if (e.key == key) {
      *value = e.value;
      return 1;
    }
  return 0;
}

int urb_lru_layer_is_empty(const urb_lru* c, uint32_t layer) {
  return !c || !c->has(layer) || c->layers[layer].empty() ? 1 : 0;
}

uint32_t urb_lru_layer_capacity(const urb_lru* c, uint32_t layer) {
  return c && c->has(layer) ? c->capacities[layer] : 0;
}

void urb_lru_residency(const urb_lru* c, uint32_t layer, uint64_t* experts, uint64_t* bytes) {
  if (!experts || !bytes) return;
  *experts = 0;
  *bytes = 0;
  if (!c || !c->has(layer)) return;
  uint64_t b = 0;
  for (const Entry& e : c->layers[layer]) b = sat_add(b, e.bytes);
  *experts = c->layers[layer].size();
  *bytes = b;
}

size_t urb_lru_entries(const urb_lru* c, uint32_t layer, uint64_t* keys, uint64_t* last_used,
                       uint64_t* values) {
  if (!c || !c->has(layer)) return 0;
  const auto& entries = c->layers[layer];
  for (size_t i = 0; i < entries.size(); ++i) {
    if (keys) keys[i] = entries[i].key;
    if (last_used) last_used[i] = entries[i].last_used;
    if (values) values[i] = entries[i].value;
  }
  return entries.size();
}

uint64_t urb_lru_clock(const urb_lru* c) { return c ? c->clock : 0; }
void urb_lru_set_clock(urb_lru* c, uint64_t clock) {
  if (c) c->clock = clock;
}

size_t urb_lru_drain_layer(urb_lru* c, urb_lru_telemetry* t, uint32_t layer,
                           uint64_t* values_out) {
  if (!c || !t || !c->has(layer)) return 0;
  std::vector<Entry> entries;
  entries.swap(c->layers[layer]);
  uint64_t bytes = 0;
  for (size_t i = 0; i < entries.size(); ++i) {
    bytes = sat_add(bytes, entries[i].bytes);
    if (values_out) values_out[i] = entries[i].value;
  }
  t->evictions = sat_add(t->evictions, entries.size());
  t->resident_experts = sat_sub(t->resident_experts, entries.size());
  t->resident_bytes = sat_sub(t->resident_bytes, bytes);
  return entries.size();
}

int urb_lru_can_insert_without_eviction(const urb_lru* c, uint32_t layer, const uint64_t* keys,
                                        size_t n) {
  if (!c || !c->has(layer) || (n && !keys)) return 0;
  const size_t cap = c->capacities[layer];
  if (cap == 0) return 0;
  std::vector<uint64_t> missing;
  for (size_t i = 0; i < n; ++i)
    if (!c->contains(layer, keys[i]) &&
        std::find(missing.begin(), missing.end(), keys[i]) == missing.end())
      missing.push_back(keys[i]);
  return c->layers[layer].size() + missing.size() <= cap ? 1 : 0;
}

size_t urb_lru_projected_misses(const urb_lru* c, uint32_t layer, const uint64_t* keys,
                                size_t n) {
  if (!c || !c->has(layer) || (n && !keys)) return n;
  return c->projected(layer, keys, n).second;
}

int urb_lru_grouped_access_order(const urb_lru* c, uint32_t layer, const uint64_t* keys,
                                 size_t n, uint64_t* order_out, size_t* order_n) {
  if (!c || !c->has(layer) || !order_out || !order_n || (n && !keys)) return 0;
  // once timestamps would saturate, key order no longer stands for recency
  if (c->clock > kMax - (uint64_t)n) return 0;
  const std::vector<uint64_t> grouped = last_use_order(keys, n);
  if (grouped.size() == n) return 0;
  if (c->projected(layer, grouped.data(), grouped.size()).second >
      c->projected(layer, keys, n).second)
    return 0;
  std::copy(grouped.begin(), grouped.end(), order_out);
  *order_n = grouped.size();
  return 1;
}

void urb_lru_finish_grouped_accesses(urb_lru* c, uint32_t layer, const uint64_t* keys, size_t n,
                                     size_t groups) {
  // the clock advanced once per group access since the schedule began, so it is at least
  // `groups`; a call that breaks this (or names another layer) changes nothing
  if (!c || !c->has(layer) || (n && !keys) || c->clock < groups) return;
  if (c->clock - groups > kMax - n) return;
  const uint64_t initial = c->clock - groups;
  c->clock = initial + n;
  for (Entry& e : c->layers[layer])
    for (size_t i = n; i-- > 0;)
      if (keys[i] == e.key) {
        e.last_used = initial + i + 1;
        break;
      }
}

urb_lru_plan* urb_lru_grouped_access_plan(const urb_lru* c, uint32_t layer, const uint64_t* keys,
                                          size_t n) {
  if (!c || !c->has(layer) || !keys) return nullptr;
  if (c->capacities[layer] == 0 || n == 0) return nullptr;
  if (c->clock > kMax - (uint64_t)n) return nullptr;
  std::vector<uint64_t> order = last_use_order(keys, n);
  auto proj = c->projected(layer, keys, n);
  size_t minimum = 0;
  for (uint64_t k : order)
    if (!c->contains(layer, k)) ++minimum;
  if (order.size() == n && minimum == proj.second) return nullptr;
  // stable partition: resident keys first, last-use order kept inside both parts
  std::stable_sort(order.begin(), order.end(), [&](uint64_t a, uint64_t b) {
    return c->contains(layer, a) && !c->contains(layer, b);
  });
  urb_lru_plan* p = new urb_lru_plan;
  p->layer = layer;
  p->order = std::move(order);
  p->retained = std::move(proj.first);
  std::sort(p->retained.begin(), p->retained.end(),
            [](const Keyed& a, const Keyed& b) { return a.first < b.first; });
  p->initial_clock = c->clock;
  p->final_clock = c->clock + n;
  return p;
}

void urb_lru_plan_destroy(urb_lru_plan* plan) { delete plan; }

size_t urb_lru_plan_order(const urb_lru_plan* plan, uint64_t* order_out) {
  if (!plan || !order_out) return 0;
  std::copy(plan->order.begin(), plan->order.end(), order_out);
  return plan->order.size();
}

int urb_lru_access_grouped(urb_lru* c, urb_lru_telemetry* t, const urb_lru_plan* plan,
                           uint64_t key, urb_lru_load_fn load, void* user, uint64_t* value,
                           uint64_t* evicted, int* has_evicted) {
  if (!c || !t || !plan || !load || !value || !evicted || !has_evicted || !c->has(plan->layer))
    return URB_ERR_ARGUMENT;
  const uint32_t layer = plan->layer;
  if (c->contains(layer, key))
    return urb_lru_access(c, t, layer, key, load, user, value, evicted, has_evicted);
  *has_evicted = 0;
  uint64_t v = 0, bytes = 0, read = 0;
  const int st = load(user, layer, key, &v, &bytes, &read);
  if (st) return st;  // nothing changed
  c->clock = sat_add(c->clock, 1);
  t->misses = sat_add(t->misses, 1);
  t->bytes_read = sat_add(t->bytes_read, read);
  *value = v;
  if (!plan->retains(key)) {
    *evicted = v;  // transient: not part of the final hot set
    *has_evicted = 1;
    return 0;
  }
  auto& entries = c->layers[layer];
  if (entries.size() == c->capacities[layer]) {
    const long p = victim(entries, [&](const Entry& e) { return !plan->retains(e.key); });
    const Entry e = entries[(size_t)p];
    entries.erase(entries.begin() + p);
    c->evicted_account(t, e);
    *evicted = e.value;
    *has_evicted = 1;
  }
  t->resident_experts = sat_add(t->resident_experts, 1);
  t->resident_bytes = sat_add(t->resident_bytes, bytes);
  entries.push_back({key, c->clock, bytes, v});
  return 0;
}

void urb_lru_finish_grouped_plan(urb_lru* c, const urb_lru_plan* plan) {
  if (!c || !plan || !c->has(plan->layer)) return;
  // after the schedule only final keys are resident
  for (Entry& e : c->layers[plan->layer])
    if (plan->retains(e.key)) e.last_used = plan->retained_use(e.key);
  c->clock = plan->final_clock;
}

int urb_lru_prepare_ordered_batch(urb_lru* c, urb_lru_telemetry* t, uint32_t layer,
                                  const uint64_t* keys, size_t n, uint64_t* evicted_out,
                                  size_t* n_evicted) {
  if (!c || !t || !c->has(layer) || !evicted_out || !n_evicted || (n && !keys)) return 0;
  const size_t cap = c->capacities[layer];
  if (cap == 0 || n == 0 || n > cap) return 0;
  for (size_t i = 0; i < n; ++i)
    for (size_t j = 0; j < i; ++j)
      if (keys[j] == keys[i]) return 0;
  struct Sim {
    uint64_t key, last_used;
  };
  std::vector<Sim> sim;
  for (const Entry& e : c->layers[layer]) sim.push_back({e.key, e.last_used});
  uint64_t clk = c->clock;
  std::vector<uint64_t> victims;
  for (size_t i = 0; i < n; ++i) {
    clk = sat_add(clk, 1);
    auto it = std::find_if(sim.begin(), sim.end(), [&](const Sim& s) { return s.key == keys[i]; });
    if (it != sim.end()) {
      it->last_used = clk;
      continue;
    }
    if (sim.size() == cap) {
      const long p = victim(sim, [](const Sim&) { return true; });
      victims.push_back(sim[(size_t)p].key);
      sim.erase(sim.begin() + p);
    }
    sim.push_back({keys[i], clk});
  }
  for (uint64_t k : victims)
    if (!c->contains(layer, k)) return 0;
  // Once the clock saturates, timestamps tie and an original entry the batch reloaded can be
  // evicted a second time (the reference's "every simulated eviction refers to an original
  // entry" then panics): refuse the batch, changing nothing.
  for (size_t i = 0; i < victims.size(); ++i)
    for (size_t j = 0; j < i; ++j)
      if (victims[i] == victims[j]) return 0;
  auto& entries = c->layers[layer];
  size_t m = 0;
  for (uint64_t k : victims) {
    auto it = std::find_if(entries.begin(), entries.end(), [&](const Entry& e) { return e.key == k; });
    const Entry e = *it;
    entries.erase(it);
    c->evicted_account(t, e);
    evicted_out[m++] = e.value;
  }
  *n_evicted = m;
  return 1;
}

uint32_t urb_lru_lend_unused_capacity(urb_lru* c, uint32_t layer, uint32_t maximum) {
  if (!c || !c->has(layer)) return 0;
  const uint32_t steady = c->capacities[layer];
  uint64_t elsewhere = 0;
  for (size_t l = 0; l < c->layers.size(); ++l)
    if (l != layer) elsewhere += c->layers[l].size();
  const uint64_t available = sat_sub(c->budget, elsewhere);
  c->capacities[layer] = (uint32_t)std::min<uint64_t>(available, maximum);
  return steady;
}

size_t urb_lru_restore_layer_capacity(urb_lru* c, urb_lru_telemetry* t, uint32_t layer,
                                      uint32_t capacity, uint64_t* evicted_out) {
  if (!c || !t || !c->has(layer)) return 0;
  c->capacities[layer] = capacity;
  auto& entries = c->layers[layer];
  size_t m = 0;
  while (entries.size() > capacity) {
    const long p = victim(entries, [](const Entry&) { return true; });
    const Entry e = entries[(size_t)p];
    entries.erase(entries.begin() + p);
    c->evicted_account(t, e);
    if (evicted_out) evicted_out[m] = e.value;
    ++m;
  }
  return m;
}

}  // extern "C"
