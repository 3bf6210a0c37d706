// C entry points over the reference's own SlotPool, placement parser and
// records manifest parser
// (components/moe/src/store.cpp, manifest.cpp), compiled from the reference
// sources into oracle/_ref/libds41_refpool.so by `make ref`.
// TEST INFRASTRUCTURE ONLY: tests/ compare the library's ExpertPool against it.
// Error codes: -1 std::runtime_error, -2 std::out_of_range, -3 other
// std::logic_error, -4 std::invalid_argument.
#include <cstring>
#include <fstream>
#include <stdexcept>
#include <unordered_set>
#include <vector>
#include "ds41/store.hpp"

namespace {
template <class F> int guarded(F f) {
  try {
    return f();
  } catch (const std::out_of_range &) {
    return -2;
  } catch (const std::invalid_argument &) {
    return -4;
  } catch (const std::logic_error &) {
    return -3;
  } catch (const std::runtime_error &) {
    return -1;
  }
}
int put(const std::vector<ds41::SlotPool::Allocation> &a, int64_t *out) {
  for (size_t i = 0; i < a.size(); ++i) {
    out[4 * i] = a[i].id;
    out[4 * i + 1] = (int64_t)a[i].slot;
    out[4 * i + 2] = a[i].hit;
    out[4 * i + 3] = a[i].evicted;
  }
  return (int)a.size();
}
}  // namespace

extern "C" {
void *refpool_create(size_t slots, unsigned recent, unsigned decay, int distinct) {
  return new ds41::SlotPool(slots, recent, decay, distinct != 0);
}
void refpool_destroy(void *p) { delete static_cast<ds41::SlotPool *>(p); }
int refpool_expert_count() { return (int)ds41::expert_count; }
int refpool_policy(void *p, const uint32_t *budget, int hard, const uint32_t *pins, int npins, unsigned recent,
                   unsigned decay, int distinct) {
  return guarded([&] {
    ds41::Placement q;
    for (int l = 0; l < 43; ++l) q.dynamic_slots_per_layer[l] = budget[l];
    q.hard_layer_budgets = hard != 0;
    q.vram_pins.assign(pins, pins + npins);
    q.recent_window = recent;
    q.decay_interval = decay;
    q.distinct_lfu = distinct != 0;
    static_cast<ds41::SlotPool *>(p)->policy(q);
    return 0;
  });
}
int refpool_acquire(void *p, const uint32_t *ids, int n, int prefetch, int64_t *out) {
  return guarded([&] {
    return put(static_cast<ds41::SlotPool *>(p)->acquire(std::vector<ds41::ExpertId>(ids, ids + n), prefetch != 0),
               out);
  });
}
int refpool_borrow(void *p, const uint32_t *ids, int n, int64_t *out) {
  return guarded(
      [&] { return put(static_cast<ds41::SlotPool *>(p)->borrow(std::vector<ds41::ExpertId>(ids, ids + n)), out); });
}
int refpool_release(void *p, const int64_t *in, int n) {
  return guarded([&] {
    std::vector<ds41::SlotPool::Allocation> a;
    for (int i = 0; i < n; ++i)
      a.push_back({(ds41::ExpertId)in[4 * i], (size_t)in[4 * i + 1], in[4 * i + 2] != 0, in[4 * i + 3]});
    static_cast<ds41::SlotPool *>(p)->release(a);
    return 0;
  });
}
int refpool_touch(void *p, const uint32_t *ids, int n) {
  return guarded([&] {
    static_cast<ds41::SlotPool *>(p)->touch(std::vector<ds41::ExpertId>(ids, ids + n));
    return 0;
  });
}
int refpool_pin(void *p, uint32_t id) {
  return guarded([&] {
    static_cast<ds41::SlotPool *>(p)->pin(id);
    return 0;
  });
}
int refpool_unpin(void *p, uint32_t id) {
  return guarded([&] {
    static_cast<ds41::SlotPool *>(p)->unpin(id);
    return 0;
  });
}
int refpool_residency(void *p, uint32_t id) { return static_cast<ds41::SlotPool *>(p)->residency(id); }
void refpool_reset(void *p) { static_cast<ds41::SlotPool *>(p)->reset_history(); }
// Placement fields: out_u32 = {recent, decay, distinct, hard}; budgets [43] each.
int refplacement_load(const char *path, uint32_t *out_u32, uint32_t *budget, uint32_t *host_budget, uint32_t *vram,
                      int *nvram, int vcap, uint32_t *host, int *nhost, int hcap) {
  return guarded([&] {
    const ds41::Placement q = ds41::load_placement(path);
    out_u32[0] = q.recent_window;
    out_u32[1] = q.decay_interval;
    out_u32[2] = q.distinct_lfu;
    out_u32[3] = q.hard_layer_budgets;
    for (int l = 0; l < 43; ++l) {
      budget[l] = (uint32_t)q.dynamic_slots_per_layer[l];
      host_budget[l] = (uint32_t)q.host_slots_per_layer[l];
    }
    if ((int)q.vram_pins.size() > vcap || (int)q.host_residents.size() > hcap) return -1;
    *nvram = (int)q.vram_pins.size();
    *nhost = (int)q.host_residents.size();
    std::memcpy(vram, q.vram_pins.data(), 4 * q.vram_pins.size());
    std::memcpy(host, q.host_residents.data(), 4 * q.host_residents.size());
    return 0;
  });
}
// Records manifest: rec[15] per record = id, bytes, 6 x (offset, bytes), extent count;
// ext[6] per extent = record index, file_offset, bytes, dst_offset, required, expected;
// paths 4096 bytes per extent. Returns the record count.
int refrecords_load(const char *path, int cap, uint64_t *rec, int ecap, uint64_t *ext, char *paths, int *n_ext) {
  return guarded([&] {
    const auto r = ds41::load_records(path);
    if ((int)r.size() > cap) return -1;
    int k = 0;
    for (size_t i = 0; i < r.size(); ++i) {
      uint64_t *o = rec + 15 * i;
      const ds41::TensorView v[6] = {r[i].gate, r[i].gate_scale, r[i].up, r[i].up_scale, r[i].down, r[i].down_scale};
      o[0] = r[i].id;
      o[1] = r[i].bytes;
      for (int j = 0; j < 6; ++j) {
        o[2 + 2 * j] = v[j].offset;
        o[3 + 2 * j] = v[j].bytes;
      }
      o[14] = r[i].extents.size();
      for (const auto &e : r[i].extents) {
        if (k >= ecap || e.path.size() >= 4096) return -1;
        uint64_t *x = ext + 6 * k;
        x[0] = i;
        x[1] = e.file_offset;
        x[2] = e.bytes;
        x[3] = e.dst_offset;
        x[4] = e.required_bytes;
        x[5] = e.expected_file_bytes;
        std::memcpy(paths + 4096 * k, e.path.c_str(), e.path.size() + 1);
        ++k;
      }
    }
    *n_ext = k;
    return (int)r.size();
  });
}
// Two-tier extensions of the reference SlotPool and its drift controller.
void *refpool_retain(void *p, uint32_t id, int *rc) {
  void *out = nullptr;
  *rc = guarded([&] {
    out = new std::shared_ptr<const void>(static_cast<ds41::SlotPool *>(p)->retain(id));
    return 0;
  });
  return out;
}
void refpool_token_release(void *t) { delete static_cast<std::shared_ptr<const void> *>(t); }
int refpool_reserve(void *p, size_t target, const uint32_t *wanted, int n, int64_t *out) {
  return guarded([&] {
    std::unordered_set<ds41::ExpertId> w(wanted, wanted + n);
    return put(static_cast<ds41::SlotPool *>(p)->reserve(target, w), out);
  });
}
int refpool_drained(void *p, size_t slot) {
  return guarded([&] {
    static_cast<ds41::SlotPool *>(p)->drained(slot);
    return 0;
  });
}
int refpool_peer(void *p, void *peer, int host) {
  static_cast<ds41::SlotPool *>(p)->peer(static_cast<const ds41::SlotPool *>(peer), host != 0);
  return 0;
}
int refpool_exclusive(void *p, int on) {
  static_cast<ds41::SlotPool *>(p)->exclusive(on != 0);
  return 0;
}
int refpool_decay_interval(void *p, unsigned d) {
  static_cast<ds41::SlotPool *>(p)->decay_interval(d);
  return 0;
}
int refpool_fast_minima(void *p, int on) {
  static_cast<ds41::SlotPool *>(p)->fast_minima(on != 0);
  return 0;
}
int refpool_switch_target_layer(void *p, const uint32_t *pins, int npins, unsigned layer) {
  return guarded([&] {
    ds41::Placement q;
    q.vram_pins.assign(pins, pins + npins);
    static_cast<ds41::SlotPool *>(p)->switch_target_layer(q, layer);
    return 0;
  });
}
void *refdrift_create(const uint32_t *pins, int npins, unsigned recent, unsigned decay, int distinct, int hard,
                      void *vram, void *ram, int *rc) {
  void *out = nullptr;
  *rc = guarded([&] {
    ds41::Placement q;
    q.vram_pins.assign(pins, pins + npins);
    q.recent_window = recent;
    q.decay_interval = decay;
    q.distinct_lfu = distinct != 0;
    q.hard_layer_budgets = hard != 0;
    out = new ds41::DriftPolicy(q, *static_cast<ds41::SlotPool *>(vram), *static_cast<ds41::SlotPool *>(ram));
    return 0;
  });
  return out;
}
int refdrift_before(void *d, const uint32_t *ids, int n) {
  return guarded([&] {
    static_cast<ds41::DriftPolicy *>(d)->before(std::vector<ds41::ExpertId>(ids, ids + n));
    return 0;
  });
}
int refdrift_after(void *d, const uint32_t *ids, int n) {
  return guarded([&] {
    static_cast<ds41::DriftPolicy *>(d)->after(std::vector<ds41::ExpertId>(ids, ids + n));
    return 0;
  });
}
int refdrift_active(void *d) { return static_cast<ds41::DriftPolicy *>(d)->active() ? 1 : 0; }
uint64_t refdrift_tokens(void *d) { return static_cast<ds41::DriftPolicy *>(d)->completed_tokens(); }
void refdrift_destroy(void *d) { delete static_cast<ds41::DriftPolicy *>(d); }
}
