// Host-side expert slot pool: which expert occupies which HBM slot, chosen by
// the reference's deterministic LFU policy (components/moe/include/ds41/store.hpp:80-157,
// components/moe/src/store.cpp:15-196 SlotPool), and the text placement format
// that configures it (components/moe/src/manifest.cpp:8-34 load_placement).
//
// Expert ids are flattened layer by layer (layer l owns ids first[l] ..
// first[l] + experts[l] - 1), which covers the reference's 40 x 384 target +
// 3 x 128 drafter space (store.hpp:16) and the verify stack's L x E space.
//
// Policy, as the reference's:
// - every demand (non-prefetch acquire, or touch) advances the clock of each
//   layer it names once; every `decay` ticks of a layer's clock halve the
//   counts of all that layer's experts, before this demand's counts are added;
//   counts add once per distinct id (distinct LFU) or once per occurrence;
// - a miss takes the lowest empty slot (of its layer under hard budgets), else
//   evicts a victim: never pinned, leased or wanted by the same call; first
//   among slots not used within the last `recent` ticks of their layer's clock,
//   then among all; an over-budget layer's slot before any other; then the
//   lowest (count, last-acquire stamp, slot index);
// - the whole call is rejected before any state changes when the distinct ids
//   exceed the slots it could use.
// Not carried over: retention tokens, draining/reserve, the two-tier peer and
// late-layer score adjustments and the drift controller, which belong to the
// reference's RAM/NVMe tiers (this build's host tier is a static pinned copy of
// every non-resident expert).
#pragma once
#include <cstdint>
#include <fstream>
#include <sstream>
#include <stdexcept>
#include <string>
#include <unordered_set>
#include <vector>

namespace ds41g {

struct PoolError : std::runtime_error {
  int code;  // -1 capacity, -2 id out of range, -3 illegal state, -4 invalid argument
  PoolError(int c, const std::string &m) : std::runtime_error(m), code(c) {}
};

struct PoolPolicy {
  uint32_t recent = 6, decay = 32;
  bool distinct = true, hard = false;
  std::vector<uint32_t> budget;       // per layer, dynamic slots (pinned slots excluded)
  std::vector<uint32_t> host_budget;  // per layer (parsed, used by host tiers)
  std::vector<uint32_t> pins, host;   // vram pins, host residents
};

class ExpertPool {
 public:
  struct Alloc {
    uint32_t id;
    int32_t slot;
    bool hit;
    int64_t evicted;
  };

  ExpertPool(size_t slots, std::vector<uint32_t> layer_experts, uint32_t recent = 6, uint32_t decay = 32,
             bool distinct = true)
      : slot_(slots), per_layer_(std::move(layer_experts)), recent_(recent), decay_(decay), distinct_(distinct) {
    if (!slots) throw PoolError(-4, "empty slot pool");
    if (per_layer_.empty()) throw PoolError(-4, "no layers");
    first_.resize(per_layer_.size() + 1, 0);
    for (size_t l = 0; l < per_layer_.size(); ++l) first_[l + 1] = first_[l] + per_layer_[l];
    n_ids_ = first_.back();
    layer_.resize(n_ids_);
    for (uint32_t l = 0; l < per_layer_.size(); ++l)
      for (uint32_t e = first_[l]; e < first_[l + 1]; ++e) layer_[e] = l;
    where_.assign(n_ids_, -1);
    count_.assign(n_ids_, 0);
    last_.assign(n_ids_, 0);
    tick_.assign(per_layer_.size(), 0);
    budget_.assign(per_layer_.size(), 0);
  }

  size_t slots() const { return slot_.size(); }
  uint32_t ids() const { return n_ids_; }
  uint32_t layer_of(uint32_t id) const { return layer_[id]; }
  uint32_t first_of(uint32_t layer) const { return first_[layer]; }
  size_t layers() const { return per_layer_.size(); }

  void policy(const PoolPolicy &p) {
    recent_ = p.recent;
    decay_ = p.decay;
    distinct_ = p.distinct;
    budget_.assign(per_layer_.size(), 0);
    for (size_t l = 0; l < p.budget.size() && l < budget_.size(); ++l) budget_[l] = p.budget[l];
    any_budget_ = false;
    for (auto b : budget_) any_budget_ |= b != 0;
    hard_ = p.hard;
    slot_layer_.clear();
    if (hard_) {  // slots are dealt to layers in order: pins + budget of layer 0, then layer 1, ...
      std::vector<size_t> pins(per_layer_.size(), 0);
      for (auto id : p.pins) ++pins.at(layer_of(check(id)));
      for (uint32_t l = 0; l < per_layer_.size(); ++l) slot_layer_.insert(slot_layer_.end(), pins[l] + budget_[l], l);
      if (slot_layer_.size() != slot_.size()) throw PoolError(-4, "hard layer capacities must cover every slot");
      for (size_t s = 0; s < slot_.size(); ++s)
        if (slot_[s].id >= 0 && layer_of((uint32_t)slot_[s].id) != slot_layer_[s])
          throw PoolError(-3, "hard policy requires a compatible pool");
    }
  }

  void reset_history() {
    std::fill(count_.begin(), count_.end(), 0u);
    std::fill(last_.begin(), last_.end(), 0ull);
    std::fill(tick_.begin(), tick_.end(), 0ull);
  }

  void touch(const std::vector<uint32_t> &ids) {
    for (auto e : ids) check(e);
    const std::vector<uint32_t> uniq = distinct_ids(ids);
    std::vector<char> named(per_layer_.size(), 0);
    for (auto e : uniq) named[layer_of(e)] = 1;
    for (uint32_t l = 0; l < per_layer_.size(); ++l) {
      if (!named[l]) continue;
      const uint64_t t = ++tick_[l];
      if (decay_ && t % decay_ == 0)
        for (uint32_t e = first_[l]; e < first_[l + 1]; ++e) count_[e] >>= 1;
    }
    for (auto e : distinct_ ? uniq : ids) {
      if (count_[e] != UINT32_MAX) ++count_[e];
      last_[e] = tick_[layer_of(e)];
    }
  }

  std::vector<Alloc> acquire(const std::vector<uint32_t> &input, bool prefetch = false) {
    for (auto e : input) check(e);
    const std::vector<uint32_t> ids = distinct_ids(input);
    const std::unordered_set<uint32_t> wanted(ids.begin(), ids.end());
    auto usable = [&](const Slot &s) { return s.id < 0 || wanted.count((uint32_t)s.id) || (!s.pinned && !s.leases); };
    if (hard_) {
      std::vector<size_t> need(per_layer_.size(), 0), have(per_layer_.size(), 0);
      for (auto e : ids) ++need[layer_of(e)];
      for (size_t s = 0; s < slot_.size(); ++s) have[slot_layer_[s]] += usable(slot_[s]);
      for (size_t l = 0; l < need.size(); ++l)
        if (need[l] > have[l]) throw PoolError(-1, "need set exceeds hard layer capacity");
    }
    size_t have = 0;
    for (const auto &s : slot_) have += usable(s);
    if (ids.size() > have) throw PoolError(-1, "need set exceeds unleased slot capacity; split the batch");
    if (!prefetch) touch(input);
    std::vector<size_t> held(per_layer_.size(), 0);  // unpinned occupied slots per layer
    for (const auto &s : slot_)
      if (s.id >= 0 && !s.pinned) ++held[layer_of((uint32_t)s.id)];
    std::vector<Alloc> out;
    out.reserve(ids.size());
    for (auto e : ids) {
      int slot = where_[e];
      const bool hit = slot >= 0;
      int64_t evicted = -1;
      if (!hit) {
        const int want_layer = hard_ ? (int)layer_of(e) : -1;
        for (size_t s = 0; s < slot_.size() && slot < 0; ++s)
          if (slot_[s].id < 0 && (want_layer < 0 || slot_layer_[s] == (uint32_t)want_layer)) slot = (int)s;
        if (slot < 0) slot = victim(wanted, held, want_layer);
        if (slot < 0) throw PoolError(-3, "capacity check disagreed with victim search");
        evicted = slot_[slot].id;
        if (evicted >= 0) {
          --held[layer_of((uint32_t)evicted)];
          where_[evicted] = -1;
        }
        ++held[layer_of(e)];
        where_[e] = slot;
        slot_[slot].id = e;
      }
      Slot &s = slot_[slot];
      ++s.leases;
      s.stamp = ++stamp_;
      out.push_back({e, slot, hit, evicted});
    }
    return out;
  }

  std::vector<Alloc> borrow(const std::vector<uint32_t> &ids) {
    for (auto e : ids) check(e);
    std::vector<Alloc> out;
    for (auto e : distinct_ids(ids))
      if (where_[e] >= 0) out.push_back({e, where_[e], true, -1});
    for (const auto &a : out) ++slot_[a.slot].leases;
    return out;
  }

  void release(const std::vector<Alloc> &lease) {
    std::vector<uint32_t> take(slot_.size(), 0);
    for (const auto &a : lease) {
      if (a.slot < 0 || (size_t)a.slot >= slot_.size() || slot_[a.slot].id != (int64_t)a.id ||
          ++take[a.slot] > slot_[a.slot].leases)
        throw PoolError(-3, "invalid or duplicate lease release");
    }
    for (const auto &a : lease) --slot_[a.slot].leases;
  }

  void pin(uint32_t id) {
    const int s = residency(id);
    if (s < 0) throw PoolError(-3, "pin requires a resident expert");
    slot_[s].pinned = true;
  }
  void unpin(uint32_t id) {  // a non-resident (or unknown) id is left alone
    const int s = residency(id);
    if (s >= 0) slot_[s].pinned = false;
  }
  int residency(uint32_t id) const { return id < n_ids_ ? where_[id] : -1; }
  uint32_t frequency(uint32_t id) const { return id < n_ids_ ? count_[id] : 0; }

 private:
  struct Slot {
    int64_t id = -1;
    uint32_t leases = 0;
    bool pinned = false;
    uint64_t stamp = 0;
  };

  uint32_t check(uint32_t id) const {
    if (id >= n_ids_) throw PoolError(-2, "expert id");
    return id;
  }
  static std::vector<uint32_t> distinct_ids(const std::vector<uint32_t> &ids) {
    std::vector<uint32_t> u;
    std::unordered_set<uint32_t> seen;
    for (auto e : ids)
      if (seen.insert(e).second) u.push_back(e);
    return u;
  }
  // Victim: lexicographic minimum of (within budget, count, stamp, slot) over
  // the evictable slots, first excluding those used in the recent window.
  int victim(const std::unordered_set<uint32_t> &wanted, const std::vector<size_t> &held, int want_layer) const {
    for (int pass = 0; pass < 2; ++pass) {
      int best = -1;
      bool best_in = true;
      for (size_t s = 0; s < slot_.size(); ++s) {
        const Slot &c = slot_[s];
        if (c.id < 0 || c.pinned || c.leases || wanted.count((uint32_t)c.id)) continue;
        if (want_layer >= 0 && slot_layer_[s] != (uint32_t)want_layer) continue;
        const uint32_t id = (uint32_t)c.id, l = layer_of(id);
        if (pass == 0 && recent_ && last_[id] && last_[id] + recent_ >= tick_[l]) continue;
        const bool in = !(any_budget_ && held[l] > budget_[l]);
        if (best < 0 || (!in && best_in) || (in == best_in && before((int)s, best))) {
          best = (int)s;
          best_in = in;
        }
      }
      if (best >= 0) return best;
    }
    return -1;
  }
  bool before(int a, int b) const {
    const uint32_t ca = count_[(uint32_t)slot_[a].id], cb = count_[(uint32_t)slot_[b].id];
    if (ca != cb) return ca < cb;
    if (slot_[a].stamp != slot_[b].stamp) return slot_[a].stamp < slot_[b].stamp;
    return a < b;
  }

  std::vector<Slot> slot_;
  std::vector<uint32_t> per_layer_, first_, layer_;
  uint32_t n_ids_ = 0;
  std::vector<int32_t> where_;
  std::vector<uint32_t> count_;
  std::vector<uint64_t> last_, tick_;
  std::vector<uint32_t> budget_, slot_layer_;
  uint32_t recent_, decay_;
  bool distinct_, hard_ = false, any_budget_ = false;
  uint64_t stamp_ = 0;
};

// Placement text (components/moe/src/manifest.cpp:8-34; e.g. the reference's
// profiles/p80-mtp48.placement): one directive per line, '#' comments:
//   vram <id> | host <id>           (each id at most once over both)
//   pools hard|soft                 budget <layer> <n> | host_budget <layer> <n>
//   recent <n> | decay <n>          lfu distinct|multiplicity
inline PoolPolicy parse_placement(std::istream &in, const std::vector<uint32_t> &layer_experts) {
  uint64_t total = 0;
  for (auto n : layer_experts) total += n;
  PoolPolicy p;
  p.budget.assign(layer_experts.size(), 0);
  p.host_budget.assign(layer_experts.size(), 0);
  std::unordered_set<uint32_t> named;
  std::string line;
  while (std::getline(in, line)) {
    if (line.empty() || line[0] == '#') continue;
    std::istringstream w(line);
    std::string op;
    w >> op;
    if (op == "vram" || op == "host") {
      uint32_t id;
      w >> id;
      if (!w || id >= total || !named.insert(id).second) throw PoolError(-4, "invalid/overlapping placement expert");
      (op == "vram" ? p.pins : p.host).push_back(id);
    } else if (op == "pools") {
      std::string m;
      w >> m;
      if (m != "hard" && m != "soft") throw PoolError(-4, "invalid pool mode");
      p.hard = m == "hard";
    } else if (op == "budget" || op == "host_budget") {
      uint32_t l;
      uint64_t n;
      w >> l >> n;
      if (!w || l >= layer_experts.size() || n > layer_experts[l]) throw PoolError(-4, "invalid layer slot budget");
      (op == "budget" ? p.budget : p.host_budget)[l] = (uint32_t)n;
    } else if (op == "recent" || op == "decay") {
      uint64_t n;
      w >> n;
      if (!w || n > UINT32_MAX) throw PoolError(-4, "invalid policy interval");
      (op == "recent" ? p.recent : p.decay) = (uint32_t)n;
    } else if (op == "lfu") {
      std::string m;
      w >> m;
      if (m != "distinct" && m != "multiplicity") throw PoolError(-4, "invalid LFU counting mode");
      p.distinct = m == "distinct";
    } else {
      throw PoolError(-4, "unknown placement directive");
    }
    std::string rest;
    if (w >> rest) throw PoolError(-4, "trailing placement tokens");
  }
  return p;
}

}  // namespace ds41g
