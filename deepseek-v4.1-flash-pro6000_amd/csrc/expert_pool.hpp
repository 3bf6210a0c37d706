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
// Two-tier extensions (store.hpp:87-105, store.cpp:56-66,130-152,164-190):
// - retention tokens: while a caller holds a token of a slot's current
//   occupant, that slot is neither evicted nor counted as usable capacity;
// - reserve/drained: policy victims are moved into draining slots (no
//   occupant, not allocatable) until empty + draining slots reach a target,
//   and return to service one by one;
// - a peer pool (the other tier of a VRAM/RAM pair) and late target layers:
//   the victim order uses a score, the count adjusted by the peer's residency
//   (exclusive host pools score peer-resident experts 0; in a late layer a
//   host pool halves the count of peer-resident experts and a VRAM pool
//   doubles the count of experts the peer lacks), and a late layer's counts
//   decay every 512 (VRAM) or 128 (host) of its ticks; switching a target
//   layer to late releases that layer's VRAM pins into its budget;
// - fast minima (fast_minima): with distinct counting and soft budgets, the
//   victim search reads a per-layer cache of the least evictable slot (all,
//   and outside the recent window), rebuilt for a layer only once something
//   that can change it happened (the layer's residency, leases, pins, counts
//   or stamps, a retention token of the layer, or, for a late or exclusive
//   layer, the peer's residency of it). A reserve() does not mark the layers
//   of its wanted set, so a cache rebuilt under that set can keep skipping
//   those experts afterwards; the reference's cache behaves the same way, and
//   the decisions stay identical to it;
// - DriftControl (DriftPolicy, store.hpp:161-178, store.cpp:220-255): a
//   width-one, token-major controller that switches every target layer of
//   both pools to late once the pinned hit rate over the last 128 tokens falls
//   below one half.
#pragma once
#include <algorithm>
#include <cstdint>
#include <atomic>
#include <deque>
#include <fstream>
#include <memory>
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
    late_.assign(per_layer_.size(), 0);
    dirty_.assign(per_layer_.size(), 1);
    best_any_.assign(per_layer_.size(), -1);
    best_old_.assign(per_layer_.size(), -1);
    epoch_.assign(per_layer_.size(), 0);
    peer_seen_.assign(per_layer_.size(), 0);
    ret_seen_.assign(per_layer_.size(), 0);
    ret_epoch_ = std::make_shared<RetainEpochs>(per_layer_.size());
    for (auto &x : *ret_epoch_) x.store(0);
  }

  size_t slots() const { return slot_.size(); }
  uint32_t ids() const { return n_ids_; }
  uint32_t layer_of(uint32_t id) const { return layer_[id]; }
  uint32_t first_of(uint32_t layer) const { return first_[layer]; }
  size_t layers() const { return per_layer_.size(); }

  void policy(const PoolPolicy &p) {
    mark_all();
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
    mark_all();
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
      dirty_[l] = 1;
      const uint64_t t = ++tick_[l];
      const uint32_t decay = late_[l] ? (host_ ? 128u : 512u) : decay_;
      if (decay && t % decay == 0)
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
    auto usable = [&](const Slot &s) {
      return !s.draining && (s.id < 0 || wanted.count((uint32_t)s.id) || (!s.pinned && !s.leases && !retained(s)));
    };
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
    for (auto e : ids) dirty_[layer_of(e)] = 1;
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
          if (slot_[s].id < 0 && !slot_[s].draining && (want_layer < 0 || slot_layer_[s] == (uint32_t)want_layer))
            slot = (int)s;
        if (slot < 0) slot = fast_ && distinct_ && !hard_ ? fast_victim(wanted, held) : victim(wanted, held, want_layer);
        if (slot < 0) throw PoolError(-3, "capacity check disagreed with victim search");
        evicted = slot_[slot].id;
        if (evicted >= 0) {
          moved(layer_of((uint32_t)evicted));
          --held[layer_of((uint32_t)evicted)];
          where_[evicted] = -1;
        }
        moved(layer_of(e));
        ++held[layer_of(e)];
        where_[e] = slot;
        slot_[slot].id = e;
        slot_[slot].hold = std::make_shared<const uint32_t>(e);  // a new occupant: earlier tokens are moot
      }
      Slot &s = slot_[slot];
      dirty_[layer_of(e)] = 1;
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
    for (const auto &a : out) {
      ++slot_[a.slot].leases;
      dirty_[layer_of(a.id)] = 1;
    }
    return out;
  }

  void release(const std::vector<Alloc> &lease) {
    std::vector<uint32_t> take(slot_.size(), 0);
    for (const auto &a : lease) {
      if (a.slot < 0 || (size_t)a.slot >= slot_.size() || slot_[a.slot].id != (int64_t)a.id ||
          ++take[a.slot] > slot_[a.slot].leases)
        throw PoolError(-3, "invalid or duplicate lease release");
    }
    for (const auto &a : lease) {
      --slot_[a.slot].leases;
      dirty_[layer_of(a.id)] = 1;
    }
  }

  void pin(uint32_t id) {
    const int s = residency(id);
    if (s < 0) throw PoolError(-3, "pin requires a resident expert");
    slot_[s].pinned = true;
    dirty_[layer_of(id)] = 1;
  }
  void unpin(uint32_t id) {  // a non-resident (or unknown) id is left alone
    const int s = residency(id);
    if (s < 0) return;
    slot_[s].pinned = false;
    dirty_[layer_of(id)] = 1;
  }
  int residency(uint32_t id) const { return id < n_ids_ ? where_[id] : -1; }
  uint32_t frequency(uint32_t id) const { return id < n_ids_ ? count_[id] : 0; }

  // A token of the slot's current occupant: the slot keeps it (no eviction, no reserve) while any
  // copy of the token lives. Dropping a copy is thread-safe and never touches the pool.
  // With fast minima the token also moves the layer's retention epoch when it is taken and when
  // its last copy is dropped, so that the layer's cached minima are rebuilt.
  std::shared_ptr<const void> retain(uint32_t id) const {
    const int s = residency(check(id));
    if (s < 0) throw PoolError(-3, "retain requires a resident expert");
    if (!fast_) return slot_[s].hold;
    std::shared_ptr<RetainEpochs> ep = ret_epoch_;
    const uint32_t l = layer_of(id);
    std::shared_ptr<const uint32_t> hold = slot_[s].hold;
    const void *addr = hold.get();
    (*ep)[l].fetch_add(1, std::memory_order_release);
    return std::shared_ptr<const void>(addr, [hold, ep, l](const void *) mutable {
      hold.reset();
      (*ep)[l].fetch_add(1, std::memory_order_release);
    });
  }

  // Moves policy victims (never wanted, pinned, leased or retained) into draining slots until the
  // empty and draining slots number `target`, or no victim is left; returns one allocation per
  // victim (slot, evicted = its expert). No clock moves.
  std::vector<Alloc> reserve(size_t target, const std::unordered_set<uint32_t> &wanted) {
    if (hard_) throw PoolError(-3, "reserve requires soft layer budgets");
    std::vector<Alloc> out;
    size_t idle = 0;
    for (const auto &s : slot_) idle += s.id < 0;
    if (idle >= target) return out;
    std::vector<size_t> held_n(per_layer_.size(), 0);
    for (const auto &s : slot_)
      if (s.id >= 0 && !s.pinned) ++held_n[layer_of((uint32_t)s.id)];
    for (; idle < target; ++idle) {
      const int v = fast_ && distinct_ ? fast_victim(wanted, held_n) : victim(wanted, held_n, -1);
      if (v < 0) break;
      const uint32_t e = (uint32_t)slot_[v].id;
      moved(layer_of(e));
      --held_n[layer_of(e)];
      where_[e] = -1;
      slot_[v].id = -1;
      slot_[v].draining = true;
      slot_[v].hold.reset();
      out.push_back({e, v, false, (int64_t)e});
    }
    return out;
  }
  // A draining slot returns to service.
  void drained(size_t slot) {
    if (slot >= slot_.size() || !slot_[slot].draining || slot_[slot].id >= 0)
      throw PoolError(-3, "drained requires a draining slot");
    slot_[slot].draining = false;
  }

  // The other tier of a two-tier pair (same id space); host: this pool is the host (RAM) tier.
  void peer(const ExpertPool *p, bool host) {
    if (p && p->n_ids_ != n_ids_) throw PoolError(-4, "peer pools must share the expert id space");
    peer_ = p;
    host_ = host;
    mark_all();
  }
  void exclusive(bool on) {
    exclusive_ = on;
    mark_all();
  }
  void decay_interval(uint32_t d) {
    decay_ = d;
    mark_all();
  }
  void fast_minima(bool on) {
    fast_ = on;
    mark_all();
  }
  // Turns target layer l (l < 40: the drafter's layers 40.. of the reference's space never
  // switch) late, once; a VRAM pool unpins the layer's VRAM pins and adds one budget slot each.
  void switch_target_layer(const PoolPolicy &p, uint32_t l) {
    if (l >= kTargetLayers || l >= per_layer_.size() || late_[l]) return;
    late_[l] = 1;
    dirty_[l] = 1;
    if (!host_)
      for (auto id : p.pins)
        if (id < n_ids_ && layer_of(id) == l) {
          unpin(id);
          ++budget_[l];
        }
    any_budget_ = false;
    for (auto b : budget_) any_budget_ |= b != 0;
  }
  bool late(uint32_t l) const { return l < late_.size() && late_[l]; }
  // The victim-order count of a resident expert: its LFU count adjusted by the peer's residency.
  uint64_t score(uint32_t id) const {
    uint64_t f = count_[id];
    if (!peer_) return f;
    const bool peer_has = peer_->where_[id] >= 0;
    if (exclusive_ && host_ && peer_has) return 0;
    if (late_[layer_of(id)]) {
      if (host_) {
        if (peer_has) f >>= 1;
      } else if (!peer_has) {
        f <<= 1;
      }
    }
    return f;
  }

  static constexpr uint32_t kTargetLayers = 40;

 private:
  struct Slot {
    int64_t id = -1;
    uint32_t leases = 0;
    bool pinned = false;
    bool draining = false;                // no occupant, not allocatable until drained()
    uint64_t stamp = 0;
    std::shared_ptr<const uint32_t> hold;  // the occupant's token; held while callers keep copies
  };
  static bool retained(const Slot &s) { return s.hold.use_count() > 1; }
  using RetainEpochs = std::vector<std::atomic<uint64_t>>;
  void mark_all() { std::fill(dirty_.begin(), dirty_.end(), (char)1); }
  // A slot of layer l gained or lost an occupant.
  void moved(uint32_t l) {
    dirty_[l] = 1;
    ++epoch_[l];
  }
  // fast_minima's victim: the per-layer cached least slots (rebuilt where stale), then the same
  // cross-layer choice as victim(): over-budget layers first, then (score, stamp, slot).
  int fast_victim(const std::unordered_set<uint32_t> &wanted, const std::vector<size_t> &held_n) {
    const uint32_t L = (uint32_t)per_layer_.size();
    for (uint32_t l = 0; l < L; ++l) {
      const uint64_t ret = (*ret_epoch_)[l].load(std::memory_order_acquire);
      const bool peer_moved = (late_[l] || exclusive_) && peer_ && peer_seen_[l] != peer_->epoch_[l];
      if (!dirty_[l] && !peer_moved && ret == ret_seen_[l]) continue;
      int any = -1, old = -1;
      for (uint32_t e = first_[l]; e < first_[l + 1]; ++e) {
        const int j = where_[e];
        if (j < 0) continue;
        const Slot &c = slot_[j];
        if (c.pinned || c.leases || retained(c) || wanted.count(e)) continue;
        if (any < 0 || before(j, any)) any = j;
        if (recent_ && last_[e] && last_[e] + recent_ >= tick_[l]) continue;
        if (old < 0 || before(j, old)) old = j;
      }
      best_any_[l] = any;
      best_old_[l] = old;
      dirty_[l] = 0;
      ret_seen_[l] = ret;
      if (peer_) peer_seen_[l] = peer_->epoch_[l];
    }
    for (int pass = 0; pass < 2; ++pass) {
      int best = -1;
      bool best_over = false;
      for (uint32_t l = 0; l < L; ++l) {
        const int j = pass ? best_any_[l] : best_old_[l];
        if (j < 0) continue;
        const bool over = any_budget_ && held_n[l] > budget_[l];
        if (best < 0 || (over && !best_over) || (over == best_over && before(j, best))) {
          best = j;
          best_over = over;
        }
      }
      if (best >= 0) return best;
    }
    return -1;
  }

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
  // Victim: lexicographic minimum of (within budget, score, stamp, slot) over
  // the evictable slots, first excluding those used in the recent window.
  int victim(const std::unordered_set<uint32_t> &wanted, const std::vector<size_t> &held, int want_layer) const {
    for (int pass = 0; pass < 2; ++pass) {
      int best = -1;
      bool best_in = true;
      for (size_t s = 0; s < slot_.size(); ++s) {
        const Slot &c = slot_[s];
        if (c.id < 0 || c.pinned || c.leases || retained(c) || wanted.count((uint32_t)c.id)) continue;
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
    const uint64_t ca = score((uint32_t)slot_[a].id), cb = score((uint32_t)slot_[b].id);
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
  const ExpertPool *peer_ = nullptr;
  bool host_ = false, exclusive_ = false, fast_ = false;
  std::vector<char> late_;
  // fast minima: per-layer cache and what invalidates it
  std::vector<char> dirty_;
  std::vector<int> best_any_, best_old_;
  std::vector<uint64_t> epoch_, peer_seen_, ret_seen_;
  std::shared_ptr<RetainEpochs> ret_epoch_;
};

// Width-one, token-major controller over a VRAM pool and its host peer (DriftPolicy): the
// caller brackets each target layer's demand with before()/after() in layer order 0..39 of
// every token. after() counts the token's distinct ids that are VRAM pins; over a window of the
// last 128 complete tokens, a pinned hit rate below one half, seen at the start of a token,
// turns every target layer of both pools late (once). Layers from 40 on are ignored.
class DriftControl {
 public:
  DriftControl(const PoolPolicy &p, ExpertPool &vram, ExpertPool &ram) : p_(p), vram_(vram), ram_(ram) {
    if (p.hard || !p.distinct || p.recent != 2 || p.decay != 256)
      throw PoolError(-4, "drift-0-50 requires soft recent2 distinct decay256");
    pinned_.assign(vram.ids(), 0);
    for (auto e : p.pins) {
      if (e >= vram.ids()) throw PoolError(-2, "expert id");
      pinned_[e] = 1;
    }
    vram_.peer(&ram_, false);
    ram_.peer(&vram_, true);
  }
  void before(const std::vector<uint32_t> &ids) {
    const uint32_t l = one_layer(ids);
    if (l >= ExpertPool::kTargetLayers) return;
    if (open_ || l != next_) throw PoolError(-4, "drift requires complete width-one token-major traversal");
    if (l == 0 && !active_ && window_.size() == kWindow && requests_ && 2 * hits_ < requests_) {
      const uint32_t n = std::min<uint32_t>(ExpertPool::kTargetLayers, (uint32_t)vram_.layers());
      for (uint32_t t = 0; t < n; ++t) {
        vram_.switch_target_layer(p_, t);
        ram_.switch_target_layer(p_, t);
      }
      active_ = true;
    }
    open_ = true;
  }
  void after(const std::vector<uint32_t> &ids) {
    if (ids.empty()) throw PoolError(-4, "empty drift demand");
    // an id past the space names no target layer (as a drafter layer's does): nothing to count
    if (ids.front() >= vram_.ids()) return;
    const uint32_t l = vram_.layer_of(ids.front());
    if (l >= ExpertPool::kTargetLayers) return;
    if (!open_ || l != next_) throw PoolError(-3, "unpaired drift completion");
    std::unordered_set<uint32_t> seen;
    for (auto e : ids) {
      check(e);
      if (seen.insert(e).second) {
        ++tok_requests_;
        tok_hits_ += pinned_[e];
      }
    }
    open_ = false;
    const uint32_t n = std::min<uint32_t>(ExpertPool::kTargetLayers, (uint32_t)vram_.layers());
    if (++next_ < n) return;
    next_ = 0;
    ++tokens_;
    window_.push_back({tok_hits_, tok_requests_});
    hits_ += tok_hits_;
    requests_ += tok_requests_;
    tok_hits_ = tok_requests_ = 0;
    if (window_.size() > kWindow) {
      hits_ -= window_.front().first;
      requests_ -= window_.front().second;
      window_.pop_front();
    }
  }
  bool active() const { return active_; }
  uint64_t completed_tokens() const { return tokens_; }

 private:
  static constexpr size_t kWindow = 128;
  uint32_t check(uint32_t e) const {
    if (e >= vram_.ids()) throw PoolError(-4, "drift demand must represent one layer");
    return e;
  }
  uint32_t one_layer(const std::vector<uint32_t> &ids) const {
    if (ids.empty()) throw PoolError(-4, "empty drift demand");
    const uint32_t l = vram_.layer_of(check(ids.front()));
    for (auto e : ids)
      if (vram_.layer_of(check(e)) != l) throw PoolError(-4, "drift demand must represent one layer");
    return l;
  }
  PoolPolicy p_;
  ExpertPool &vram_, &ram_;
  std::vector<char> pinned_;
  std::deque<std::pair<uint64_t, uint64_t>> window_;
  uint64_t hits_ = 0, requests_ = 0, tok_hits_ = 0, tok_requests_ = 0, tokens_ = 0;
  uint32_t next_ = 0;
  bool active_ = false, open_ = false;
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
