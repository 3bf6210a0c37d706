// Host-side expert slot pool: which expert occupies which HBM slot, under the
// deterministic LFU residency policy of the reference's VRAM slot pool
// (components/moe/include/ds41/store.hpp:80-157, components/moe/src/store.cpp:15-219),
// the drift controller that switches the pool pair to its late-layer rules
// (store.hpp:161-178, store.cpp:220-255), and the text placement format that
// configures both (components/moe/src/manifest.cpp:8-34).
//
// Expert ids are flattened layer by layer (layer l owns ids base(l) ..
// base(l) + size(l) - 1), which covers the reference's 40 x 384 target + 3 x 128
// drafter space and the verify stack's L x E space.
//
// The policy, as this pool states it:
// - Demand. Every demand (an acquire that is not a prefetch, or a touch) ticks
//   the clock of each layer it names once, in ascending layer order; a layer
//   whose clock reaches a multiple of its decay interval halves the use counts
//   of all its experts, and only then are the demand's uses counted (once per
//   distinct id, or once per occurrence in multiplicity mode).
// - Placement. A miss takes the lowest-index empty slot (of its own layer's
//   slots under hard budgets); with none free it evicts the slot with the
//   smallest victim key among the evictable ones (occupied, not pinned, leased,
//   retained or wanted by the same call). The key is, in order: used within the
//   last `recent` ticks of its layer (those go last), its layer within its
//   soft budget (over-budget layers go first), its score (the use count,
//   adjusted by a peer pool's residency for late or exclusive layers), the
//   stamp of its last grant, and the slot index.
// - A call is rejected whole, before any change, when its distinct ids exceed
//   the slots it could use.
// - Retention tokens (retain): while any copy of a token of a slot's current
//   occupant lives, the slot is neither evicted nor counted as usable.
// - Draining (reserve/drained): policy victims become empty, unallocatable
//   slots until the idle slots reach a target; drained() returns one.
// - Peer pools and late layers: a VRAM/RAM pair sees each other's residency;
//   an exclusive host pool scores experts the VRAM peer holds 0; in a late
//   layer a host pool halves the score of experts its peer holds and a VRAM pool
//   doubles the score of experts its peer lacks, and the layer decays every 512
//   (VRAM) or 128 (host) of its ticks; turning a target layer late releases the
//   VRAM pool's pins of that layer into its budget.
// - Victim memo (fast_minima, distinct counting, soft budgets): each layer
//   keeps its least evictable slot from the last time it was examined and is
//   re-examined only after something that can change it (its residency, a
//   lease, pin, count or stamp of it, a retention token of it, or, for a late
//   or exclusive layer, the peer's residency of it). reserve() does not mark
//   the layers of its wanted set, so a memo made under that set can keep
//   skipping those experts until the layer changes; decisions stay equal to the
//   reference pool's, which behaves the same way.
#pragma once
#include <algorithm>
#include <atomic>
#include <cstdint>
#include <deque>
#include <istream>
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
  static constexpr uint32_t kTargetLayers = 40;  // layers from 40 on (the drafter's) never turn late

  ExpertPool(size_t slots, std::vector<uint32_t> layer_experts, uint32_t recent = 6, uint32_t decay = 32,
             bool distinct = true)
      : slot_(slots), recent_(recent), decay_(decay), distinct_(distinct) {
    if (slots == 0) throw PoolError(-4, "a pool needs at least one slot");
    if (layer_experts.empty()) throw PoolError(-4, "a pool needs at least one layer");
    layer_.resize(layer_experts.size());
    uint32_t base = 0;
    for (size_t l = 0; l < layer_.size(); ++l) {
      layer_[l].base = base;
      layer_[l].size = layer_experts[l];
      base += layer_experts[l];
    }
    expert_.resize(base);
    for (uint32_t l = 0; l < layer_.size(); ++l)
      for (uint32_t i = 0; i < layer_[l].size; ++i) expert_[layer_[l].base + i].layer = l;
    token_events_ = std::make_shared<TokenEvents>(layer_.size());
    for (auto &c : *token_events_) c.store(0);
  }

  size_t slots() const { return slot_.size(); }
  uint32_t ids() const { return (uint32_t)expert_.size(); }
  size_t layers() const { return layer_.size(); }
  uint32_t layer_of(uint32_t id) const { return expert_[id].layer; }
  uint32_t first_of(uint32_t layer) const { return layer_[layer].base; }
  int residency(uint32_t id) const { return id < ids() ? expert_[id].slot : -1; }
  uint32_t frequency(uint32_t id) const { return id < ids() ? expert_[id].uses : 0; }
  bool late(uint32_t l) const { return l < layer_.size() && layer_[l].late; }

  void policy(const PoolPolicy &p) {
    forget_all_memos();
    recent_ = p.recent;
    decay_ = p.decay;
    distinct_ = p.distinct;
    for (size_t l = 0; l < layer_.size(); ++l) layer_[l].budget = l < p.budget.size() ? p.budget[l] : 0;
    refresh_budgets();
    hard_ = p.hard;
    owner_.clear();
    if (!hard_) return;
    // hard budgets deal the slots out in layer order: each layer's pins, then its budget
    std::vector<uint32_t> pinned(layer_.size(), 0);
    for (uint32_t id : p.pins) ++pinned[layer_of(valid(id))];
    for (uint32_t l = 0; l < layer_.size(); ++l) owner_.insert(owner_.end(), pinned[l] + layer_[l].budget, l);
    if (owner_.size() != slot_.size())
      throw PoolError(-4, "hard budgets plus pins deal " + std::to_string(owner_.size()) + " slots to a pool of " +
                              std::to_string(slot_.size()));
    for (size_t s = 0; s < slot_.size(); ++s)
      if (slot_[s].expert >= 0 && layer_of((uint32_t)slot_[s].expert) != owner_[s])
        throw PoolError(-3, "slot " + std::to_string(s) + " holds an expert of another layer than hard budgets give it");
  }

  void reset_history() {
    forget_all_memos();
    for (auto &x : expert_) {
      x.uses = 0;
      x.last_tick = 0;
    }
    for (auto &y : layer_) y.ticks = 0;
  }

  void touch(const std::vector<uint32_t> &ids) {
    for (uint32_t e : ids) valid(e);
    demand(ids, first_occurrences(ids));
  }

  std::vector<Alloc> acquire(const std::vector<uint32_t> &input, bool prefetch = false) {
    for (uint32_t e : input) valid(e);
    const std::vector<uint32_t> want = first_occurrences(input);
    const std::unordered_set<uint32_t> wanted(want.begin(), want.end());
    check_capacity(want, wanted);
    for (uint32_t e : want) forget_memo(layer_of(e));
    if (!prefetch) demand(input, want);
    std::vector<size_t> held = held_per_layer();
    std::vector<Alloc> out;
    out.reserve(want.size());
    for (uint32_t e : want) {
      Alloc a{e, expert_[e].slot, expert_[e].slot >= 0, -1};
      if (!a.hit) {
        a.slot = free_slot(hard_ ? (int)layer_of(e) : -1);
        if (a.slot < 0) a.slot = memo_usable() ? memo_victim(wanted, held) : lowest_key_slot(wanted, held, hard_ ? (int)layer_of(e) : -1);
        if (a.slot < 0) throw PoolError(-3, "no victim although the capacity check passed");
        a.evicted = slot_[a.slot].expert;
        if (a.evicted >= 0) {
          vacate(a.slot);
          --held[layer_of((uint32_t)a.evicted)];
        }
        occupy(a.slot, e);
        ++held[layer_of(e)];
      }
      Slot &s = slot_[a.slot];
      forget_memo(layer_of(e));
      ++s.leases;
      s.grant = ++grants_;
      out.push_back(a);
    }
    return out;
  }

  // Leases on the experts already resident (no clock moves, no stamps).
  std::vector<Alloc> borrow(const std::vector<uint32_t> &ids) {
    for (uint32_t e : ids) valid(e);
    std::vector<Alloc> out;
    for (uint32_t e : first_occurrences(ids))
      if (expert_[e].slot >= 0) out.push_back({e, expert_[e].slot, true, -1});
    for (const Alloc &a : out) {
      ++slot_[a.slot].leases;
      forget_memo(layer_of(a.id));
    }
    return out;
  }

  void release(const std::vector<Alloc> &lease) {
    std::vector<uint32_t> taken(slot_.size(), 0);
    for (const Alloc &a : lease) {
      const bool ok = a.slot >= 0 && (size_t)a.slot < slot_.size() && slot_[a.slot].expert == (int64_t)a.id &&
                      ++taken[a.slot] <= slot_[a.slot].leases;
      if (!ok) throw PoolError(-3, "release of a lease the pool does not hold (slot " + std::to_string(a.slot) + ")");
    }
    for (const Alloc &a : lease) {
      --slot_[a.slot].leases;
      forget_memo(layer_of(a.id));
    }
  }

  void pin(uint32_t id) {
    const int s = residency(id);
    if (s < 0) throw PoolError(-3, "only a resident expert can be pinned");
    slot_[s].pinned = true;
    forget_memo(layer_of(id));
  }
  void unpin(uint32_t id) {  // a non-resident (or unknown) id is left alone
    const int s = residency(id);
    if (s < 0) return;
    slot_[s].pinned = false;
    forget_memo(layer_of(id));
  }

  // A token of the slot's current occupant, kept by the slot while any copy of it lives (it is
  // never evicted or reserved meanwhile). Dropping a copy is thread-safe and never touches the
  // pool, which may already be gone. With the victim memo on, taking the token and dropping its
  // last copy both count as events of the layer, so its memo is made again.
  std::shared_ptr<const void> retain(uint32_t id) const {
    const int s = residency(valid(id));
    if (s < 0) throw PoolError(-3, "only a resident expert can be retained");
    if (!memo_) return slot_[s].token;
    std::shared_ptr<TokenEvents> events = token_events_;
    const uint32_t l = layer_of(id);
    std::shared_ptr<const uint32_t> token = slot_[s].token;
    const void *addr = token.get();
    (*events)[l].fetch_add(1, std::memory_order_release);
    return std::shared_ptr<const void>(addr, [token, events, l](const void *) mutable {
      token.reset();
      (*events)[l].fetch_add(1, std::memory_order_release);
    });
  }

  // Moves policy victims (never wanted, pinned, leased or retained) into draining slots until the
  // idle (empty or draining) slots number `target`, or no victim is left; one allocation per
  // victim (slot, evicted = its expert). No clock moves.
  std::vector<Alloc> reserve(size_t target, const std::unordered_set<uint32_t> &wanted) {
    if (hard_) throw PoolError(-3, "draining needs soft budgets");
    size_t idle = 0;
    for (const Slot &s : slot_) idle += s.expert < 0;
    std::vector<Alloc> out;
    if (idle >= target) return out;
    std::vector<size_t> held = held_per_layer();
    for (; idle < target; ++idle) {
      const int v = memo_ && distinct_ ? memo_victim(wanted, held) : lowest_key_slot(wanted, held, -1);
      if (v < 0) break;
      const uint32_t e = (uint32_t)slot_[v].expert;
      vacate(v);
      --held[layer_of(e)];
      slot_[v].draining = true;
      out.push_back({e, v, false, (int64_t)e});
    }
    return out;
  }
  void drained(size_t slot) {
    if (slot >= slot_.size() || !slot_[slot].draining || slot_[slot].expert >= 0)
      throw PoolError(-3, "slot " + std::to_string(slot) + " is not draining");
    slot_[slot].draining = false;
  }

  // The other tier of a two-tier pair (same id space); host: this pool is the host (RAM) tier.
  void peer(const ExpertPool *p, bool host) {
    if (p && p->ids() != ids()) throw PoolError(-4, "a peer pool must cover the same expert ids");
    peer_ = p;
    host_ = host;
    forget_all_memos();
  }
  void exclusive(bool on) {
    exclusive_ = on;
    forget_all_memos();
  }
  void decay_interval(uint32_t d) {
    decay_ = d;
    forget_all_memos();
  }
  void fast_minima(bool on) {
    memo_ = on;
    forget_all_memos();
  }
  // Turns target layer l late, once; a VRAM pool unpins the layer's VRAM pins and adds one budget
  // slot for each.
  void switch_target_layer(const PoolPolicy &p, uint32_t l) {
    if (l >= kTargetLayers || l >= layer_.size() || layer_[l].late) return;
    layer_[l].late = true;
    forget_memo(l);
    if (!host_)
      for (uint32_t id : p.pins)
        if (id < ids() && layer_of(id) == l) {
          unpin(id);
          ++layer_[l].budget;
        }
    refresh_budgets();
  }
  // The score in the victim order: the use count, adjusted by the peer's residency.
  uint64_t score(uint32_t id) const {
    const uint64_t uses = expert_[id].uses;
    if (!peer_) return uses;
    const bool peer_holds = peer_->expert_[id].slot >= 0;
    if (exclusive_ && host_ && peer_holds) return 0;
    if (!layer_[layer_of(id)].late) return uses;
    if (host_) return peer_holds ? uses >> 1 : uses;
    return peer_holds ? uses : uses << 1;
  }

 private:
  struct Slot {
    int64_t expert = -1;
    uint32_t leases = 0;
    bool pinned = false, draining = false;
    uint64_t grant = 0;                     // stamp of the last grant (acquire)
    std::shared_ptr<const uint32_t> token;  // the occupant's retention token
  };
  struct Layer {
    uint32_t base = 0, size = 0;
    uint64_t ticks = 0;  // demands that named the layer
    uint32_t budget = 0;
    bool late = false;
    uint64_t moves = 0;  // occupants gained or lost (what a peer's memo watches)
    // victim memo: the layer's least evictable slot when last examined (-1 none)
    bool memo_stale = true;
    int memo_slot = -1;
    bool memo_recent = false;
    uint64_t seen_peer_moves = 0, seen_token_events = 0;
  };
  struct Expert {
    int32_t slot = -1;
    uint32_t uses = 0;
    uint64_t last_tick = 0;  // the layer's tick of its last demand (0: never)
    uint32_t layer = 0;
  };
  using TokenEvents = std::vector<std::atomic<uint64_t>>;
  // The order of eviction: the smaller key goes first.
  struct VictimKey {
    bool recent, in_budget;
    uint64_t score, grant;
    int slot;
    bool operator<(const VictimKey &o) const {
      if (recent != o.recent) return !recent;
      if (in_budget != o.in_budget) return !in_budget;
      if (score != o.score) return score < o.score;
      if (grant != o.grant) return grant < o.grant;
      return slot < o.slot;
    }
  };

  uint32_t valid(uint32_t id) const {
    if (id >= ids()) throw PoolError(-2, "expert id " + std::to_string(id) + " is outside the pool's id space");
    return id;
  }
  static std::vector<uint32_t> first_occurrences(const std::vector<uint32_t> &ids) {
    std::vector<uint32_t> u;
    std::unordered_set<uint32_t> seen;
    for (uint32_t e : ids)
      if (seen.insert(e).second) u.push_back(e);
    return u;
  }
  static bool retained(const Slot &s) { return s.token.use_count() > 1; }
  bool memo_usable() const { return memo_ && distinct_ && !hard_; }
  void forget_memo(uint32_t l) { layer_[l].memo_stale = true; }
  void forget_all_memos() {
    for (auto &y : layer_) y.memo_stale = true;
  }
  void refresh_budgets() {
    any_budget_ = false;
    for (const auto &y : layer_) any_budget_ |= y.budget != 0;
  }
  bool recent(uint32_t id) const {
    const Expert &x = expert_[id];
    return recent_ && x.last_tick && x.last_tick + recent_ >= layer_[x.layer].ticks;
  }
  bool over_budget(uint32_t l, const std::vector<size_t> &held) const {
    return any_budget_ && held[l] > layer_[l].budget;
  }
  // A slot a call may take: free (not draining), or its occupant is wanted by the call, or it is
  // neither pinned, leased nor retained.
  bool usable(const Slot &s, const std::unordered_set<uint32_t> &wanted) const {
    if (s.draining) return false;
    return s.expert < 0 || wanted.count((uint32_t)s.expert) || (!s.pinned && !s.leases && !retained(s));
  }
  bool evictable(const Slot &s, const std::unordered_set<uint32_t> &wanted) const {
    return s.expert >= 0 && !s.pinned && !s.leases && !retained(s) && !wanted.count((uint32_t)s.expert);
  }
  void check_capacity(const std::vector<uint32_t> &want, const std::unordered_set<uint32_t> &wanted) const {
    if (hard_) {
      std::vector<size_t> need(layer_.size(), 0), room(layer_.size(), 0);
      for (uint32_t e : want) ++need[layer_of(e)];
      for (size_t s = 0; s < slot_.size(); ++s) room[owner_[s]] += usable(slot_[s], wanted);
      for (size_t l = 0; l < layer_.size(); ++l)
        if (need[l] > room[l])
          throw PoolError(-1, "layer " + std::to_string(l) + " needs " + std::to_string(need[l]) +
                                  " slots, its hard budget leaves " + std::to_string(room[l]));
    }
    size_t room = 0;
    for (const Slot &s : slot_) room += usable(s, wanted);
    if (want.size() > room)
      throw PoolError(-1, "the call needs " + std::to_string(want.size()) + " slots, " + std::to_string(room) +
                              " are usable");
  }
  // One demand: ticks the named layers (decay first), then counts the uses.
  void demand(const std::vector<uint32_t> &ids, const std::vector<uint32_t> &distinct_ids) {
    std::vector<char> named(layer_.size(), 0);
    for (uint32_t e : distinct_ids) named[layer_of(e)] = 1;
    for (uint32_t l = 0; l < layer_.size(); ++l) {
      if (!named[l]) continue;
      Layer &y = layer_[l];
      forget_memo(l);
      const uint64_t t = ++y.ticks;
      const uint32_t interval = y.late ? (host_ ? 128u : 512u) : decay_;
      if (interval && t % interval == 0)
        for (uint32_t i = 0; i < y.size; ++i) expert_[y.base + i].uses >>= 1;
    }
    for (uint32_t e : distinct_ ? distinct_ids : ids) {
      Expert &x = expert_[e];
      if (x.uses != UINT32_MAX) ++x.uses;
      x.last_tick = layer_[x.layer].ticks;
    }
  }
  std::vector<size_t> held_per_layer() const {  // occupied, unpinned slots per layer
    std::vector<size_t> held(layer_.size(), 0);
    for (const Slot &s : slot_)
      if (s.expert >= 0 && !s.pinned) ++held[layer_of((uint32_t)s.expert)];
    return held;
  }
  int free_slot(int only_layer) const {
    for (size_t s = 0; s < slot_.size(); ++s)
      if (slot_[s].expert < 0 && !slot_[s].draining && (only_layer < 0 || owner_[s] == (uint32_t)only_layer))
        return (int)s;
    return -1;
  }
  void vacate(int s) {
    const uint32_t e = (uint32_t)slot_[s].expert;
    Layer &y = layer_[layer_of(e)];
    forget_memo(layer_of(e));
    ++y.moves;
    expert_[e].slot = -1;
    slot_[s].expert = -1;
    slot_[s].token.reset();
  }
  void occupy(int s, uint32_t e) {
    Layer &y = layer_[layer_of(e)];
    forget_memo(layer_of(e));
    ++y.moves;
    expert_[e].slot = s;
    slot_[s].expert = e;
    slot_[s].token = std::make_shared<const uint32_t>(e);  // earlier occupants' tokens no longer bind
  }
  VictimKey key_of(int s, bool in_budget) const {
    const uint32_t e = (uint32_t)slot_[s].expert;
    return VictimKey{recent(e), in_budget, score(e), slot_[s].grant, s};
  }
  // Every evictable slot (of one layer's dealt slots under hard budgets), smallest key.
  int lowest_key_slot(const std::unordered_set<uint32_t> &wanted, const std::vector<size_t> &held, int only_layer) const {
    int best = -1;
    VictimKey best_key{};
    for (size_t s = 0; s < slot_.size(); ++s) {
      const Slot &c = slot_[s];
      if (!evictable(c, wanted) || (only_layer >= 0 && owner_[s] != (uint32_t)only_layer)) continue;
      const VictimKey k = key_of((int)s, !over_budget(layer_of((uint32_t)c.expert), held));
      if (best < 0 || k < best_key) {
        best = (int)s;
        best_key = k;
      }
    }
    return best;
  }
  // The same choice from the layers' memos, each re-made first where something may have changed.
  int memo_victim(const std::unordered_set<uint32_t> &wanted, const std::vector<size_t> &held) {
    int best = -1;
    VictimKey best_key{};
    for (uint32_t l = 0; l < layer_.size(); ++l) {
      Layer &y = layer_[l];
      const uint64_t tokens = (*token_events_)[l].load(std::memory_order_acquire);
      const bool peer_moved = peer_ && (y.late || exclusive_) && y.seen_peer_moves != peer_->layer_[l].moves;
      if (y.memo_stale || peer_moved || tokens != y.seen_token_events) {
        int pick = -1;
        VictimKey pick_key{};
        for (uint32_t i = 0; i < y.size; ++i) {  // the layer's experts in id order
          const int s = expert_[y.base + i].slot;
          if (s < 0 || !evictable(slot_[s], wanted)) continue;
          const VictimKey k = key_of(s, true);
          if (pick < 0 || k < pick_key) {
            pick = s;
            pick_key = k;
          }
        }
        y.memo_slot = pick;
        y.memo_recent = pick >= 0 && pick_key.recent;
        y.memo_stale = false;
        y.seen_token_events = tokens;
        if (peer_) y.seen_peer_moves = peer_->layer_[l].moves;
      }
      if (y.memo_slot < 0) continue;
      VictimKey k = key_of(y.memo_slot, !over_budget(l, held));
      k.recent = y.memo_recent;  // the memo's standing, as it was made
      if (best < 0 || k < best_key) {
        best = y.memo_slot;
        best_key = k;
      }
    }
    return best;
  }

  std::vector<Slot> slot_;
  std::vector<Layer> layer_;
  std::vector<Expert> expert_;
  std::vector<uint32_t> owner_;  // hard budgets: the layer each slot is dealt to
  uint32_t recent_, decay_;
  bool distinct_, hard_ = false, any_budget_ = false, memo_ = false;
  uint64_t grants_ = 0;
  const ExpertPool *peer_ = nullptr;
  bool host_ = false, exclusive_ = false;
  std::shared_ptr<TokenEvents> token_events_;
};

// The drift controller over a VRAM pool and its RAM peer: each target layer's demand of a token
// is bracketed by before()/after(), layers 0..39 in order, one token at a time. after() counts the
// demand's distinct ids and how many of them are VRAM pins; once the last 128 complete tokens show
// pins serving less than half of their requests, the next token's first before() turns every
// target layer of both pools late (once). Demands of layers from 40 on are not counted.
class DriftControl {
 public:
  DriftControl(const PoolPolicy &p, ExpertPool &vram, ExpertPool &ram) : policy_(p), vram_(vram), ram_(ram) {
    if (p.hard || !p.distinct || p.recent != 2 || p.decay != 256)
      throw PoolError(-4, "the drift controller runs soft budgets, distinct counting, recent 2 and decay 256");
    is_pin_.assign(vram.ids(), 0);
    for (uint32_t e : p.pins) {
      if (e >= vram.ids()) throw PoolError(-2, "pin " + std::to_string(e) + " is outside the id space");
      is_pin_[e] = 1;
    }
    vram_.peer(&ram_, false);
    ram_.peer(&vram_, true);
  }
  void before(const std::vector<uint32_t> &ids) {
    const uint32_t l = demand_layer(ids);
    if (l >= ExpertPool::kTargetLayers) return;
    if (open_ || l != next_)
      throw PoolError(-4, "layer " + std::to_string(l) + " out of turn (expected " + std::to_string(next_) + ")");
    if (l == 0 && !switched_ && history_.size() == kWindow && asked_ && 2 * served_ < asked_) {
      const uint32_t n = std::min<uint32_t>(ExpertPool::kTargetLayers, (uint32_t)vram_.layers());
      for (uint32_t t = 0; t < n; ++t) {
        vram_.switch_target_layer(policy_, t);
        ram_.switch_target_layer(policy_, t);
      }
      switched_ = true;
    }
    open_ = true;
  }
  void after(const std::vector<uint32_t> &ids) {
    if (ids.empty()) throw PoolError(-4, "a demand names at least one expert");
    if (ids.front() >= vram_.ids()) return;  // names no target layer (as a drafter layer's ids)
    const uint32_t l = vram_.layer_of(ids.front());
    if (l >= ExpertPool::kTargetLayers) return;
    if (!open_ || l != next_) throw PoolError(-3, "after() without its before() for layer " + std::to_string(l));
    std::unordered_set<uint32_t> seen;
    for (uint32_t e : ids) {
      if (e >= vram_.ids()) throw PoolError(-4, "a demand's ids must lie in one layer");
      if (!seen.insert(e).second) continue;
      ++token_asked_;
      token_served_ += is_pin_[e];
    }
    open_ = false;
    const uint32_t n = std::min<uint32_t>(ExpertPool::kTargetLayers, (uint32_t)vram_.layers());
    if (++next_ < n) return;
    next_ = 0;
    ++tokens_;
    history_.push_back({token_served_, token_asked_});
    served_ += token_served_;
    asked_ += token_asked_;
    token_served_ = token_asked_ = 0;
    if (history_.size() > kWindow) {
      served_ -= history_.front().first;
      asked_ -= history_.front().second;
      history_.pop_front();
    }
  }
  bool active() const { return switched_; }
  uint64_t completed_tokens() const { return tokens_; }

 private:
  static constexpr size_t kWindow = 128;
  uint32_t demand_layer(const std::vector<uint32_t> &ids) const {
    if (ids.empty()) throw PoolError(-4, "a demand names at least one expert");
    uint32_t l = 0;
    for (size_t i = 0; i < ids.size(); ++i) {
      if (ids[i] >= vram_.ids()) throw PoolError(-4, "a demand's ids must lie in one layer");
      const uint32_t li = vram_.layer_of(ids[i]);
      if (i && li != l) throw PoolError(-4, "a demand's ids must lie in one layer");
      l = li;
    }
    return l;
  }
  PoolPolicy policy_;
  ExpertPool &vram_, &ram_;
  std::vector<char> is_pin_;
  std::deque<std::pair<uint64_t, uint64_t>> history_;  // per complete token: (pinned ids, ids)
  uint64_t served_ = 0, asked_ = 0, token_served_ = 0, token_asked_ = 0, tokens_ = 0;
  uint32_t next_ = 0;
  bool switched_ = false, open_ = false;
};

// Placement text (the reference's profiles/*.placement). One directive per line; blank lines and
// lines starting with '#' are skipped; every directive takes exactly its operands (plain decimal
// numbers):
//   vram <id> | host <id>            an expert pinned in VRAM / resident in RAM (each id once
//                                    over both lists)
//   pools hard|soft                  budget <layer> <n> | host_budget <layer> <n>  (n <= layer size)
//   recent <n> | decay <n>           (n < 2^32)
//   lfu distinct|multiplicity
inline PoolPolicy parse_placement(std::istream &in, const std::vector<uint32_t> &layer_experts) {
  uint64_t total = 0;
  for (uint32_t n : layer_experts) total += n;
  PoolPolicy p;
  p.budget.assign(layer_experts.size(), 0);
  p.host_budget.assign(layer_experts.size(), 0);
  std::unordered_set<uint64_t> listed;
  std::string line;
  uint64_t lineno = 0;
  const auto fail = [&](const std::string &why) {
    throw PoolError(-4, "placement line " + std::to_string(lineno) + ": " + why);
  };
  const auto number = [&](const std::string &tok, uint64_t limit) {
    if (tok.empty() || tok.size() > 20 || tok.find_first_not_of("0123456789") != std::string::npos)
      fail("'" + tok + "' is not a decimal number");
    const unsigned long long v = std::stoull(tok);
    if (v > limit) fail(tok + " exceeds " + std::to_string(limit));
    return (uint64_t)v;
  };
  while (std::getline(in, line)) {
    ++lineno;
    if (line.empty() || line[0] == '#') continue;
    std::istringstream words(line);
    std::vector<std::string> tok;
    for (std::string w; words >> w;) tok.push_back(w);
    if (tok.empty()) fail("no directive");
    const std::string &op = tok[0];
    const size_t operands = op == "budget" || op == "host_budget" ? 2 : 1;
    if (tok.size() != operands + 1) fail("'" + op + "' takes " + std::to_string(operands) + " operand(s)");
    if (op == "vram" || op == "host") {
      if (total == 0) fail("no experts to place");
      const uint64_t id = number(tok[1], total - 1);
      if (!listed.insert(id).second) fail("expert " + tok[1] + " is placed twice");
      (op == "vram" ? p.pins : p.host).push_back((uint32_t)id);
    } else if (op == "pools") {
      if (tok[1] != "hard" && tok[1] != "soft") fail("pools are hard or soft");
      p.hard = tok[1] == "hard";
    } else if (op == "budget" || op == "host_budget") {
      if (layer_experts.empty()) fail("no layers");
      const uint64_t l = number(tok[1], layer_experts.size() - 1);
      const uint64_t n = number(tok[2], layer_experts[l]);
      (op == "budget" ? p.budget : p.host_budget)[l] = (uint32_t)n;
    } else if (op == "recent" || op == "decay") {
      (op == "recent" ? p.recent : p.decay) = (uint32_t)number(tok[1], UINT32_MAX);
    } else if (op == "lfu") {
      if (tok[1] != "distinct" && tok[1] != "multiplicity") fail("lfu counting is distinct or multiplicity");
      p.distinct = tok[1] == "distinct";
    } else {
      fail("unknown directive '" + op + "'");
    }
  }
  return p;
}

}  // namespace ds41g
