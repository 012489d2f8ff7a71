// Native slot-pool bookkeeping: the (layer, expert) -> slot table with
// sampled LFU/LRU eviction of engine_v3.ExpertPool, as host C++ so that the
// per-layer acquire/prefetch costs microseconds, not Python dict traffic.
//
// Semantics follow engine_v3.py step by step:
//   state ............ :214-226 (slot_of, key_of, freq, free, pending,
//                      from_prefetch, pinned, clock, born, last_use, use_clock)
//   protect window ... :310-311 (24 * max(1, depth), passed in as `window`)
//   _alloc ........... :313-374 (free list popped from the end; else the
//                      lowest score among >= 24 samples taken at stride 7919
//                      from a rotating start, skipping pinned/pending/empty;
//                      entries younger than the window score +2^30)
//   _touch ........... :376-380
//   prefetch ......... :383-396 (skip resident/pending; bail on exhaustion)
//   acquire .......... :398-454 (hits, demand misses, waits on pending
//                      prefetches: touched in the loop and again after the
//                      wait; pinned = this call's slots at the end)
//   stats ............ :456-464
// A prefetch "completes" when the caller says so (moe_policy_complete), the
// role of the worker epilogue at engine_v3.py:292-301.
#include <cstdint>
#include <cstring>
#include <new>
#include <vector>

#include "../../include/moe_stream.h"

namespace {

constexpr int kSample = 24;
constexpr int64_t kStride = 7919;
constexpr int64_t kYoung = int64_t(1) << 30;

}  // namespace

struct moe_policy {
  int32_t n_slots, n_layers, n_experts, evict, window;
  std::vector<int32_t> slot_of;     // key -> slot or -1
  std::vector<int32_t> key_of;      // slot -> key or -1
  std::vector<int64_t> freq, born, last_use;
  std::vector<uint8_t> resident_born;  // born[] valid
  std::vector<uint8_t> pending, from_prefetch;
  std::vector<uint8_t> pinned;      // per slot
  std::vector<int32_t> pinned_list;
  std::vector<int32_t> free_list;
  int64_t clock = 0, use_clock = 0;
  int64_t n_prefetch_hit = 0, n_cache_hit = 0, n_miss = 0;
  int64_t n_prefetch_bail = 0, n_prefetch_issued = 0;

  int32_t key(int32_t layer, int32_t expert) const { return layer * n_experts + expert; }

  void pin(int32_t slot) {
    if (!pinned[slot]) {
      pinned[slot] = 1;
      pinned_list.push_back(slot);
    }
  }
  void clear_pins() {
    for (int32_t s : pinned_list) pinned[s] = 0;
    pinned_list.clear();
  }

  // -1 when exhausted
  int32_t alloc(int32_t k) {
    clock += 1;
    int32_t slot;
    if (!free_list.empty()) {
      slot = free_list.back();
      free_list.pop_back();
    } else {
      int32_t victim = -1;
      int64_t best = 0;
      const int64_t n = n_slots;
      const int64_t start = clock % n;
      int seen = 0;
      for (int64_t j = 0; j < n; ++j) {
        const int32_t sidx = (int32_t)((start + j * kStride) % n);
        const int32_t kk = key_of[sidx];
        if (kk < 0 || pinned[sidx] || pending[kk]) continue;
        const bool young = clock - (resident_born[kk] ? born[kk] : 0) < window;
        int64_t base;
        if (evict == MOE_EVICT_ASIS) base = 0;
        else if (evict == MOE_EVICT_LRU) base = last_use[kk];
        else base = freq[kk];
        const int64_t f = base + (young ? kYoung : 0);
        if (victim < 0 || f < best) {
          best = f;
          victim = sidx;
        }
        ++seen;
        if (seen >= kSample && victim >= 0 && best < kYoung) break;
      }
      if (victim < 0) return -1;
      const int32_t vk = key_of[victim];
      from_prefetch[vk] = 0;
      resident_born[vk] = 0;
      born[vk] = 0;
      last_use[vk] = 0;
      freq[vk] = 0;
      slot_of[vk] = -1;
      slot = victim;
    }
    key_of[slot] = k;
    slot_of[k] = slot;
    born[k] = clock;
    resident_born[k] = 1;
    return slot;
  }

  void touch(int32_t k) {
    use_clock += 1;
    last_use[k] = use_clock;
    freq[k] += 1;
  }

  void cancel(int32_t k) {
    const int32_t slot = slot_of[k];
    pending[k] = 0;
    from_prefetch[k] = 0;
    resident_born[k] = 0;
    born[k] = 0;
    last_use[k] = 0;
    freq[k] = 0;
    slot_of[k] = -1;
    if (slot >= 0) {
      key_of[slot] = -1;
      free_list.push_back(slot);
    }
  }

  void complete(int32_t k) {
    if (pending[k]) {
      pending[k] = 0;
      from_prefetch[k] = 1;
    }
  }
};

namespace {
bool bad_key(const moe_policy *p, int32_t layer, int32_t expert) {
  return layer < 0 || layer >= p->n_layers || expert < 0 || expert >= p->n_experts;
}
}  // namespace

extern "C" {

int moe_policy_create(int32_t n_slots, int32_t n_layers, int32_t n_experts,
                      int32_t evict, int32_t window, moe_policy **out) {
  if (!out || n_slots <= 0 || n_layers <= 0 || n_experts <= 0 || window < 0 ||
      (evict != MOE_EVICT_LFU && evict != MOE_EVICT_LRU && evict != MOE_EVICT_ASIS))
    return MOE_ERR_INVALID;
  if ((int64_t)n_layers * n_experts > INT32_MAX) return MOE_ERR_INVALID;
  moe_policy *p = new (std::nothrow) moe_policy();
  if (!p) return MOE_ERR_INVALID;
  p->n_slots = n_slots;
  p->n_layers = n_layers;
  p->n_experts = n_experts;
  p->evict = evict;
  p->window = window;
  const size_t nk = (size_t)n_layers * n_experts;
  p->slot_of.assign(nk, -1);
  p->freq.assign(nk, 0);
  p->born.assign(nk, 0);
  p->last_use.assign(nk, 0);
  p->resident_born.assign(nk, 0);
  p->pending.assign(nk, 0);
  p->from_prefetch.assign(nk, 0);
  p->key_of.assign(n_slots, -1);
  p->pinned.assign(n_slots, 0);
  p->free_list.resize(n_slots);
  for (int32_t i = 0; i < n_slots; ++i) p->free_list[i] = i;
  *out = p;
  return MOE_OK;
}

int moe_policy_destroy(moe_policy *p) {
  delete p;
  return MOE_OK;
}

int moe_policy_prefetch(moe_policy *p, int32_t layer, const int32_t *experts,
                        int32_t n, int32_t *fill_slots, int32_t *fill_experts,
                        int32_t *bailed) {
  if (!p || (n > 0 && (!experts || !fill_slots || !fill_experts))) return MOE_ERR_INVALID;
  if (bailed) *bailed = 0;
  int32_t issued = 0;
  for (int32_t i = 0; i < n; ++i) {
    if (bad_key(p, layer, experts[i])) return MOE_ERR_INVALID;
    const int32_t k = p->key(layer, experts[i]);
    if (p->slot_of[k] >= 0 || p->pending[k]) continue;
    const int32_t slot = p->alloc(k);
    if (slot < 0) {
      p->n_prefetch_bail += 1;
      if (bailed) *bailed = 1;
      break;
    }
    p->n_prefetch_issued += 1;
    p->pending[k] = 1;
    fill_slots[issued] = slot;
    fill_experts[issued] = experts[i];
    ++issued;
  }
  return issued;
}

int moe_policy_acquire(moe_policy *p, int32_t layer, const int32_t *experts,
                       int32_t n, int32_t *slots_out, int32_t *miss_idx,
                       int32_t *n_miss, int32_t *wait_idx, int32_t *n_wait) {
  if (!p || n < 0 || (n > 0 && (!experts || !slots_out || !miss_idx || !wait_idx)) ||
      !n_miss || !n_wait)
    return MOE_ERR_INVALID;
  for (int32_t i = 0; i < n; ++i)
    if (bad_key(p, layer, experts[i])) return MOE_ERR_INVALID;
  int32_t nm = 0, nw = 0;
  for (int32_t i = 0; i < n; ++i) {
    const int32_t k = p->key(layer, experts[i]);
    const bool pend = p->pending[k] != 0;
    int32_t slot = p->slot_of[k];
    bool missed = false;
    slots_out[i] = -1;
    if (!pend && slot < 0) {
      slot = p->alloc(k);
      if (slot < 0) {
        *n_miss = nm;
        *n_wait = nw;
        return MOE_ERR_EXHAUSTED;
      }
      p->pin(slot);
      p->touch(k);
      miss_idx[nm++] = i;
      missed = true;
    } else if (slot >= 0) {
      p->pin(slot);
      p->touch(k);
    }
    if (pend) {
      wait_idx[nw++] = i;
    } else if (slot >= 0 && !missed) {
      const bool early = p->from_prefetch[k] != 0;
      p->from_prefetch[k] = 0;
      if (early) p->n_prefetch_hit += 1;
      else p->n_cache_hit += 1;
      slots_out[i] = slot;
    }
    if (missed) slots_out[i] = slot;
  }
  for (int32_t w = 0; w < nw; ++w) {
    const int32_t i = wait_idx[w];
    const int32_t k = p->key(layer, experts[i]);
    p->complete(k);
    p->pending[k] = 0;
    p->from_prefetch[k] = 0;
    slots_out[i] = p->slot_of[k];
    p->pin(slots_out[i]);
    p->touch(k);
    p->n_prefetch_hit += 1;
  }
  p->n_miss += nm;
  p->clear_pins();
  for (int32_t i = 0; i < n; ++i)
    if (slots_out[i] >= 0) p->pin(slots_out[i]);
  *n_miss = nm;
  *n_wait = nw;
  return MOE_OK;
}

int moe_policy_complete(moe_policy *p, int32_t layer, int32_t expert) {
  if (!p || bad_key(p, layer, expert)) return MOE_ERR_INVALID;
  p->complete(p->key(layer, expert));
  return MOE_OK;
}

int moe_policy_cancel(moe_policy *p, int32_t layer, int32_t expert) {
  if (!p || bad_key(p, layer, expert)) return MOE_ERR_INVALID;
  const int32_t k = p->key(layer, expert);
  if (!p->pending[k]) return MOE_ERR_INVALID;
  p->cancel(k);
  return MOE_OK;
}

int moe_policy_lookup(const moe_policy *p, int32_t layer, int32_t expert) {
  if (!p || bad_key(p, layer, expert)) return MOE_ERR_INVALID;
  return p->slot_of[p->key(layer, expert)];
}

int moe_policy_is_pending(const moe_policy *p, int32_t layer, int32_t expert) {
  if (!p || bad_key(p, layer, expert)) return MOE_ERR_INVALID;
  return p->pending[p->key(layer, expert)];
}

int moe_policy_table(const moe_policy *p, int32_t *table) {
  if (!p || !table) return MOE_ERR_INVALID;
  std::memcpy(table, p->slot_of.data(), p->slot_of.size() * sizeof(int32_t));
  return MOE_OK;
}

int moe_policy_stats(const moe_policy *p, int64_t *out) {
  if (!p || !out) return MOE_ERR_INVALID;
  out[0] = p->n_prefetch_hit + p->n_cache_hit + p->n_miss;
  out[1] = p->n_prefetch_hit;
  out[2] = p->n_cache_hit;
  out[3] = p->n_miss;
  out[4] = p->n_prefetch_bail;
  out[5] = p->n_prefetch_issued;
  out[6] = p->clock;
  out[7] = p->use_clock;
  return MOE_OK;
}

}  // extern "C"
