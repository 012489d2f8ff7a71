// Native per-layer engine loop of the streaming pool for bs=1 decode: the
// steps of streaming_call (engine_v3.py:493-609) without a Python frame in
// between.  Per layer, in the reference's order:
//   1. route + one lookahead (engine_v3.py:509-515) on the compute stream;
//   2. the router writes the layer's ids and predictions straight into
//      coherent pinned host memory; the host waits for them there (the one
//      host synchronisation of engine_v3.py:515, without a copy command or a
//      stream synchronisation);
//   3. recall bookkeeping of the previous layer's prediction (:521-523);
//   4. prefetch of the predicted layer-(l+1) experts (:521-527, ExpertPool.
//      prefetch :383-396): fills from the pinned host store on the side
//      stream, one event per prefetch batch, pending until retired;
//   5. acquire (:537-552, ExpertPool.acquire :398-454): misses filled on the
//      compute stream, in-flight prefetches become stream waits;
//   6. the expert block (the decode kernels) on the compute stream, its slot
//      refs carried in the kernel arguments (no copy to the device).
// Further prefetch depths (the reference's PF_DEPTH list, engine_v3.py:61,
// 509-527; moe_engine_layer_depths): the first depth's router rides in the
// route launch of step 1; the router of each further depth d runs on x_l as
// a route launch of its own on the engine's lookahead stream beside step 1,
// and the host waits for all of them at once.  Their predictions are
// prefetched after the first depth's, in the list's order (the policy sees
// the reference's call sequence), and their copies are issued once the
// expert block is enqueued, since none is needed before layer l+2.
// Reuse of the pinned buffers is safe by stream order: the host rewrites
// them only after it has seen the next layer's router output, and that
// router started after the previous expert block completed.
// The slot policy is the same native policy ExpertPool uses; the engine owns
// the pending fills' events.

#include <atomic>
#include <chrono>
#include <cstring>
#include <unordered_map>
#include <vector>

namespace {

constexpr int kEngineMaxPred = 64;
constexpr int kEngineMaxDepths = 4;  // first depth + 3 further ones

}  // namespace

struct moe_engine {
  moe_pool_view pool;
  moe_geom geom;
  moe::PoolArgs pa;                    // kernel view of the pool, checked at creation
  const moe::FfnLaunch *ffn = nullptr; // decode kernels for the geometry
  moe_policy *policy = nullptr;
  const char *store = nullptr;      // pinned host (or device) records
  int64_t record_bytes = 0, n_records = 0;
  int32_t L = 0, E = 0, k = 0, kp = 0;
  hipStream_t compute = nullptr, side = nullptr;
  // device buffers
  float *d_scores = nullptr;
  void *d_route_ws = nullptr, *d_ffn_ws = nullptr;
  size_t route_ws_bytes = 0, ffn_ws_bytes = 0;
  // coherent pinned host memory the router writes: host and kernel
  // addresses of ids and predictions
  int32_t *h_ids = nullptr, *h_pred = nullptr;
  int32_t *k_ids = nullptr, *k_pred = nullptr;
  // further lookahead depths: their predictions (pinned, as above), the
  // lookahead stream their route launches run on, the event that orders
  // them after x, and the launches' own ids, scores and workspace
  int32_t *h_predx[kEngineMaxDepths - 1] = {}, *k_predx[kEngineMaxDepths - 1] = {};
  hipStream_t look = nullptr;
  hipEvent_t x_ready = nullptr;
  int32_t *d_idsx = nullptr;
  float *d_scoresx = nullptr;
  void *d_route_wsx = nullptr;
  int32_t h_refs[MOE_MAX_TOPK] = {};               // this layer's slot refs
  // bookkeeping
  std::unordered_map<int64_t, hipEvent_t> pending;   // key -> its fill's event
  std::vector<hipEvent_t> free_events;
  // the first depth's unique prediction per target layer, taken when that
  // layer routes (the reference's _PRED dict, engine_v3.py:521-523)
  std::vector<std::vector<int32_t>> pred_for;
  std::vector<char> pred_set;
  int64_t bytes_read = 0, bytes_exposed = 0, recall_hit = 0, recall_total = 0;
};

namespace {

int64_t engine_key(const moe_engine *e, int32_t layer, int32_t expert) {
  return (int64_t)layer * e->E + expert;
}

int engine_event(moe_engine *e, hipEvent_t *ev) {
  if (!e->free_events.empty()) {
    *ev = e->free_events.back();
    e->free_events.pop_back();
    return MOE_OK;
  }
  MOE_HIP(hipEventCreateWithFlags(ev, hipEventDisableTiming));
  return MOE_OK;
}

// Retire prefetch fills whose events completed (the worker epilogue,
// engine_v3.py:292-301).  One event may cover several keys.
int engine_poll(moe_engine *e) {
  std::vector<hipEvent_t> done;
  for (auto it = e->pending.begin(); it != e->pending.end();) {
    const hipError_t q = hipEventQuery(it->second);
    if (q == hipSuccess) {
      moe_policy_complete(e->policy, (int32_t)(it->first / e->E), (int32_t)(it->first % e->E));
      done.push_back(it->second);
      it = e->pending.erase(it);
    } else if (q == hipErrorNotReady) {
      ++it;
    } else {
      return hip_fail(q, "hipEventQuery");
    }
  }
  for (hipEvent_t ev : done) {
    bool shared = false;
    for (const auto &kv : e->pending) shared = shared || kv.second == ev;
    bool listed = false;
    for (hipEvent_t f : e->free_events) listed = listed || f == ev;
    if (!shared && !listed) e->free_events.push_back(ev);
  }
  return MOE_OK;
}

// Wait for the router's ids and the predictions of n_pred lookahead
// launches in pinned memory.  Every entry is -1 before the launches and is
// written once with an id in [0, E), so all entries non-negative means the
// outputs are complete.  The streams are queried only once a wait has run
// past 1 ms (and every 1 ms after), so that a failed launch ends the wait with
// its error: a query on every pass of a normal (~30 us) wait cost the loop
// 13 % of its rate.
int engine_wait_route(moe_engine *e, const int32_t *const *preds, int n_pred) {
  using clock = std::chrono::steady_clock;
  const volatile int32_t *ids = e->h_ids;
  auto ready = [&]() {
    bool r = true;
    for (int32_t i = 0; i < e->k; ++i) r = r && ids[i] >= 0;
    for (int j = 0; j < n_pred; ++j) {
      const volatile int32_t *pred = preds[j];
      for (int32_t i = 0; i < e->kp; ++i) r = r && pred[i] >= 0;
    }
    return r;
  };
  clock::time_point next{};
  for (uint32_t spin = 0; !ready(); ++spin) {
    if (spin % 1024 != 1023) continue;
    const clock::time_point now = clock::now();
    if (next == clock::time_point{}) {
      next = now + std::chrono::milliseconds(1);
      continue;
    }
    if (now < next) continue;
    next = now + std::chrono::milliseconds(1);
    const hipError_t q = hipStreamQuery(e->compute);
    const hipError_t ql = hipStreamQuery(e->look);
    if (q != hipSuccess && q != hipErrorNotReady) return hip_fail(q, "router launch");
    if (ql != hipSuccess && ql != hipErrorNotReady) return hip_fail(ql, "lookahead launch");
    if (q == hipErrorNotReady || ql == hipErrorNotReady) continue;
    if (!ready()) return fail(MOE_ERR_INVALID, "router finished without writing its ids");
  }
  std::atomic_thread_fence(std::memory_order_acquire);
  return MOE_OK;
}

// Unique predicted ids, ascending (np.unique of the prediction).
std::vector<int32_t> engine_unique(const int32_t *pred, int32_t n) {
  std::vector<int32_t> up(pred, pred + n);
  std::sort(up.begin(), up.end());
  up.erase(std::unique(up.begin(), up.end()), up.end());
  return up;
}

int engine_fill(moe_engine *e, int32_t layer, const int32_t *experts, const int32_t *slots,
                int32_t n, hipStream_t s) {
  if (n <= 0) return MOE_OK;
  std::vector<int64_t> recs(n);
  for (int32_t i = 0; i < n; ++i) recs[i] = (int64_t)layer * e->E + experts[i];
  const int rc =
      moe_fill_slots(&e->pool, e->store, e->record_bytes, e->n_records, recs.data(), slots, n, s);
  if (rc) return rc;
  e->bytes_read += (int64_t)n * e->record_bytes;
  return MOE_OK;
}

}  // namespace

extern "C" {

int moe_engine_create(const moe_pool_view *pool, const moe_geom *g, int32_t n_layers,
                      int32_t E, int32_t k, int32_t k_pred, moe_policy *policy,
                      const void *store, int64_t record_bytes, int64_t n_records,
                      void *compute_stream, void *side_stream, moe_engine **out) {
  if (!out) return fail(MOE_ERR_INVALID, "out is NULL");
  *out = nullptr;
  if (!pool || !g || !policy || !store) return fail(MOE_ERR_INVALID, "NULL pool/geom/policy/store");
  if (n_layers <= 0 || E <= 0 || E > moe::kRouteMaxE || k <= 0 || k > MOE_MAX_TOPK || k > E)
    return fail(MOE_ERR_INVALID, "n_layers=%d E=%d k=%d", n_layers, E, k);
  if (k_pred <= 0 || k_pred > E || k_pred > kEngineMaxPred)
    return fail(MOE_ERR_INVALID, "k_pred=%d outside [1, min(E, %d)]", k_pred, kEngineMaxPred);
  if (record_bytes <= 0 || n_records < (int64_t)n_layers * E)
    return fail(MOE_ERR_INVALID, "store has %lld records of %lld bytes, need %lld",
                (long long)n_records, (long long)record_bytes, (long long)n_layers * E);
  moe::PoolArgs pa;
  const int rc = make_pool_args(pool, g, &pa);
  if (rc) return rc;
  const moe::FfnLaunch *ffn = moe::find_ffn(g->d_model, g->d_ff, g->has_proj_bias);
  if (!ffn)
    return fail(MOE_ERR_UNSUPPORTED, "no decode kernel for d_model=%d d_ff=%d", g->d_model,
                g->d_ff);
  if (ffn->down_lds(k) > 65536)
    return fail(MOE_ERR_UNSUPPORTED, "k=%d needs %zu bytes of LDS in the down kernel", k,
                ffn->down_lds(k));
  if (g->act != MOE_ACT_SWIGLU && g->act != MOE_ACT_SWIGLU_CLAMP)
    return fail(MOE_ERR_INVALID, "unknown activation %d", g->act);
  moe_engine *e = new moe_engine();
  e->pool = *pool;
  e->geom = *g;
  e->pa = pa;
  e->ffn = ffn;
  e->policy = policy;
  e->store = static_cast<const char *>(store);
  e->record_bytes = record_bytes;
  e->n_records = n_records;
  e->L = n_layers;
  e->pred_for.resize(n_layers);
  e->pred_set.assign(n_layers, 0);
  e->E = E;
  e->k = k;
  e->kp = k_pred;
  e->compute = static_cast<hipStream_t>(compute_stream);
  e->side = static_cast<hipStream_t>(side_stream);
  e->route_ws_bytes = moe_route_workspace(1, E);
  e->ffn_ws_bytes = moe_ffn_decode_workspace(g, 1, k);
  hipError_t err = hipSuccess;
  auto dmalloc = [&](void **p, size_t b) {
    if (err == hipSuccess) err = hipMalloc(p, b);
    if (err == hipSuccess) err = hipMemset(*p, 0, b);
  };
  dmalloc(reinterpret_cast<void **>(&e->d_scores), 256);
  dmalloc(&e->d_route_ws, e->route_ws_bytes);
  dmalloc(reinterpret_cast<void **>(&e->d_idsx), 256);
  dmalloc(reinterpret_cast<void **>(&e->d_scoresx), 256);
  dmalloc(&e->d_route_wsx, e->route_ws_bytes);
  dmalloc(&e->d_ffn_ws, e->ffn_ws_bytes);
  auto shared = [&](int32_t **h, int32_t **k) {
    if (err == hipSuccess)
      err = hipHostMalloc(reinterpret_cast<void **>(h), 256,
                          hipHostMallocMapped | hipHostMallocCoherent);
    if (err == hipSuccess) err = hipHostGetDevicePointer(reinterpret_cast<void **>(k), *h, 0);
    if (err == hipSuccess) memset(*h, 0xff, 256);
  };
  shared(&e->h_ids, &e->k_ids);
  shared(&e->h_pred, &e->k_pred);
  for (int i = 0; i < kEngineMaxDepths - 1; ++i) shared(&e->h_predx[i], &e->k_predx[i]);
  if (err == hipSuccess) err = hipStreamCreateWithFlags(&e->look, hipStreamNonBlocking);
  if (err == hipSuccess) err = hipEventCreateWithFlags(&e->x_ready, hipEventDisableTiming);
  if (err != hipSuccess) {
    moe_engine_destroy(e);
    return hip_fail(err, "engine buffers");
  }
  *out = e;
  return MOE_OK;
}

int moe_engine_destroy(moe_engine *e) {
  if (!e) return MOE_OK;
  if (e->compute) (void)hipStreamSynchronize(e->compute);
  if (e->side) (void)hipStreamSynchronize(e->side);
  if (e->look) (void)hipStreamSynchronize(e->look);
  std::vector<hipEvent_t> evs = e->free_events;
  for (const auto &kv : e->pending) evs.push_back(kv.second);
  std::sort(evs.begin(), evs.end());
  evs.erase(std::unique(evs.begin(), evs.end()), evs.end());
  for (hipEvent_t ev : evs) (void)hipEventDestroy(ev);
  (void)hipFree(e->d_scores);
  (void)hipFree(e->d_route_ws);
  (void)hipFree(e->d_ffn_ws);
  (void)hipFree(e->d_idsx);
  (void)hipFree(e->d_scoresx);
  (void)hipFree(e->d_route_wsx);
  (void)hipHostFree(e->h_ids);
  (void)hipHostFree(e->h_pred);
  for (int i = 0; i < kEngineMaxDepths - 1; ++i) (void)hipHostFree(e->h_predx[i]);
  if (e->x_ready) (void)hipEventDestroy(e->x_ready);
  if (e->look) (void)hipStreamDestroy(e->look);
  delete e;
  return MOE_OK;
}

int moe_engine_layer_depths(moe_engine *e, int32_t layer, const uint16_t *x,
                            const uint16_t *W, const uint16_t *bias, int32_t mode,
                            int32_t renorm, const int32_t *depths, int32_t n_depths,
                            const uint16_t *const *W_look, const uint16_t *const *bias_look,
                            uint16_t *y) {
  if (!e) return fail(MOE_ERR_INVALID, "engine is NULL");
  if (layer < 0 || layer >= e->L) return fail(MOE_ERR_INVALID, "layer %d outside [0, %d)", layer, e->L);
  if (!x || !W || !y) return fail(MOE_ERR_INVALID, "NULL x/W/y");
  if (n_depths < 0 || n_depths > kEngineMaxDepths || (n_depths > 0 && (!depths || !W_look)))
    return fail(MOE_ERR_INVALID, "n_depths=%d outside [0, %d] or NULL depths/W_look", n_depths,
                kEngineMaxDepths);
  for (int32_t j = 0; j < n_depths; ++j)
    if (depths[j] <= 0) return fail(MOE_ERR_INVALID, "depth %d is not positive", depths[j]);
  // the depths that name a layer of the stack and come with a router
  bool on[kEngineMaxDepths] = {};
  for (int32_t j = 0; j < n_depths; ++j)
    on[j] = W_look[j] != nullptr && (int64_t)layer + depths[j] < e->L;
  const bool look = n_depths > 0 && on[0];
  auto bias_of = [&](int32_t j) { return bias_look ? bias_look[j] : nullptr; };
  // 1. route + the first lookahead, outputs into pinned memory reset to -1;
  // further depths on the lookahead stream, ordered after x
  for (int32_t i = 0; i < e->k; ++i) e->h_ids[i] = -1;
  for (int32_t i = 0; look && i < e->kp; ++i) e->h_pred[i] = -1;
  const int32_t *preds[kEngineMaxDepths];
  int n_pred = 0;
  if (look) preds[n_pred++] = e->h_pred;
  bool further = false;
  for (int32_t j = 1; j < n_depths; ++j) {
    if (!on[j]) continue;
    for (int32_t i = 0; i < e->kp; ++i) e->h_predx[j - 1][i] = -1;
    preds[n_pred++] = e->h_predx[j - 1];
    further = true;
  }
  std::atomic_thread_fence(std::memory_order_release);
  if (further) {
    MOE_HIP(hipEventRecord(e->x_ready, e->compute));
    MOE_HIP(hipStreamWaitEvent(e->look, e->x_ready, 0));
  }
  int rc = moe_route(x, 1, e->geom.d_model, W, bias, e->E, mode, renorm, e->k, e->k_ids,
                     e->d_scores, look ? W_look[0] : nullptr, look ? bias_of(0) : nullptr, e->kp,
                     look ? e->k_pred : nullptr, nullptr, nullptr, nullptr, e->d_route_ws,
                     e->route_ws_bytes, e->compute);
  if (rc) return rc;
  // a further depth's ids: top-kp of its router's logits (top_k_indices,
  // engine_v3.py:476-483), the lookahead rows of a route launch on that router
  for (int32_t j = 1; j < n_depths; ++j) {
    if (!on[j]) continue;
    rc = moe_route(x, 1, e->geom.d_model, W_look[j], bias_of(j), e->E, MOE_ROUTE_TOPK_SOFTMAX, 0,
                   1, e->d_idsx, e->d_scoresx, W_look[j], bias_of(j), e->kp, e->k_predx[j - 1],
                   nullptr, nullptr, nullptr, e->d_route_wsx, e->route_ws_bytes, e->look);
    if (rc) return rc;
  }
  // 2. one host synchronisation for routing and speculation
  rc = engine_wait_route(e, preds, n_pred);
  if (rc) return rc;
  // 3. recall of the prediction made for this layer (first depth only, as
  // the reference's _PRED)
  if (e->pred_set[layer]) {
    int32_t hit = 0;
    for (int32_t i = 0; i < e->k; ++i)
      for (int32_t p : e->pred_for[layer]) hit += p == e->h_ids[i];
    e->recall_hit += hit;
    e->recall_total += e->k;
    e->pred_set[layer] = 0;
  }
  rc = engine_poll(e);
  if (rc) return rc;
  // 4. prefetch of each depth's target layer in the list's order (unique
  // predicted ids, ascending, as np.unique); the first depth's copies now,
  // the further depths' after the expert block's launch
  struct Deferred {
    int32_t tgt, n;
    int32_t slots[kEngineMaxPred], exps[kEngineMaxPred];
  };
  Deferred later[kEngineMaxDepths - 1];
  int n_later = 0;
  // Every prefetch the policy counts as pending gets a fill and an event, or
  // is cancelled (unmapped, its slot freed) before an error returns: a
  // pending entry without an event would let its target layer's acquire
  // read a slot that was never filled.
  auto cancel = [&](int32_t tgt, const int32_t *exps, int32_t n) {
    for (int32_t i = 0; i < n; ++i) (void)moe_policy_cancel(e->policy, tgt, exps[i]);
  };
  auto cancel_later = [&](int from) {
    for (int i = from; i < n_later; ++i) cancel(later[i].tgt, later[i].exps, later[i].n);
  };
  for (int32_t j = 0, pj = 0; j < n_depths; ++j) {
    if (!on[j] || (j == 0 && !look)) continue;
    const std::vector<int32_t> up = engine_unique(preds[pj++], e->kp);
    const int32_t tgt = layer + depths[j];
    if (j == 0) {
      e->pred_for[tgt] = up;
      e->pred_set[tgt] = 1;
    }
    Deferred &d = later[n_later];
    int32_t bailed = 0;
    const int n = moe_policy_prefetch(e->policy, tgt, up.data(), (int32_t)up.size(), d.slots,
                                      d.exps, &bailed);
    if (n < 0) {
      cancel_later(0);
      return fail(n, "policy prefetch failed");
    }
    if (n == 0) continue;
    if (j > 0) {
      d.tgt = tgt;
      d.n = n;
      ++n_later;
      continue;
    }
    hipEvent_t ev = nullptr;
    rc = engine_fill(e, tgt, d.exps, d.slots, n, e->side);
    if (!rc) rc = engine_event(e, &ev);
    if (!rc && hipEventRecord(ev, e->side) != hipSuccess) {
      e->free_events.push_back(ev);
      rc = fail(MOE_ERR_HIP, "hipEventRecord failed");
    }
    if (rc) {
      cancel(tgt, d.exps, n);
      cancel_later(0);
      return rc;
    }
    for (int i = 0; i < n; ++i) e->pending[engine_key(e, tgt, d.exps[i])] = ev;
  }
  // 5-6 run as one step whose result is returned after the further depths'
  // copies are issued: the policy already counts those prefetches as
  // pending, so they are issued (with their events) whatever happens here
  auto block = [&]() -> int {
    // 5. acquire: misses on the compute stream, pending prefetches as waits
    int32_t miss_idx[MOE_MAX_TOPK], wait_idx[MOE_MAX_TOPK], n_miss = 0, n_wait = 0;
    rc = moe_policy_acquire(e->policy, layer, e->h_ids, e->k, e->h_refs, miss_idx, &n_miss,
                            wait_idx, &n_wait);
    if (rc) return fail(rc, rc == MOE_ERR_EXHAUSTED ? "pool exhausted: every slot pinned or pending"
                                                    : "policy acquire failed");
    if (n_miss > 0) {
      int32_t exps[MOE_MAX_TOPK], slots[MOE_MAX_TOPK];
      for (int32_t i = 0; i < n_miss; ++i) {
        exps[i] = e->h_ids[miss_idx[i]];
        slots[i] = e->h_refs[miss_idx[i]];
      }
      rc = engine_fill(e, layer, exps, slots, n_miss, e->compute);
      if (rc) return rc;
      e->bytes_exposed += (int64_t)n_miss * e->record_bytes;
    }
    for (int32_t w = 0; w < n_wait; ++w) {
      const auto it = e->pending.find(engine_key(e, layer, e->h_ids[wait_idx[w]]));
      if (it == e->pending.end()) continue;
      MOE_HIP(hipStreamWaitEvent(e->compute, it->second, 0));
      hipEvent_t ev = it->second;
      e->pending.erase(it);
      bool shared = false;
      for (const auto &kv : e->pending) shared = shared || kv.second == ev;
      if (!shared) e->free_events.push_back(ev);
    }
    // 6. the expert block, slot refs in the kernel arguments; pool arguments
    // and launch shapes were checked at creation, x by the router
    moe::RefList refs{};
    for (int32_t i = 0; i < e->k; ++i) refs.inl[i] = e->h_refs[i];
    (void)hipGetLastError();
    moe::launch_ffn_decode(e->ffn, e->pa, refs, e->d_scores, x, 1, e->k,
                           static_cast<uint16_t *>(e->d_ffn_ws), y, nullptr, e->geom.act,
                           e->geom.alpha, e->geom.limit, e->compute);
    MOE_HIP(hipGetLastError());
    return MOE_OK;
  };
  const int rc_block = block();
  // 7. the further depths' prefetch copies, one event per depth
  for (int i = 0; i < n_later; ++i) {
    const Deferred &d = later[i];
    hipEvent_t ev = nullptr;
    rc = engine_fill(e, d.tgt, d.exps, d.slots, d.n, e->side);
    if (!rc) rc = engine_event(e, &ev);
    if (!rc && hipEventRecord(ev, e->side) != hipSuccess) {
      e->free_events.push_back(ev);
      rc = fail(MOE_ERR_HIP, "hipEventRecord failed");
    }
    if (rc) {
      cancel_later(i);
      return rc;
    }
    for (int k = 0; k < d.n; ++k) e->pending[engine_key(e, d.tgt, d.exps[k])] = ev;
  }
  return rc_block;
}

int moe_engine_layer(moe_engine *e, int32_t layer, const uint16_t *x, const uint16_t *W,
                     const uint16_t *bias, int32_t mode, int32_t renorm,
                     const uint16_t *W_next, const uint16_t *bias_next, uint16_t *y) {
  const int32_t depth = 1;
  return moe_engine_layer_depths(e, layer, x, W, bias, mode, renorm, &depth, 1, &W_next,
                                 &bias_next, y);
}

int moe_engine_counters(const moe_engine *e, int64_t *out) {
  if (!e || !out) return fail(MOE_ERR_INVALID, "NULL engine/out");
  out[0] = e->bytes_read;
  out[1] = e->bytes_exposed;
  out[2] = e->recall_hit;
  out[3] = e->recall_total;
  out[4] = (int64_t)e->pending.size();
  return MOE_OK;
}

}  // extern "C"
