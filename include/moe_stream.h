/*
 * moe_stream.h -- C ABI of the MI355X expert hot path of moe-stream.
 *
 * Plain C: device pointers, sizes and a hipStream_t (passed as void*).  No
 * exceptions cross this boundary; every entry point returns an int status
 * (MOE_OK = 0, negative on error) and moe_last_error() describes the last
 * failure of the calling thread.  All buffers are owned by the caller (the
 * convention of the reference's array_from_ptr, ext/src/zerocopy.cpp:76-97).
 * Calls on one stream are ordered by that stream; the caller serialises
 * calls that share a workspace.
 *
 * bf16 values are passed as uint16_t bit patterns; 4-bit codes as uint32_t
 * words, element i of a row in word i>>3 at bit 4*(i&7) (low nibble first).
 */
#ifndef MOE_STREAM_H
#define MOE_STREAM_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

enum {
  MOE_OK = 0,
  MOE_ERR_INVALID = -1,     /* bad argument (null, size, alignment, range) */
  MOE_ERR_UNSUPPORTED = -2, /* geometry with no compiled kernel            */
  MOE_ERR_HIP = -3,         /* the HIP runtime reported an error           */
  MOE_ERR_EXHAUSTED = -4,   /* slot pool exhausted (every slot pinned)     */
  MOE_ERR_DEVICE = -5,      /* a kernel flagged an out-of-range slot ref   */
  MOE_ERR_TIMEOUT = -6      /* a kernel's bounded wait for another workgroup
                               gave up (moe_stack_decode with
                               MOE_STACK_ORDINARY whose grid was not resident
                               at once); that launch's outputs are invalid  */
};

/* Gated activation between gate/up and down. */
enum { MOE_ACT_SWIGLU = 0, MOE_ACT_SWIGLU_CLAMP = 1 };

/* Routing rule. */
enum {
  MOE_ROUTE_SOFTMAX_TOPK = 0, /* softmax over E, top-k, optional renorm (Qwen3)   */
  MOE_ROUTE_TOPK_SOFTMAX = 1  /* top-k of raw logits, softmax over the k (gpt-oss) */
};

#define MOE_MAX_COMPONENTS 12
#define MOE_MAX_TOPK 16

/* Expert geometry.  d_model = hidden size D, d_ff = expert intermediate F. */
typedef struct moe_geom {
  int32_t d_model;
  int32_t d_ff;
  int32_t group_size;    /* 64 */
  int32_t bits;          /* 4  */
  int32_t has_proj_bias; /* 1 for gpt-oss: each projection adds a bf16 bias  */
  int32_t act;           /* MOE_ACT_*                                        */
  float alpha;           /* clamped SwiGLU alpha (1.702)                     */
  float limit;           /* clamped SwiGLU limit (7.0)                       */
} moe_geom;

/*
 * The slot pool as the kernels see it: one array per component shaped
 * [n_slots, *shape] (the reference's layout, engine_v3.py:180-206), plus an
 * optional expert store in the repacked record layout (repack.py:73-82,141):
 * record r at store + r*record_bytes, component c at comp_offset[c] in it.
 *
 * Component order: proj-major over (gate_proj, up_proj, down_proj), then
 * part over (weight, scales, biases[, bias]) -- 9 components, or 12 when
 * has_proj_bias.
 *
 * A slot reference is an int32: ref >= 0 names pool slot `ref`; ref < 0
 * names store record (-ref - 1).
 */
typedef struct moe_pool_view {
  int32_t n_components;
  int32_t n_slots;
  void *base[MOE_MAX_COMPONENTS];
  int64_t slot_bytes[MOE_MAX_COMPONENTS];
  const void *store;
  int64_t record_bytes;
  int64_t n_records;
  int64_t comp_offset[MOE_MAX_COMPONENTS];
} moe_pool_view;

/* Library identity and error reporting. */
int moe_version(void);
const char *moe_last_error(void);

/* Bytes of the components of one expert for a geometry: writes up to 12
 * component sizes and returns the number of components (or < 0). */
int moe_component_bytes(const moe_geom *g, int64_t *bytes_out);

/*
 * Batch-1 (small T) expert block: for each token t and routed expert j,
 *   y_t = sum_j scores[t*k+j] * down_j( act(gate_j(x_t), up_j(x_t)) )
 * read from the pool/store via slot_refs[t*k+j].  Dequant, gate/up, the
 * activation, down and the weighted combine are fused into two kernels; the
 * [T*k, d_ff] intermediate never leaves the workspace.  fp32 accumulation.
 *
 * Replaces the three mx.gather_qmm calls + swiglu + weighted sum of
 * engine_v3.py:588-600 (Qwen3) and engine_120b.py:132-145 (gpt-oss), and the
 * disabled fused Metal kernel kernels.moe_expert_mlp (kernels.py:231-252).
 *
 * x: bf16 [T, d_model]; out_bf16: bf16 [T, d_model] (may be NULL);
 * out_f32: fp32 [T, d_model] (may be NULL; debug output).
 * workspace: device memory of at least moe_ffn_decode_workspace() bytes.
 */
size_t moe_ffn_decode_workspace(const moe_geom *g, int32_t T, int32_t k);
int moe_ffn_decode(const moe_pool_view *pool, const moe_geom *g,
                   const int32_t *slot_refs, const float *scores,
                   const uint16_t *x, int32_t T, int32_t k,
                   uint16_t *out_bf16, float *out_f32,
                   void *workspace, size_t workspace_bytes, void *stream);

/*
 * moe_ffn_decode for callers that cannot allocate device memory (code under
 * HIP graph capture, tight serving loops, harnesses that forbid hipMalloc):
 * no workspace argument, nothing allocated or freed.  This entry point has
 * no counterpart in the reference.  The [T*k, d_ff] activations go to a
 * fixed device array of the library, one per GPU, held until the process
 * ends: T * k * d_ff * 2 bytes must not exceed moe_ffn_decode_static_bytes()
 * (2 MiB; MOE_ERR_INVALID beyond, before any device work).  Every call on a
 * GPU shares that GPU's array, so calls that overlap on one GPU (other
 * streams, other threads) race; calls ordered on one stream do not.
 * Results are those of moe_ffn_decode (the same kernels).
 */
size_t moe_ffn_decode_static_bytes(void);
int moe_ffn_decode_static(const moe_pool_view *pool, const moe_geom *g,
                          const int32_t *slot_refs, const float *scores,
                          const uint16_t *x, int32_t T, int32_t k,
                          uint16_t *out_bf16, float *out_f32, void *stream);

/* The two halves of moe_ffn_decode, for callers that time or schedule them
 * separately: _up writes the bf16 [T*k, d_ff] activations into the
 * workspace, _down reads them (same workspace) and writes the combined
 * output.  moe_ffn_decode == _up then _down on one stream. */
int moe_ffn_decode_up(const moe_pool_view *pool, const moe_geom *g,
                      const int32_t *slot_refs, const uint16_t *x, int32_t T,
                      int32_t k, void *workspace, size_t workspace_bytes,
                      void *stream);
int moe_ffn_decode_down(const moe_pool_view *pool, const moe_geom *g,
                        const int32_t *slot_refs, const float *scores,
                        int32_t T, int32_t k, uint16_t *out_bf16,
                        float *out_f32, void *workspace,
                        size_t workspace_bytes, void *stream);

/*
 * Multi-token (prefill / batched) expert block: the same contract as
 * moe_ffn_decode -- y_t = sum_j scores[t*k+j] * down_j(act(gate_j(x_t),
 * up_j(x_t))) with expert j read via slot_refs[t*k+j] -- computed by
 * grouping the T*k pairs per slot reference and running each group as a bf16
 * MFMA contraction over the 4-bit codes (fp32 accumulation).  For T*k well
 * above the number of distinct slots, where an expert's weights serve many
 * tokens per read.  Results are deterministic and independent of how pairs
 * group.
 *
 * Replaces the batched (prefill) mx.gather_qmm calls, swiglu and weighted sum
 * of engine_v3.py:588-600 and engine_120b.py:132-145.
 *
 * Limits: pool->n_slots + (store ? pool->n_records : 0) <= 16256; T*k <=
 * 2^24.  workspace: at least moe_ffn_grouped_workspace() bytes (no zeroing
 * needed).
 */
size_t moe_ffn_grouped_workspace(const moe_geom *g, int32_t T, int32_t k);
int moe_ffn_grouped(const moe_pool_view *pool, const moe_geom *g,
                    const int32_t *slot_refs, const float *scores,
                    const uint16_t *x, int32_t T, int32_t k,
                    uint16_t *out_bf16, float *out_f32,
                    void *workspace, size_t workspace_bytes, void *stream);

/*
 * Router + top-k (+ lookahead + slot lookup) for T tokens in one launch.
 *   logits = x @ W.T (+ bias), materialised as bf16;
 *   mode SOFTMAX_TOPK: probs = bf16(softmax(logits)); top-k of probs; scores
 *     = probs (renormalised, in bf16 steps, when renorm != 0)
 *     (top_k_experts, engine_v3.py:467-473);
 *   mode TOPK_SOFTMAX: top-k of logits; scores = bf16(softmax(selected))
 *     (top_k_route, engine_120b.py:65-70).
 * ids are ranked (value descending, ties to the lower expert id).
 * Limits: E <= 128, k <= 16, k_pred <= 64; T <= 16 with d_model <= 4096 (a
 *   multiple of 8) runs one fused launch; T > 16 (prefill, up to 2^20
 *   tokens) needs d_model a multiple of 32 and runs a bf16 MFMA logits
 *   kernel, then the same selection.
 * Lookahead (W_next != NULL): pred_ids[t, 0..k_pred) = top-k_pred of the raw
 *   bf16 logits of x @ W_next.T (+ bias_next) (top_k_indices,
 *   engine_v3.py:476-483, engine_120b.py:73-75).
 * Slot lookup (table != NULL): slot_refs[t*k+j] = table[ids[t*k+j]], the
 *   device mirror of ExpertPool.slot_of for this layer (engine_v3.py:215);
 *   *miss_count (if not NULL) is incremented by the number of refs < 0.
 * scores are fp32 holding bf16-representable values.
 * workspace: at least moe_route_workspace() bytes, zeroed once before first
 * use (for T <= 16 it holds a sequence word the kernel advances by one per
 * launch and the router logits as entries tagged with it, so no clearing is
 * needed between launches).
 */
size_t moe_route_workspace(int32_t T, int32_t E);
int moe_route(const uint16_t *x, int32_t T, int32_t d_model,
              const uint16_t *W, const uint16_t *bias, int32_t E,
              int32_t mode, int32_t renorm, int32_t k,
              int32_t *ids, float *scores,
              const uint16_t *W_next, const uint16_t *bias_next,
              int32_t k_pred, int32_t *pred_ids,
              const int32_t *table, int32_t *slot_refs, int32_t *miss_count,
              void *workspace, size_t workspace_bytes, void *stream);

/* moe_stack_decode flags */
enum {
  MOE_STACK_COOPERATIVE = 0, /* default: a cooperative launch                  */
  MOE_STACK_ORDINARY = 1     /* an ordinary launch (see below)                  */
};

/*
 * Whole-token decode of an n_layers stack in ONE launch: for
 * each layer l, route x[l] with W[l] (+ bias[l]) and look ahead with W[l+1],
 * look the routed experts up in table[l] (slot refs, as moe_route), run the
 * expert block, write y[l].  Per-layer outputs: ids/scores/slot_refs
 * [n_layers, k], pred [n_layers, k_pred] (last layer: untouched),
 * miss_count [n_layers] (incremented).  Equivalent to moe_route +
 * moe_ffn_decode per layer on one stream, with the layer's phases chained by
 * device-side counters instead of kernel boundaries, and layer l+1 starting
 * only after y[l] is complete.
 * epoch: 1 for the first launch on a zeroed workspace, then 2, 3, ... while
 * (epoch + 1) * n_layers < 2^32 (past that, MOE_ERR_INVALID); after
 * MOE_ERR_DEVICE or MOE_ERR_TIMEOUT, or to go past that bound, zero the
 * workspace and restart at 1.  A workspace serves one stack (one n_layers)
 * at a time.
 * The pool must be in the packed layout (the reference's, engine_v3.py:180-
 * 206, repack.py:73-82,141): slot_bytes[c] = the component's bytes, and with
 * a store, comp_offset[c] = the components back to back and record_bytes =
 * their sum rounded up to 16 KiB; otherwise MOE_ERR_UNSUPPORTED (the kernel
 * takes these as constants of its geometry).
 * One workgroup per CU, all resident at once, each waiting for the others.
 * flags = MOE_STACK_COOPERATIVE: a cooperative launch, which guarantees
 * that.  flags = MOE_STACK_ORDINARY: an ordinary launch (~16 us less
 * dispatch cost per token) when the kernel's occupancy lets the device hold
 * the grid, else cooperative anyway; the CALLER guarantees that no other
 * kernel (another stream, another process, a fill on a side stream) holds
 * CUs of the device while it runs.  The kernel's waits are bounded: an
 * ordinary launch whose grid could not be placed at once ends with
 * MOE_ERR_TIMEOUT from moe_check_device_error, never a hang; rerun that
 * token cooperatively on a zeroed workspace (epoch 1).
 * This fuses the per-layer calls of streaming_call (engine_v3.py:493-609) for
 * a device-resident pool; it has no single counterpart in the reference.
 */
size_t moe_stack_workspace(const moe_geom *g, int32_t n_layers, int32_t E, int32_t k);
/* Phase trace of moe_stack_decode: while set, each launch writes wall-clock
 * stamps (wall_clock64 ticks, 100 MHz) of every workgroup (up to 256) at the
 * 15 phase points of every layer into device_buf ([256][n_layers][15]
 * uint64; point 0 = layer start, 6 = the workgroup's down rows published;
 * a point a workgroup does not reach keeps its old value).  A launch with a
 * buffer smaller than that fails with MOE_ERR_INVALID.  NULL turns it off.
 * Process-wide setting; outputs are the same with and without it. */
int moe_stack_trace(void *device_buf, size_t bytes);
int moe_stack_decode(const moe_pool_view *pool, const moe_geom *g, int32_t n_layers,
                     int32_t E, int32_t k, const uint16_t *x, const uint16_t *W,
                     const uint16_t *bias, int32_t mode, int32_t renorm, int32_t k_pred,
                     const int32_t *table, uint16_t *y, int32_t *ids, float *scores,
                     int32_t *slot_refs, int32_t *pred, int32_t *miss_count,
                     uint32_t epoch, int32_t flags, void *workspace,
                     size_t workspace_bytes, void *stream);

/*
 * Device-side (layer, expert) -> slot lookup for n ids (the index build of
 * engine_v3.py:550-552 against the slot table of engine_v3.py:215):
 * slot_refs[i] = table[ids[i]] for ids in [0, E); *miss_count (if not NULL)
 * is incremented by the number of refs < 0.  An id outside [0, E) gives
 * ref 0 and raises the device error flag that moe_check_device_error
 * reports as MOE_ERR_DEVICE.
 */
int moe_slot_lookup(const int32_t *table, int32_t E, const int32_t *ids,
                    int32_t n, int32_t *slot_refs, int32_t *miss_count,
                    void *stream);

/* Slot fills: copy n whole expert records into pool slots.
 * src_records: record indices into `src_store` (host pinned or device
 * memory laid out like pool->store, src_n_records records of
 * src_record_bytes; NULL means pool->store with the view's record size and
 * count), dst_slots: pool slots.  Host index arrays; every index is range
 * checked on the host (MOE_ERR_INVALID) before anything is enqueued.  Enqueued on `stream`.
 * A pool in the record layout (every component c at base + comp_offset[c]
 * of one base with slot stride src_record_bytes, i.e. each slot holds one
 * whole record) takes one hipMemcpyAsync per record (the copy engines, no
 * compute units).  Otherwise a source the GPU can read (HBM or pinned host
 * memory) is copied by kernels, up to 160 records per launch, and pageable
 * memory by hipMemcpyAsync per component.  Replaces ExpertPool._read
 * (engine_v3.py:255-290). */
int moe_fill_slots(const moe_pool_view *pool, const void *src_store,
                   int64_t src_record_bytes, int64_t src_n_records,
                   const int64_t *src_records, const int32_t *dst_slots, int32_t n,
                   void *stream);

/* Pinned host memory for the expert store (hipHostMalloc). */
int moe_host_alloc(size_t bytes, void **out);
int moe_host_free(void *p);

/* Events for stream-ordered slot reuse (the role of needs_barrier,
 * engine_v3.py:228-231, 601-607). */
int moe_event_create(void **ev);
int moe_event_destroy(void *ev);
int moe_event_record(void *ev, void *stream);
int moe_event_query(void *ev);                 /* 1 done, 0 pending, <0 err */
int moe_stream_wait_event(void *stream, void *ev);
int moe_event_elapsed_ms(void *start, void *stop, float *ms);

/* Read and clear the device error word set by the kernels, synchronising
 * `stream`.  Returns MOE_OK, MOE_ERR_TIMEOUT (a bounded cross-workgroup wait
 * gave up; the message also says if a slot ref was out of range) or
 * MOE_ERR_DEVICE (an out-of-range slot ref, whose contribution was zero). */
int moe_check_device_error(void *stream);

/*
 * Slot-pool bookkeeping (host only, no device calls): the (layer, expert) ->
 * slot table with sampled LFU/LRU eviction of ExpertPool
 * (engine_v3.py:213-236 state, :303-380 _alloc/_touch, :383-396 prefetch,
 * :398-454 acquire, :456-464 stats).  Fills are the caller's job: prefetch
 * and acquire report which slots to fill with which experts.  A prefetch
 * stays pending until moe_policy_complete (the fill finished) or until an
 * acquire of that expert waits on it.
 */
typedef struct moe_policy moe_policy;
enum { MOE_EVICT_LFU = 0, MOE_EVICT_LRU = 1, MOE_EVICT_ASIS = 2 };

/* window: entries younger than this many allocations are protected
 * (24 * max(1, prefetch depth) in the reference). */
int moe_policy_create(int32_t n_slots, int32_t n_layers, int32_t n_experts,
                      int32_t evict, int32_t window, moe_policy **out);
int moe_policy_destroy(moe_policy *p);
/* Returns the number of fills issued (written to fill_slots/fill_experts,
 * capacity n); *bailed = 1 when the pool was exhausted (silent bail). */
int moe_policy_prefetch(moe_policy *p, int32_t layer, const int32_t *experts,
                        int32_t n, int32_t *fill_slots, int32_t *fill_experts,
                        int32_t *bailed);
/* slots_out[i] = slot of experts[i]; miss_idx[0..*n_miss) = positions the
 * caller must fill now; wait_idx[0..*n_wait) = positions whose prefetch fill
 * the caller must wait for.  MOE_ERR_EXHAUSTED when every slot is pinned or
 * pending. */
int moe_policy_acquire(moe_policy *p, int32_t layer, const int32_t *experts,
                       int32_t n, int32_t *slots_out, int32_t *miss_idx,
                       int32_t *n_miss, int32_t *wait_idx, int32_t *n_wait);
int moe_policy_complete(moe_policy *p, int32_t layer, int32_t expert);
/* A pending prefetch whose fill was never issued (the caller's copy or event
 * call failed): the key is unmapped and its slot returns to the free list,
 * so a later acquire of it is a miss filled on demand rather than a wait on
 * a fill that does not exist.  The reference's fill worker drops the pending
 * entry on failure but keeps the mapping (engine_v3.py:292-301); this keeps
 * a failed fill's slot from being read.  MOE_ERR_INVALID if not pending. */
int moe_policy_cancel(moe_policy *p, int32_t layer, int32_t expert);
/* slot of (layer, expert) or -1 */
int moe_policy_lookup(const moe_policy *p, int32_t layer, int32_t expert);
int moe_policy_is_pending(const moe_policy *p, int32_t layer, int32_t expert);
/* table[layer * n_experts + expert] = slot or -1 (the device slot table) */
int moe_policy_table(const moe_policy *p, int32_t *table);
/* out[8] = total, prefetch hits, cache hits, misses, prefetch bails,
 * prefetches issued, allocation clock, use clock */
int moe_policy_stats(const moe_policy *p, int64_t *out);

/*
 * Native per-layer engine loop of the streaming pool, bs=1 decode: the steps
 * of streaming_call (engine_v3.py:493-609) -- route + lookahead, one host
 * synchronisation, prefetch of the predicted next-layer experts
 * (ExpertPool.prefetch, engine_v3.py:383-396) as fills on side_stream,
 * acquire (ExpertPool.acquire, :398-454) with misses filled on
 * compute_stream and in-flight prefetches turned into stream waits, then the
 * expert block -- without returning to the caller in between.  `policy` is
 * the pool's slot policy (moe_policy_create), shared with the caller;
 * `store` holds n_records records of record_bytes (pinned host memory for
 * DMA fills, or device memory).  moe_engine_layer is synchronous up to the
 * routing (it waits for the layer's route kernel) and leaves the expert
 * block enqueued on compute_stream.  The engine owns the events of its
 * pending prefetches; a pool driven by an engine is not filled by anyone
 * else meanwhile.
 */
typedef struct moe_engine moe_engine;
int moe_engine_create(const moe_pool_view *pool, const moe_geom *g, int32_t n_layers,
                      int32_t E, int32_t k, int32_t k_pred, moe_policy *policy,
                      const void *store, int64_t record_bytes, int64_t n_records,
                      void *compute_stream, void *side_stream, moe_engine **out);
int moe_engine_destroy(moe_engine *e);
/* One layer: x [1, d_model] bf16 -> y [1, d_model] bf16.  W_next/bias_next:
 * the next layer's router for the lookahead (NULL at the last layer). */
int moe_engine_layer(moe_engine *e, int32_t layer, const uint16_t *x, const uint16_t *W,
                     const uint16_t *bias, int32_t mode, int32_t renorm,
                     const uint16_t *W_next, const uint16_t *bias_next, uint16_t *y);
/* One layer with a list of prefetch depths (the reference's PF_DEPTH list,
 * engine_v3.py:61, 509-527): for each depths[j] > 0 whose target layer
 * (layer + depths[j]) is in the stack and whose router W_look[j] is not NULL,
 * the top-k_pred experts of that router on x are prefetched for the target
 * layer, in the list's order; recall is counted for depths[0] only.
 * bias_look may be NULL (no router biases) or hold NULL entries.
 * n_depths <= 4.  moe_engine_layer is this call with depths = {1}. */
int moe_engine_layer_depths(moe_engine *e, int32_t layer, const uint16_t *x,
                            const uint16_t *W, const uint16_t *bias, int32_t mode,
                            int32_t renorm, const int32_t *depths, int32_t n_depths,
                            const uint16_t *const *W_look, const uint16_t *const *bias_look,
                            uint16_t *y);
/* out[5] = bytes read into the pool, bytes read on the critical path
 * (misses), routed experts that were predicted, routed experts counted for
 * recall, prefetches still pending */
int moe_engine_counters(const moe_engine *e, int64_t *out);

#ifdef __cplusplus
}
#endif

#endif /* MOE_STREAM_H */
