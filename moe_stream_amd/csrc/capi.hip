// C ABI of the expert hot path: argument checks, geometry dispatch, slot
// fills, pinned host memory and events.  No exceptions cross this boundary;
// failures return a negative status and set a thread-local message.
#include <algorithm>
#include <cstdarg>
#include <cstdio>
#include <mutex>
#include <string>

#include "launchers.h"

namespace {

thread_local std::string g_err;

int fail(int code, const char *fmt, ...) {
  char buf[512];
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(buf, sizeof(buf), fmt, ap);
  va_end(ap);
  g_err = buf;
  return code;
}

int hip_fail(hipError_t e, const char *what) {
  return fail(MOE_ERR_HIP, "%s: %s", what, hipGetErrorString(e));
}

#define MOE_HIP(call)                                   \
  do {                                                  \
    hipError_t e_ = (call);                             \
    if (e_ != hipSuccess) return hip_fail(e_, #call);   \
  } while (0)

bool aligned(const void *p, size_t a) {
  return (reinterpret_cast<uintptr_t>(p) % a) == 0;
}

// Component sizes of one expert: proj-major (gate, up, down) x part-major
// (weight, scales, biases[, bias]); the order of repack.py:35-37 and
// repack_gptoss.py:54-55.
int component_bytes(const moe_geom *g, int64_t *b) {
  if (!g) return fail(MOE_ERR_INVALID, "geom is NULL");
  if (g->group_size != 64 || g->bits != 4)
    return fail(MOE_ERR_UNSUPPORTED, "only 4-bit affine, group 64 (got %d-bit, group %d)",
                g->bits, g->group_size);
  if (g->d_model <= 0 || g->d_ff <= 0 || g->d_model % 64 || g->d_ff % 64)
    return fail(MOE_ERR_INVALID, "d_model=%d d_ff=%d must be positive multiples of 64",
                g->d_model, g->d_ff);
  const int np = g->has_proj_bias ? 4 : 3;
  const int64_t D = g->d_model, F = g->d_ff;
  for (int p = 0; p < 3; ++p) {
    const int64_t out = (p == 2) ? D : F, in = (p == 2) ? F : D;
    b[p * np + 0] = out * in / 2;          // uint32 codes, 8 per word
    b[p * np + 1] = out * (in / 64) * 2;   // bf16 scales
    b[p * np + 2] = out * (in / 64) * 2;   // bf16 biases
    if (np == 4) b[p * np + 3] = out * 2;  // bf16 projection bias
  }
  return np * 3;
}

// The persistent decode kernel takes slot strides, store component offsets
// and the record size as constants of its geometry (moe::PackedLayout): the
// pool must be the packed per-component [n_slots, *shape] arrays and the
// store the repacked records, as the reference's pool and store are.
int check_packed_layout(const moe_pool_view *v, const moe_geom *g) {
  int64_t cb[MOE_MAX_COMPONENTS];
  const int nc = component_bytes(g, cb);
  if (nc < 0) return nc;
  int64_t off = 0;
  for (int c = 0; c < nc; ++c) {
    if (v->n_slots > 0 && v->slot_bytes[c] != cb[c])
      return fail(MOE_ERR_UNSUPPORTED,
                  "persistent decode needs packed slots: component %d stride %lld != %lld", c,
                  (long long)v->slot_bytes[c], (long long)cb[c]);
    if (v->store && v->comp_offset[c] != off)
      return fail(MOE_ERR_UNSUPPORTED,
                  "persistent decode needs repacked records: component %d at %lld != %lld", c,
                  (long long)v->comp_offset[c], (long long)off);
    off += cb[c];
  }
  const int64_t rec = (off + 16383) / 16384 * 16384;
  if (v->store && v->record_bytes != rec)
    return fail(MOE_ERR_UNSUPPORTED, "persistent decode needs %lld-byte records (got %lld)",
                (long long)rec, (long long)v->record_bytes);
  return MOE_OK;
}

int make_pool_args(const moe_pool_view *v, const moe_geom *g, moe::PoolArgs *pa) {
  if (!v) return fail(MOE_ERR_INVALID, "pool view is NULL");
  int64_t cb[MOE_MAX_COMPONENTS];
  const int nc = component_bytes(g, cb);
  if (nc < 0) return nc;
  if (v->n_components != nc)
    return fail(MOE_ERR_INVALID, "pool view has %d components, geometry needs %d",
                v->n_components, nc);
  if (v->n_slots < 0) return fail(MOE_ERR_INVALID, "n_slots < 0");
  const int np = nc / 3;
  for (int c = 0; c < nc; ++c) {
    const size_t align = (c % np == 0) ? 16 : 2;
    if (v->n_slots > 0) {
      if (!v->base[c]) return fail(MOE_ERR_INVALID, "component %d base is NULL", c);
      if (!aligned(v->base[c], align) || v->slot_bytes[c] % (int64_t)align)
        return fail(MOE_ERR_INVALID, "component %d misaligned for %zu-byte loads", c, align);
      if (v->slot_bytes[c] < cb[c])
        return fail(MOE_ERR_INVALID, "component %d slot stride %lld < %lld bytes", c,
                    (long long)v->slot_bytes[c], (long long)cb[c]);
    }
    pa->base[c] = static_cast<const char *>(v->base[c]);
    pa->slot_bytes[c] = v->slot_bytes[c];
    pa->comp_offset[c] = v->comp_offset[c];
    if (v->store) {
      if (v->comp_offset[c] < 0 || v->comp_offset[c] + cb[c] > v->record_bytes)
        return fail(MOE_ERR_INVALID, "component %d [%lld,+%lld) outside the %lld-byte record",
                    c, (long long)v->comp_offset[c], (long long)cb[c],
                    (long long)v->record_bytes);
      if (v->comp_offset[c] % (int64_t)align)
        return fail(MOE_ERR_INVALID, "component %d store offset misaligned", c);
    }
  }
  for (int c = nc; c < MOE_MAX_COMPONENTS; ++c) {
    pa->base[c] = nullptr;
    pa->slot_bytes[c] = 0;
    pa->comp_offset[c] = 0;
  }
  pa->store = static_cast<const char *>(v->store);
  pa->record_bytes = v->record_bytes;
  if (v->store && (!aligned(v->store, 16) || v->record_bytes % 16))
    return fail(MOE_ERR_INVALID, "store base/record size must be 16-byte aligned");
  if (v->n_records > INT32_MAX) return fail(MOE_ERR_INVALID, "too many store records");
  pa->n_records = v->store ? (int32_t)v->n_records : 0;
  pa->n_slots = v->n_slots;
  if (pa->n_slots == 0 && pa->n_records == 0)
    return fail(MOE_ERR_INVALID, "pool view has neither slots nor store records");
  return MOE_OK;
}

}  // namespace

extern "C" {

int moe_version(void) { return 1; }

const char *moe_last_error(void) { return g_err.c_str(); }

int moe_component_bytes(const moe_geom *g, int64_t *bytes_out) {
  if (!bytes_out) return fail(MOE_ERR_INVALID, "bytes_out is NULL");
  return component_bytes(g, bytes_out);
}

size_t moe_ffn_decode_workspace(const moe_geom *g, int32_t T, int32_t k) {
  if (!g || T <= 0 || k <= 0) return 0;
  // h: bf16 [T*k, d_ff], padded to 256 bytes
  const size_t h = (size_t)T * k * g->d_ff * 2;
  return (h + 255) & ~(size_t)255;
}

// Refs of a launch read from a device array.
static moe::RefList device_refs(const int32_t *slot_refs) {
  moe::RefList r{};
  r.ptr = slot_refs;
  return r;
}

// Shared argument checks of the decode entry points.
static int ffn_prepare(const moe_pool_view *pool, const moe_geom *g,
                       const int32_t *slot_refs, int32_t T, int32_t k,
                       void *workspace, size_t workspace_bytes,
                       moe::PoolArgs *pa, const moe::FfnLaunch **L) {
  int rc = make_pool_args(pool, g, pa);
  if (rc) return rc;
  if (T <= 0) return fail(MOE_ERR_INVALID, "T=%d must be positive", T);
  if (k <= 0 || k > MOE_MAX_TOPK)
    return fail(MOE_ERR_INVALID, "k=%d outside [1, %d]", k, MOE_MAX_TOPK);
  if (!slot_refs || !workspace) return fail(MOE_ERR_INVALID, "NULL slot_refs/workspace");
  if (!aligned(workspace, 16)) return fail(MOE_ERR_INVALID, "workspace misaligned");
  if (workspace_bytes < moe_ffn_decode_workspace(g, T, k))
    return fail(MOE_ERR_INVALID, "workspace %zu < %zu bytes", workspace_bytes,
                moe_ffn_decode_workspace(g, T, k));
  if (g->act != MOE_ACT_SWIGLU && g->act != MOE_ACT_SWIGLU_CLAMP)
    return fail(MOE_ERR_INVALID, "unknown activation %d", g->act);
  *L = moe::find_ffn(g->d_model, g->d_ff, g->has_proj_bias);
  if (!*L)
    return fail(MOE_ERR_UNSUPPORTED,
                "no decode kernel compiled for d_model=%d d_ff=%d proj_bias=%d",
                g->d_model, g->d_ff, g->has_proj_bias);
  if ((*L)->down_lds(k) > 65536)
    return fail(MOE_ERR_UNSUPPORTED, "k=%d needs %zu bytes of LDS in the down kernel (max 65536)",
                k, (*L)->down_lds(k));
  return MOE_OK;
}

int moe_ffn_decode_up(const moe_pool_view *pool, const moe_geom *g,
                      const int32_t *slot_refs, const uint16_t *x, int32_t T,
                      int32_t k, void *workspace, size_t workspace_bytes,
                      void *stream) {
  moe::PoolArgs pa;
  const moe::FfnLaunch *L = nullptr;
  int rc = ffn_prepare(pool, g, slot_refs, T, k, workspace, workspace_bytes, &pa, &L);
  if (rc) return rc;
  if (!x) return fail(MOE_ERR_INVALID, "NULL x");
  if (!aligned(x, 16)) return fail(MOE_ERR_INVALID, "x must be 16-byte aligned");
  (void)hipGetLastError();
  moe::launch_ffn_up(L, pa, device_refs(slot_refs), x, T, k, static_cast<uint16_t *>(workspace),
                     g->act, g->alpha, g->limit, static_cast<hipStream_t>(stream));
  MOE_HIP(hipGetLastError());
  return MOE_OK;
}

int moe_ffn_decode_down(const moe_pool_view *pool, const moe_geom *g,
                        const int32_t *slot_refs, const float *scores,
                        int32_t T, int32_t k, uint16_t *out_bf16,
                        float *out_f32, void *workspace,
                        size_t workspace_bytes, void *stream) {
  moe::PoolArgs pa;
  const moe::FfnLaunch *L = nullptr;
  int rc = ffn_prepare(pool, g, slot_refs, T, k, workspace, workspace_bytes, &pa, &L);
  if (rc) return rc;
  if (!scores) return fail(MOE_ERR_INVALID, "NULL scores");
  if (!out_bf16 && !out_f32) return fail(MOE_ERR_INVALID, "no output buffer");
  (void)hipGetLastError();
  moe::launch_ffn_down(L, pa, device_refs(slot_refs), scores, T, k,
                       static_cast<const uint16_t *>(workspace), out_bf16, out_f32,
                       static_cast<hipStream_t>(stream));
  MOE_HIP(hipGetLastError());
  return MOE_OK;
}

int moe_ffn_decode(const moe_pool_view *pool, const moe_geom *g,
                   const int32_t *slot_refs, const float *scores,
                   const uint16_t *x, int32_t T, int32_t k, uint16_t *out_bf16,
                   float *out_f32, void *workspace, size_t workspace_bytes,
                   void *stream) {
  moe::PoolArgs pa;
  const moe::FfnLaunch *L = nullptr;
  int rc = ffn_prepare(pool, g, slot_refs, T, k, workspace, workspace_bytes, &pa, &L);
  if (rc) return rc;
  if (!scores || !x) return fail(MOE_ERR_INVALID, "NULL scores/x");
  if (!out_bf16 && !out_f32) return fail(MOE_ERR_INVALID, "no output buffer");
  if (!aligned(x, 16)) return fail(MOE_ERR_INVALID, "x must be 16-byte aligned");
  (void)hipGetLastError();
  moe::launch_ffn_decode(L, pa, device_refs(slot_refs), scores, x, T, k,
                         static_cast<uint16_t *>(workspace), out_bf16, out_f32,
                         g->act, g->alpha, g->limit,
                         static_cast<hipStream_t>(stream));
  MOE_HIP(hipGetLastError());
  return MOE_OK;
}

// ---------------------------------------------------------------------------
// moe_ffn_decode without a caller workspace: the [T*k, d_ff] activations go
// to `scratch`, a fixed device array of this library (one per GPU, held
// until the process ends).  Its device address is looked up once per device
// on the first call there, with that device current; host code uses only
// that address (the array's name is a host-side stand-in).
// ---------------------------------------------------------------------------
namespace {

constexpr size_t kScratchBytes = (size_t)2 << 20;   // MOE_FFN_DECODE_STATIC_BYTES
static __device__ __align__(256) char scratch[kScratchBytes];

constexpr int kScratchDevices = 64;
static std::mutex g_scratch_mu;
static void *g_scratch_ptr[kScratchDevices] = {};

// The current device's scratch address, looked up on its first use.
static int scratch_ptr(void **out) {
  int dev = 0;
  MOE_HIP(hipGetDevice(&dev));
  if (dev < 0 || dev >= kScratchDevices)
    return fail(MOE_ERR_UNSUPPORTED, "device %d beyond the %d the static scratch serves", dev,
                kScratchDevices);
  std::lock_guard<std::mutex> lock(g_scratch_mu);
  if (!g_scratch_ptr[dev]) {
    void *p = nullptr;
    MOE_HIP(hipGetSymbolAddress(&p, HIP_SYMBOL(scratch)));
    if (!p) return fail(MOE_ERR_HIP, "hipGetSymbolAddress(scratch) gave NULL");
    g_scratch_ptr[dev] = p;
  }
  *out = g_scratch_ptr[dev];
  return MOE_OK;
}

}  // namespace

size_t moe_ffn_decode_static_bytes(void) { return kScratchBytes; }

int moe_ffn_decode_static(const moe_pool_view *pool, const moe_geom *g,
                          const int32_t *slot_refs, const float *scores,
                          const uint16_t *x, int32_t T, int32_t k, uint16_t *out_bf16,
                          float *out_f32, void *stream) {
  if (!g) return fail(MOE_ERR_INVALID, "geom is NULL");
  if (T <= 0 || k <= 0) return fail(MOE_ERR_INVALID, "T=%d k=%d must be positive", T, k);
  const size_t need = moe_ffn_decode_workspace(g, T, k);
  if (need > kScratchBytes)
    return fail(MOE_ERR_INVALID,
                "T=%d x k=%d x d_ff=%d activations need %zu bytes, above the %zu-byte "
                "static scratch: call moe_ffn_decode with a workspace", T, k, g->d_ff, need,
                kScratchBytes);
  moe::PoolArgs pa;
  const moe::FfnLaunch *L = nullptr;
  // the size checks above come first, so an oversized call does no device work
  void *ws = nullptr;
  int rc = scratch_ptr(&ws);
  if (rc) return rc;
  rc = ffn_prepare(pool, g, slot_refs, T, k, ws, kScratchBytes, &pa, &L);
  if (rc) return rc;
  if (!scores || !x) return fail(MOE_ERR_INVALID, "NULL scores/x");
  if (!out_bf16 && !out_f32) return fail(MOE_ERR_INVALID, "no output buffer");
  if (!aligned(x, 16)) return fail(MOE_ERR_INVALID, "x must be 16-byte aligned");
  (void)hipGetLastError();
  moe::launch_ffn_decode(L, pa, device_refs(slot_refs), scores, x, T, k,
                         static_cast<uint16_t *>(ws), out_bf16, out_f32, g->act, g->alpha,
                         g->limit, static_cast<hipStream_t>(stream));
  MOE_HIP(hipGetLastError());
  return MOE_OK;
}

size_t moe_ffn_grouped_workspace(const moe_geom *g, int32_t T, int32_t k) {
  if (!g || T <= 0 || k <= 0 || (int64_t)T * k > (1 << 24) || g->d_model <= 0 ||
      g->d_ff <= 0)
    return 0;
  return moe::grouped_ws(T, k, g->d_model, g->d_ff).total;
}

int moe_ffn_grouped(const moe_pool_view *pool, const moe_geom *g,
                    const int32_t *slot_refs, const float *scores, const uint16_t *x,
                    int32_t T, int32_t k, uint16_t *out_bf16, float *out_f32,
                    void *workspace, size_t workspace_bytes, void *stream) {
  moe::PoolArgs pa;
  int rc = make_pool_args(pool, g, &pa);
  if (rc) return rc;
  if (T <= 0) return fail(MOE_ERR_INVALID, "T=%d must be positive", T);
  if (k <= 0 || k > MOE_MAX_TOPK)
    return fail(MOE_ERR_INVALID, "k=%d outside [1, %d]", k, MOE_MAX_TOPK);
  if ((int64_t)T * k > (1 << 24))
    return fail(MOE_ERR_INVALID, "T*k=%lld above 2^24", (long long)T * k);
  if (!slot_refs || !scores || !x || !workspace)
    return fail(MOE_ERR_INVALID, "NULL slot_refs/scores/x/workspace");
  if (!out_bf16 && !out_f32) return fail(MOE_ERR_INVALID, "no output buffer");
  if (!aligned(x, 16) || !aligned(workspace, 256) || (out_bf16 && !aligned(out_bf16, 8)) ||
      (out_f32 && !aligned(out_f32, 16)))
    return fail(MOE_ERR_INVALID,
                "x/out_f32 must be 16-byte, out_bf16 8-byte, workspace 256-byte aligned");
  if (g->act != MOE_ACT_SWIGLU && g->act != MOE_ACT_SWIGLU_CLAMP)
    return fail(MOE_ERR_INVALID, "unknown activation %d", g->act);
  if ((int64_t)pa.n_slots + pa.n_records > moe::kGroupMaxKeys)
    return fail(MOE_ERR_UNSUPPORTED, "n_slots + n_records = %lld above %d",
                (long long)pa.n_slots + pa.n_records, moe::kGroupMaxKeys);
  const moe::GroupedLaunch *G = moe::find_grouped(g->d_model, g->d_ff, g->has_proj_bias);
  if (!G)
    return fail(MOE_ERR_UNSUPPORTED,
                "no grouped kernel compiled for d_model=%d d_ff=%d proj_bias=%d", g->d_model,
                g->d_ff, g->has_proj_bias);
  const size_t need = moe_ffn_grouped_workspace(g, T, k);
  if (workspace_bytes < need)
    return fail(MOE_ERR_INVALID, "workspace %zu < %zu bytes", workspace_bytes, need);
  (void)hipGetLastError();
  moe::launch_grouped(G, pa, slot_refs, scores, x, T, k, out_bf16, out_f32,
                      static_cast<char *>(workspace), g->act, g->alpha, g->limit,
                      static_cast<hipStream_t>(stream));
  MOE_HIP(hipGetLastError());
  return MOE_OK;
}

size_t moe_route_workspace(int32_t T, int32_t E) {
  if (T <= 0 || E <= 0) return 0;
  // sequence word (padded to 256 B) + logits [2][T][E]: 8-byte flagged
  // entries for the one-launch path (T <= 16), fp32 for many tokens
  const size_t entry = T <= moe::kRouteMaxT ? 8 : 4;
  return 256 + (((size_t)2 * T * E * entry + 255) & ~(size_t)255);
}

int moe_route(const uint16_t *x, int32_t T, int32_t d_model, const uint16_t *W,
              const uint16_t *bias, int32_t E, int32_t mode, int32_t renorm,
              int32_t k, int32_t *ids, float *scores, const uint16_t *W_next,
              const uint16_t *bias_next, int32_t k_pred, int32_t *pred_ids,
              const int32_t *table, int32_t *slot_refs, int32_t *miss_count,
              void *workspace, size_t workspace_bytes, void *stream) {
  if (T <= 0 || T > (1 << 20)) return fail(MOE_ERR_INVALID, "T=%d outside [1, 2^20]", T);
  if (E <= 0 || E > moe::kRouteMaxE)
    return fail(MOE_ERR_INVALID, "E=%d outside [1, %d]", E, moe::kRouteMaxE);
  if (T <= moe::kRouteMaxT && (d_model <= 0 || d_model % 8 || d_model > 4096))
    return fail(MOE_ERR_INVALID, "d_model=%d must be a multiple of 8 in [8, 4096]", d_model);
  if (T > moe::kRouteMaxT && (d_model <= 0 || d_model % 32))
    return fail(MOE_ERR_INVALID, "T=%d > %d needs d_model (%d) a positive multiple of 32", T,
                moe::kRouteMaxT, d_model);
  if (k <= 0 || k > MOE_MAX_TOPK || k > E)
    return fail(MOE_ERR_INVALID, "k=%d outside [1, min(E, %d)]", k, MOE_MAX_TOPK);
  if (mode != MOE_ROUTE_SOFTMAX_TOPK && mode != MOE_ROUTE_TOPK_SOFTMAX)
    return fail(MOE_ERR_INVALID, "unknown routing mode %d", mode);
  if (!x || !W || !ids || !scores || !workspace)
    return fail(MOE_ERR_INVALID, "NULL x/W/ids/scores/workspace");
  if (!aligned(x, 16) || !aligned(W, 16))
    return fail(MOE_ERR_INVALID, "x and W must be 16-byte aligned");
  if (W_next) {
    if (!pred_ids) return fail(MOE_ERR_INVALID, "W_next given without pred_ids");
    if (k_pred <= 0 || k_pred > E || k_pred > 64)
      return fail(MOE_ERR_INVALID, "k_pred=%d outside [1, min(E, 64)]", k_pred);
    if (!aligned(W_next, 16)) return fail(MOE_ERR_INVALID, "W_next misaligned");
  }
  if (table && !slot_refs) return fail(MOE_ERR_INVALID, "table given without slot_refs");
  if (workspace_bytes < moe_route_workspace(T, E))
    return fail(MOE_ERR_INVALID, "workspace %zu < %zu bytes", workspace_bytes,
                moe_route_workspace(T, E));
  if (!aligned(workspace, 256)) return fail(MOE_ERR_INVALID, "workspace misaligned");
  moe::RouteArgs a;
  a.x = x;
  a.W = W;
  a.bias = bias;
  a.Wn = W_next;
  a.bias_n = W_next ? bias_next : nullptr;
  a.ids = ids;
  a.scores = scores;
  a.pred = pred_ids;
  a.table = table;
  a.slot_refs = slot_refs;
  a.miss_count = miss_count;
  a.counter = static_cast<uint32_t *>(workspace);
  a.logits = reinterpret_cast<float *>(static_cast<char *>(workspace) + 256);
  a.flagged = reinterpret_cast<uint64_t *>(static_cast<char *>(workspace) + 256);
  a.T = T;
  a.D = d_model;
  a.E = E;
  a.mode = mode;
  a.renorm = renorm;
  a.k = k;
  a.kp = W_next ? k_pred : 0;
  (void)hipGetLastError();
  moe::launch_route(a, static_cast<hipStream_t>(stream));
  MOE_HIP(hipGetLastError());
  return MOE_OK;
}

static uint64_t *g_stack_trace = nullptr;
static size_t g_stack_trace_bytes = 0;

int moe_stack_trace(void *device_buf, size_t bytes) {
  g_stack_trace = static_cast<uint64_t *>(device_buf);
  g_stack_trace_bytes = device_buf ? bytes : 0;
  return MOE_OK;
}

size_t moe_stack_workspace(const moe_geom *g, int32_t n_layers, int32_t E, int32_t k) {
  if (!g || n_layers <= 0 || E <= 0 || E > moe::kRouteMaxE || k <= 0) return 0;
  // (the workspace does not depend on the routing rule: any instantiation)
  const moe::StackLaunch *S =
      moe::find_stack(g->d_model, g->d_ff, k, g->has_proj_bias, g->act, -1, 0);
  if (!S) return 0;
  return S->ws_fixed + (size_t)n_layers * moe::kStackCounterBytesPerLayer;
}

int moe_stack_decode(const moe_pool_view *pool, const moe_geom *g, int32_t n_layers,
                     int32_t E, int32_t k, const uint16_t *x, const uint16_t *W,
                     const uint16_t *bias, int32_t mode, int32_t renorm, int32_t k_pred,
                     const int32_t *table, uint16_t *y, int32_t *ids, float *scores,
                     int32_t *slot_refs, int32_t *pred, int32_t *miss_count,
                     uint32_t epoch, int32_t flags, void *workspace,
                     size_t workspace_bytes, void *stream) {
  moe::PoolArgs pa;
  int rc = make_pool_args(pool, g, &pa);
  if (rc) return rc;
  const moe::StackLaunch *S =
      moe::find_stack(g->d_model, g->d_ff, k, g->has_proj_bias, g->act, mode, renorm);
  if (!S)
    return fail(MOE_ERR_UNSUPPORTED,
                "no persistent decode kernel for d_model=%d d_ff=%d k=%d proj_bias=%d act=%d "
                "routing=%d renorm=%d", g->d_model, g->d_ff, k, g->has_proj_bias, g->act, mode,
                renorm);
  rc = check_packed_layout(pool, g);
  if (rc) return rc;
  if (n_layers <= 0) return fail(MOE_ERR_INVALID, "n_layers=%d", n_layers);
  if (E <= 0 || E > moe::kRouteMaxE || 2 * E > S->nwg)
    return fail(MOE_ERR_INVALID, "E=%d outside [1, %d]", E, moe::kRouteMaxE);
  if (mode != MOE_ROUTE_SOFTMAX_TOPK && mode != MOE_ROUTE_TOPK_SOFTMAX)
    return fail(MOE_ERR_INVALID, "unknown routing mode %d", mode);
  if (k_pred <= 0 || k_pred > E || k_pred > 64)
    return fail(MOE_ERR_INVALID, "k_pred=%d outside [1, min(E, 64)]", k_pred);
  if (g->act != MOE_ACT_SWIGLU && g->act != MOE_ACT_SWIGLU_CLAMP)
    return fail(MOE_ERR_INVALID, "unknown activation %d", g->act);
  if (!x || !W || !table || !y || !ids || !scores || !slot_refs || !pred || !miss_count ||
      !workspace)
    return fail(MOE_ERR_INVALID, "NULL argument");
  if (!aligned(x, 16) || !aligned(W, 16) || !aligned(workspace, 256))
    return fail(MOE_ERR_INVALID, "x/W must be 16-byte and workspace 256-byte aligned");
  if (workspace_bytes < moe_stack_workspace(g, n_layers, E, k))
    return fail(MOE_ERR_INVALID, "workspace %zu < %zu bytes", workspace_bytes,
                moe_stack_workspace(g, n_layers, E, k));
  if (flags & ~MOE_STACK_ORDINARY) return fail(MOE_ERR_INVALID, "unknown flags 0x%x", flags);
  if (epoch == 0) return fail(MOE_ERR_INVALID, "epoch must start at 1");
  if ((uint64_t)epoch * (uint64_t)n_layers + (uint64_t)n_layers > 0xffffffffull)
    return fail(MOE_ERR_INVALID, "epoch %u too large for %d layers: zero the workspace and "
                "restart at 1", epoch, n_layers);
  moe::StackArgs a;
  a.pa = pa;
  a.x = x;
  a.W = W;
  a.bias = bias;
  a.table = table;
  a.y = y;
  a.ids = ids;
  a.scores = scores;
  a.refs_out = slot_refs;
  a.pred = pred;
  a.miss = miss_count;
  a.ws = static_cast<char *>(workspace);
  a.L = n_layers;
  a.E = E;
  a.kp = k_pred;
  a.mode = mode;
  a.renorm = renorm;
  a.act = g->act;
  a.alpha = g->alpha;
  a.limit = g->limit;
  a.epoch = epoch;
  a.trace = nullptr;
  if (g_stack_trace) {
    const size_t need = (size_t)moe::kTraceWGs * n_layers * moe::kTracePoints * 8;
    if (g_stack_trace_bytes < need)
      return fail(MOE_ERR_INVALID, "trace buffer %zu < %zu bytes", g_stack_trace_bytes, need);
    a.trace = g_stack_trace;
  }
  (void)hipGetLastError();
  MOE_HIP(moe::launch_stack(S, a, (flags & MOE_STACK_ORDINARY) != 0,
                            static_cast<hipStream_t>(stream)));
  return MOE_OK;
}

int moe_slot_lookup(const int32_t *table, int32_t E, const int32_t *ids,
                    int32_t n, int32_t *slot_refs, int32_t *miss_count,
                    void *stream) {
  if (n < 0 || E <= 0) return fail(MOE_ERR_INVALID, "n=%d E=%d", n, E);
  if (n == 0) return MOE_OK;
  if (!table || !ids || !slot_refs)
    return fail(MOE_ERR_INVALID, "NULL table/ids/slot_refs");
  (void)hipGetLastError();
  moe::launch_slot_lookup(table, E, ids, n, slot_refs, miss_count,
                          static_cast<hipStream_t>(stream));
  MOE_HIP(hipGetLastError());
  return MOE_OK;
}

namespace {

// Slot fills, one launch per batch of up to kFillBatch (record, slot) pairs
// carried in the kernel arguments (no index upload).  Work item y = (pair,
// chunk of the pair's record counted over its components in order),
// kFillChunk bytes, copied by 16-byte loads and stores; a grid of at most
// kFillHostGrid one-wave workgroups strides over the items when the source is
// pinned host memory.  That keeps the reads in flight over the host link to
// 256 KiB (enough for its rate): every read queued there delays whatever
// else crosses it, among them the command processor's fetch of the next
// dispatch of every other stream.  One wave per workgroup spreads the fill
// thinly over the CUs, so that no decode workgroup sharing a CU with it
// waits long behind its outstanding loads.  An HBM source gets a 256-thread
// workgroup per item.
constexpr int kFillBatch = 160;
constexpr int64_t kFillChunk = 64 * 1024;
constexpr int kFillHostGrid = 128, kFillHostThreads = 64, kFillHostLoads = 2;

struct FillArgs {
  char *base[MOE_MAX_COMPONENTS];
  int64_t slot_bytes[MOE_MAX_COMPONENTS];
  int64_t src_offset[MOE_MAX_COMPONENTS];
  int32_t chunk0[MOE_MAX_COMPONENTS + 1];   // first chunk of each component
  const char *src;
  int64_t record_bytes;
  int32_t nc, n;
  int32_t slot[kFillBatch];
  int64_t rec[kFillBatch];
};

extern "C++" {
template <int NT, int U>
__global__ __launch_bounds__(NT) void fill_slots_kernel(const FillArgs a) {
  const int chunks = a.chunk0[a.nc];
  for (int item = blockIdx.x; item < a.n * chunks; item += gridDim.x) {
    const int i = item / chunks, y = item % chunks;
    int c = 0;
    while (c + 1 < a.nc && y >= a.chunk0[c + 1]) ++c;
    const int64_t off = (int64_t)(y - a.chunk0[c]) * kFillChunk;
    const int64_t len = min(kFillChunk, a.slot_bytes[c] - off);
    const uint4 *s = reinterpret_cast<const uint4 *>(a.src + a.rec[i] * a.record_bytes +
                                                     a.src_offset[c] + off);
    uint4 *d = reinterpret_cast<uint4 *>(a.base[c] + (int64_t)a.slot[i] * a.slot_bytes[c] + off);
    const int n16 = (int)(len / 16);
    int j = threadIdx.x;
    for (; j + (U - 1) * NT < n16; j += U * NT) {
      uint4 v[U];
#pragma unroll
      for (int u = 0; u < U; ++u) v[u] = s[j + u * NT];
#pragma unroll
      for (int u = 0; u < U; ++u) d[j + u * NT] = v[u];
    }
    for (; j < n16; j += NT) d[j] = s[j];
  }
}
}  // extern "C++"

// The address a kernel reads `p` through: device memory as is, pinned host
// memory (hipHostMalloc) through its device mapping (*host = true); nullptr
// for pageable host memory, which only a copy engine can read.
const char *kernel_address(const void *p, bool *host) {
  hipPointerAttribute_t at;
  *host = false;
  if (hipPointerGetAttributes(&at, p) != hipSuccess) {
    (void)hipGetLastError();
    return nullptr;
  }
  if (at.type == hipMemoryTypeDevice) return static_cast<const char *>(p);
  if (at.type == hipMemoryTypeHost && at.devicePointer) {
    *host = true;
    return static_cast<const char *>(at.devicePointer);
  }
  return nullptr;
}

// The record layout: component c at base + comp_offset[c] with slot stride
// `rb` for every c, so slot s holds one whole record at base + s * rb.
bool record_layout(const moe_pool_view *pool, int64_t rb) {
  const char *b0 = static_cast<const char *>(pool->base[0]) - pool->comp_offset[0];
  for (int c = 0; c < pool->n_components; ++c)
    if (pool->slot_bytes[c] != rb ||
        static_cast<const char *>(pool->base[c]) - pool->comp_offset[c] != b0)
      return false;
  return pool->n_slots > 0;
}

}  // namespace

int moe_fill_slots(const moe_pool_view *pool, const void *src_store,
                   int64_t src_record_bytes, int64_t src_n_records,
                   const int64_t *src_records, const int32_t *dst_slots, int32_t n,
                   void *stream) {
  if (!pool) return fail(MOE_ERR_INVALID, "pool view is NULL");
  if (n < 0) return fail(MOE_ERR_INVALID, "n < 0");
  if (n == 0) return MOE_OK;
  if (!src_records || !dst_slots) return fail(MOE_ERR_INVALID, "NULL index arrays");
  const char *src = static_cast<const char *>(src_store ? src_store : pool->store);
  const int64_t rb = src_store ? src_record_bytes : pool->record_bytes;
  const int64_t nrec = src_store ? src_n_records : pool->n_records;
  if (!src || rb <= 0) return fail(MOE_ERR_INVALID, "no source store");
  if (nrec <= 0) return fail(MOE_ERR_INVALID, "source store of %lld records", (long long)nrec);
  const int nc = pool->n_components;
  if (nc != 9 && nc != 12) return fail(MOE_ERR_INVALID, "n_components=%d", nc);
  hipStream_t s = static_cast<hipStream_t>(stream);
  for (int32_t i = 0; i < n; ++i) {
    const int32_t slot = dst_slots[i];
    const int64_t rec = src_records[i];
    if (slot < 0 || slot >= pool->n_slots)
      return fail(MOE_ERR_INVALID, "slot %d outside [0, %d)", slot, pool->n_slots);
    if (rec < 0 || rec >= nrec)
      return fail(MOE_ERR_INVALID, "record %lld outside [0, %lld)", (long long)rec,
                  (long long)nrec);
  }
  // A pool in the record layout (every component at its record offset from
  // one base, slot stride = the source's record size) holds each slot's
  // record contiguously: one hipMemcpyAsync per record, which the copy
  // engines carry out without occupying compute units.
  if (record_layout(pool, rb)) {
    char *base = static_cast<char *>(pool->base[0]) - pool->comp_offset[0];
    for (int32_t i = 0; i < n; ++i)
      MOE_HIP(hipMemcpyAsync(base + (int64_t)dst_slots[i] * rb, src + src_records[i] * rb,
                             (size_t)rb, hipMemcpyDefault, s));
    return MOE_OK;
  }
  // Copy kernels for a source the GPU can read (HBM, or pinned host memory
  // over the link: one launch per batch instead of a copy call per
  // component, whose host-side cost dominated the streaming loop) with
  // 16-byte aligned pieces; pageable memory goes through hipMemcpyAsync.
  bool host_src = false;
  const char *ksrc = kernel_address(src, &host_src);
  bool kernel = ksrc != nullptr && aligned(ksrc, 16) && rb % 16 == 0;
  FillArgs fa{};
  int32_t chunks = 0;
  for (int c = 0; c < nc && kernel; ++c) {
    kernel = aligned(pool->base[c], 16) && pool->slot_bytes[c] % 16 == 0 &&
             pool->comp_offset[c] % 16 == 0 && pool->comp_offset[c] + pool->slot_bytes[c] <= rb;
    fa.base[c] = static_cast<char *>(pool->base[c]);
    fa.slot_bytes[c] = pool->slot_bytes[c];
    fa.src_offset[c] = pool->comp_offset[c];
    fa.chunk0[c] = chunks;
    chunks += (int32_t)((pool->slot_bytes[c] + kFillChunk - 1) / kFillChunk);
  }
  if (kernel) {
    fa.chunk0[nc] = chunks;
    fa.src = ksrc;
    fa.record_bytes = rb;
    fa.nc = nc;
    for (int32_t i0 = 0; i0 < n; i0 += kFillBatch) {
      fa.n = std::min<int32_t>(kFillBatch, n - i0);
      for (int32_t i = 0; i < fa.n; ++i) {
        fa.slot[i] = dst_slots[i0 + i];
        fa.rec[i] = src_records[i0 + i];
      }
      const int64_t items = (int64_t)fa.n * chunks;
      if (host_src)
        hipLaunchKernelGGL((fill_slots_kernel<kFillHostThreads, kFillHostLoads>),
                           dim3((int)std::min<int64_t>(items, kFillHostGrid)),
                           dim3(kFillHostThreads), 0, s, fa);
      else
        hipLaunchKernelGGL((fill_slots_kernel<256, 4>), dim3((int)items), dim3(256), 0, s, fa);
      MOE_HIP(hipGetLastError());
    }
    return MOE_OK;
  }
  for (int32_t i = 0; i < n; ++i) {
    const int32_t slot = dst_slots[i];
    const int64_t rec = src_records[i];
    for (int c = 0; c < nc; ++c) {
      // each component's size is its slot stride in the pool
      MOE_HIP(hipMemcpyAsync(static_cast<char *>(pool->base[c]) + slot * pool->slot_bytes[c],
                             src + rec * rb + pool->comp_offset[c],
                             (size_t)pool->slot_bytes[c], hipMemcpyDefault, s));
    }
  }
  return MOE_OK;
}

int moe_host_alloc(size_t bytes, void **out) {
  if (!out) return fail(MOE_ERR_INVALID, "out is NULL");
  *out = nullptr;
  if (bytes == 0) return fail(MOE_ERR_INVALID, "zero-byte allocation");
  MOE_HIP(hipHostMalloc(out, bytes, hipHostMallocDefault));
  return MOE_OK;
}

int moe_host_free(void *p) {
  if (!p) return MOE_OK;
  MOE_HIP(hipHostFree(p));
  return MOE_OK;
}

int moe_event_create(void **ev) {
  if (!ev) return fail(MOE_ERR_INVALID, "ev is NULL");
  hipEvent_t e;
  MOE_HIP(hipEventCreateWithFlags(&e, hipEventDefault));
  *ev = e;
  return MOE_OK;
}

int moe_event_destroy(void *ev) {
  if (!ev) return MOE_OK;
  MOE_HIP(hipEventDestroy(static_cast<hipEvent_t>(ev)));
  return MOE_OK;
}

int moe_event_record(void *ev, void *stream) {
  if (!ev) return fail(MOE_ERR_INVALID, "ev is NULL");
  MOE_HIP(hipEventRecord(static_cast<hipEvent_t>(ev), static_cast<hipStream_t>(stream)));
  return MOE_OK;
}

int moe_event_query(void *ev) {
  if (!ev) return fail(MOE_ERR_INVALID, "ev is NULL");
  hipError_t e = hipEventQuery(static_cast<hipEvent_t>(ev));
  if (e == hipSuccess) return 1;
  if (e == hipErrorNotReady) {
    (void)hipGetLastError();
    return 0;
  }
  return hip_fail(e, "hipEventQuery");
}

int moe_stream_wait_event(void *stream, void *ev) {
  if (!ev) return fail(MOE_ERR_INVALID, "ev is NULL");
  MOE_HIP(hipStreamWaitEvent(static_cast<hipStream_t>(stream), static_cast<hipEvent_t>(ev), 0));
  return MOE_OK;
}

int moe_event_elapsed_ms(void *start, void *stop, float *ms) {
  if (!start || !stop || !ms) return fail(MOE_ERR_INVALID, "NULL argument");
  MOE_HIP(hipEventElapsedTime(ms, static_cast<hipEvent_t>(start), static_cast<hipEvent_t>(stop)));
  return MOE_OK;
}

int moe_check_device_error(void *stream) {
  MOE_HIP(hipStreamSynchronize(static_cast<hipStream_t>(stream)));
  int v = 0;
  MOE_HIP(hipMemcpyFromSymbol(&v, HIP_SYMBOL(moe::g_device_error), sizeof(int), 0,
                              hipMemcpyDeviceToHost));
  if (v) {
    const int zero = 0;
    MOE_HIP(hipMemcpyToSymbol(HIP_SYMBOL(moe::g_device_error), &zero, sizeof(int), 0,
                              hipMemcpyHostToDevice));
    if (v & moe::kErrTimeout)
      return fail(MOE_ERR_TIMEOUT,
                  "a kernel's wait for another workgroup gave up (its grid was not resident "
                  "at once: another kernel held CUs of the device)%s",
                  (v & moe::kErrBadRef) ? "; a kernel also resolved an out-of-range slot "
                                          "reference" : "");
    return fail(MOE_ERR_DEVICE, "a kernel resolved an out-of-range slot reference");
  }
  return MOE_OK;
}

}  // extern "C"
