// Router, top-k, lookahead and slot lookup for a few tokens, one launch.
//
// Phase 1 (every workgroup): one wave per router row computes the fp32 dot
// x_t . W[e] for each token (bf16 pairs through v_dot2c_f32_bf16), all of
// the row's 16-byte loads issued before any arithmetic, and publishes it as
// an 8-byte device-scope entry (this launch's flag, fp32 logit).  Rows
// 0..E-1 are this layer's router, rows E..2E-1 the next layer's router
// (lookahead), when present.
// Phase 2 (workgroup 0, after its own rows): one wave per (token,
// router|lookahead) task polls that task's E entries until all carry the
// launch's flag, then turns the logits into bf16 logits, softmax and ranking
// entirely in registers -- two experts per lane, DPP reductions, k rounds of
// a packed (order-preserving 16-bit key, inverted id) integer wave max --
// and writes ids, scores, lookahead ids and the slot-table lookup.  The
// flag is the workspace's sequence word + 1; workgroup 0 stores it back
// once it has seen every entry, so the workspace needs zeroing only once.
// Workgroup 0 waits only for workgroups dispatched after it, which never
// wait for anything, and its polls are bounded (device error word).
// Many tokens (prefill, T > 16): the logits come from a bf16 MFMA kernel and a
// second kernel runs the same per-task selection.
//
// Reference semantics: top_k_experts (engine_v3.py:467-473), top_k_route
// (engine_120b.py:65-70), top_k_indices (engine_v3.py:476-483,
// engine_120b.py:73-75), slot lookup (engine_v3.py:548-552).  Ranking is
// value-descending with ties to the lower expert id (argpartition leaves the
// order of ties unspecified).
#include <algorithm>

#include "launchers.h"

namespace moe {

// bf16-representable float -> 16-bit key whose unsigned order is the float
// order (negative values flipped).
__device__ __forceinline__ int order_key(float v) {
  const uint32_t b = __float_as_uint(v) >> 16;
  return (b & 0x8000u) ? (int)(~b & 0xffffu) : (int)(b | 0x8000u);
}

__device__ __forceinline__ int popc64(uint64_t m) { return __popcll(m); }

// Top-kk of 2*64 candidates (e0 = lane, e1 = lane + 64; key < 0 = absent),
// ordered by key descending then index ascending.  Returns each lane's
// selection flags and, for selected entries, their rank.  Key and inverted
// index are packed into one int, so a single integer max picks the largest
// key and, among equal keys, the smallest index; kk rounds of a DPP wave max.
__device__ void select_topk(int key0, int key1, int kk, int lane, bool &sel0,
                            bool &sel1, int &rank0, int &rank1) {
  int p0 = key0 >= 0 ? (key0 << 8) | (255 - lane) : -1;
  int p1 = key1 >= 0 ? (key1 << 8) | (255 - (lane + 64)) : -1;
  sel0 = sel1 = false;
  rank0 = rank1 = 0;
  for (int r = 0; r < kk; ++r) {
    const int m = wave_max_i(max(p0, p1));
    if (m < 0) break;                        // fewer candidates than kk
    if (p0 == m) { sel0 = true; rank0 = r; p0 = -1; }
    if (p1 == m) { sel1 = true; rank1 = r; p1 = -1; }
  }
}

// One selection task on one wave: task < T is token t's routing (ids, scores,
// slot refs, misses), task >= T token t's lookahead prediction.  The logits
// are read with device-scope loads: in route_kernel another workgroup of the
// same launch wrote them.
// Per-task inputs loaded before the logits arrive: the bias and slot table
// entries of both candidates (clamped indices, unconditional loads).
struct TaskPre {
  float b0, b1;
  int32_t t0, t1;
};
__device__ __forceinline__ TaskPre task_pre(const RouteArgs &a, int task, int lane) {
  const bool la = task >= a.T;
  const int E = a.E, e0 = min(lane, E - 1), e1 = min(lane + 64, E - 1);
  const uint16_t *bias = la ? a.bias_n : a.bias;
  const bool tab = !la && a.table != nullptr;
  TaskPre p;
  p.b0 = bias ? bf16_to_f32(bias[e0]) : 0.f;
  p.b1 = bias ? bf16_to_f32(bias[e1]) : 0.f;
  p.t0 = tab ? a.table[e0] : 0;
  p.t1 = tab ? a.table[e1] : 0;
  return p;
}

// l0, l1: the raw router logits of experts lane and lane + 64.
__device__ void select_task(const RouteArgs &a, int task, int lane, const TaskPre &p,
                            float l0, float l1) {
  const int E = a.E;
  const int t = task % a.T;
  const bool la = task >= a.T;
  const int e0 = lane, e1 = lane + 64;
  const int32_t t0 = p.t0, t1 = p.t1;
  const float z0 = e0 < E ? round_bf16(l0 + p.b0) : -INFINITY;
  const float z1 = e1 < E ? round_bf16(l1 + p.b1) : -INFINITY;
  // ranked quantity: bf16 softmax probabilities (SOFTMAX_TOPK router) or
  // the bf16 logits (TOPK_SOFTMAX router, and every lookahead)
  float v0 = z0, v1 = z1;
  if (!la && a.mode == MOE_ROUTE_SOFTMAX_TOPK) {
    const float m = wave_max(fmaxf(z0, z1));
    const float x0 = (e0 < E) ? expf(z0 - m) : 0.f;
    const float x1 = (e1 < E) ? expf(z1 - m) : 0.f;
    const float s = group_sum<64>(x0 + x1);
    v0 = round_bf16(x0 / s);
    v1 = round_bf16(x1 / s);
  }
  const int kk = la ? a.kp : a.k;
  bool sel0, sel1;
  int r0, r1;
  select_topk(e0 < E ? order_key(v0) : -1, e1 < E ? order_key(v1) : -1, kk, lane, sel0,
              sel1, r0, r1);
  if (la) {
    if (sel0) a.pred[(int64_t)t * a.kp + r0] = e0;
    if (sel1) a.pred[(int64_t)t * a.kp + r1] = e1;
    return;
  }
  // scores of the selected experts
  float sc0 = 0.f, sc1 = 0.f;
  if (a.mode == MOE_ROUTE_SOFTMAX_TOPK) {
    sc0 = v0;
    sc1 = v1;
    if (a.renorm) {
      const float tot = round_bf16(group_sum<64>((sel0 ? v0 : 0.f) + (sel1 ? v1 : 0.f)));
      sc0 = round_bf16(v0 / tot);
      sc1 = round_bf16(v1 / tot);
    }
  } else {
    const float m = wave_max(fmaxf(sel0 ? z0 : -INFINITY, sel1 ? z1 : -INFINITY));
    const float x0 = sel0 ? expf(z0 - m) : 0.f;
    const float x1 = sel1 ? expf(z1 - m) : 0.f;
    const float s = group_sum<64>(x0 + x1);
    sc0 = round_bf16(x0 / s);
    sc1 = round_bf16(x1 / s);
  }
  bool miss0 = false, miss1 = false;
  const int64_t o0 = (int64_t)t * a.k + r0, o1 = (int64_t)t * a.k + r1;
  if (sel0) {
    a.ids[o0] = e0;
    a.scores[o0] = sc0;
    if (a.table) {
      a.slot_refs[o0] = t0;
      miss0 = t0 < 0;
    }
  }
  if (sel1) {
    a.ids[o1] = e1;
    a.scores[o1] = sc1;
    if (a.table) {
      a.slot_refs[o1] = t1;
      miss1 = t1 < 0;
    }
  }
  if (a.miss_count) {
    const int m = popc64(__ballot(miss0)) + popc64(__ballot(miss1));
    if (lane == 0 && m) atomicAdd(a.miss_count, m);
  }
}

template <int NIT>
__device__ __forceinline__ void router_rows(const RouteArgs &a, int row, int lane,
                                            uint32_t fl) {
  const bool nxt = row >= a.E;
  const int e = nxt ? row - a.E : row;
  const int n8 = a.D / 8;
  const uint4 *w4 = reinterpret_cast<const uint4 *>((nxt ? a.Wn : a.W) + (int64_t)e * a.D);
  uint4 w[NIT];
#pragma unroll
  for (int it = 0; it < NIT; ++it) {
    const int i = lane + it * 64;
    w[it] = (i < n8) ? load_stream16(w4 + i) : make_uint4(0, 0, 0, 0);
  }
  // the next token's activations load while this one's dot product runs
  uint4 vn[NIT];
  auto load_x = [&](int t) {
    const uint4 *x4 = reinterpret_cast<const uint4 *>(a.x + (int64_t)min(t, a.T - 1) * a.D);
#pragma unroll
    for (int it = 0; it < NIT; ++it)
      vn[it] = x4[min(lane + it * 64, n8 - 1)];   // unconditional, masked below
  };
  load_x(0);
  for (int t = 0; t < a.T; ++t) {
    uint4 v[NIT];
#pragma unroll
    for (int it = 0; it < NIT; ++it)
      v[it] = (lane + it * 64 < n8) ? vn[it] : make_uint4(0, 0, 0, 0);
    load_x(t + 1);
    float acc = 0.f;
#pragma unroll
    for (int it = 0; it < NIT; ++it) {
      acc = dot2_bf16(w[it].x, v[it].x, acc);
      acc = dot2_bf16(w[it].y, v[it].y, acc);
      acc = dot2_bf16(w[it].z, v[it].z, acc);
      acc = dot2_bf16(w[it].w, v[it].w, acc);
    }
    acc = group_sum<64>(acc);
    // device-scope store of (flag, logit): read by workgroup 0 on another
    // CU/XCD, whose poll of the entry is its load
    if (lane == 0)
      __hip_atomic_store(&a.flagged[((nxt ? 1 : 0) * a.T + t) * a.E + e],
                         ((uint64_t)fl << 32) | __float_as_uint(acc), __ATOMIC_RELAXED,
                         __HIP_MEMORY_SCOPE_AGENT);
  }
}

// Workgroup 0's wait for one task's E flagged logits: device-scope loads of
// both entries of every lane until all carry this launch's flag; bounded,
// a timeout sets the device error word.
__device__ __forceinline__ void poll_logits(const uint64_t *lg, int E, uint32_t fl, int lane,
                                            float &l0, float &l1) {
  const int e0 = min(lane, E - 1), e1 = min(lane + 64, E - 1);
  for (uint32_t spins = 0;; ++spins) {
    const uint64_t v0 = __hip_atomic_load(lg + e0, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    const uint64_t v1 = __hip_atomic_load(lg + e1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    l0 = __uint_as_float((uint32_t)v0);
    l1 = __uint_as_float((uint32_t)v1);
    const bool ok = (uint32_t)(v0 >> 32) == fl && (uint32_t)(v1 >> 32) == fl;
    if (__all(ok)) return;
    if (spins > kRouteSpinLimit) {
      if (lane == 0) flag_timeout();
      return;
    }
    __builtin_amdgcn_s_sleep(1);
  }
}

template <int NIT>
__global__ __launch_bounds__(256) void route_kernel(RouteArgs a) {
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  // this launch's flag: the workspace's sequence word + 1.  Workgroup 0
  // stores it back only after it has seen every row's entry, and every
  // writer reads the word before it writes, so all writers agree.
  const uint32_t fl =
      __hip_atomic_load(a.counter, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) + 1u;
  const int nrows = a.E * (a.Wn ? 2 : 1);
  const int ntask = a.T * (a.Wn ? 2 : 1);
  // Workgroup 0's own tasks see every router row (task 0) and, when T < 4,
  // every lookahead row (task T), so every writer of those has read the word
  // before workgroup 0 advances it.  Otherwise -- lookahead rows with T >= 4,
  // or workgroups that only rank (more tasks than rows) -- every workgroup
  // counts itself in once it holds the word's value, and workgroup 0 waits
  // for all of them before it advances the word.
  const bool count_in = (int)gridDim.x > (nrows + 3) / 4 || (a.Wn != nullptr && a.T >= 4);
  uint32_t *const arrived = a.counter + kRouteArrivedWord;
  if (count_in && threadIdx.x == 0) {
    uint32_t one = 1u;
    asm volatile("" : "+v"(one) : "v"(fl));   // issued once the word's value is in
    __hip_atomic_fetch_add(arrived, one, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  }
  const int row = blockIdx.x * 4 + wave;
  if (row < nrows) router_rows<NIT>(a, row, lane, fl);

  // ---- ranking: one wave per (token, router|lookahead) task, on the first
  // workgroups.  The logits travel as flagged device-scope (sc1) entries,
  // coherent across XCDs without L2 writeback/invalidate; the poll of an
  // entry is its load.
  const int task = blockIdx.x * 4 + wave;
  if (task < ntask) {
    const TaskPre p = task_pre(a, task, lane);
    const bool la = task >= a.T;
    float l0, l1;
    poll_logits(a.flagged + ((int64_t)(la ? 1 : 0) * a.T + task % a.T) * a.E, a.E, fl, lane,
                l0, l1);
    select_task(a, task, lane, p, l0, l1);
  }
  // Workgroup 0 advances the sequence word once no workgroup of this launch
  // can still read it: its tasks have seen the entries of every writer (each
  // read the word before writing), or, with count_in, every workgroup has
  // counted itself in.  The arrival word is back at zero for the next launch.
  if (blockIdx.x != 0) return;
  __syncthreads();
  if (threadIdx.x == 0) {
    if (count_in) {
      for (uint32_t spins = 0;
           __hip_atomic_load(arrived, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) < gridDim.x;
           ++spins) {
        if (spins > kRouteSpinLimit) {
          flag_timeout();
          break;
        }
        __builtin_amdgcn_s_sleep(1);
      }
      __hip_atomic_store(arrived, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    }
    __hip_atomic_store(a.counter, fl, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  }
}

// ---------------------------------------------------------------------------
// Many tokens (T > kRouteMaxT): the logits as a bf16 MFMA product.  One
// workgroup = 16 tokens x 16 router rows; its 4 waves take interleaved
// 32-input steps of K (v_mfma_f32_16x16x32_bf16: A = x rows, lane row l%16,
// inputs 8*(l/16)..+7 of the step; B = router rows) and the four fp32
// partial products are summed in a fixed order through LDS.
// blockIdx.y >= ceil(E/16) selects the lookahead router.
// ---------------------------------------------------------------------------
typedef __bf16 bf16x8_t __attribute__((ext_vector_type(8)));
typedef float f32x4_t __attribute__((ext_vector_type(4)));

__global__ __launch_bounds__(256) void route_logits_mfma_kernel(RouteArgs a) {
  __shared__ float part[4][16][17];
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int eblocks = (a.E + 15) / 16;
  const bool la = blockIdx.y >= eblocks;
  const int t0 = blockIdx.x * 16, e0 = (blockIdx.y - (la ? eblocks : 0)) * 16;
  const int row = lane & 15, kq = lane >> 4;
  const uint4 *xa =
      reinterpret_cast<const uint4 *>(a.x + (int64_t)min(t0 + row, a.T - 1) * a.D) + kq;
  const uint4 *wb = reinterpret_cast<const uint4 *>((la ? a.Wn : a.W) +
                                                    (int64_t)min(e0 + row, a.E - 1) * a.D) + kq;
  f32x4_t acc = {0.f, 0.f, 0.f, 0.f};
  const int nk = a.D / 32;
  int k = wave;
  for (; k + 12 < nk; k += 16) {   // four steps per iteration, loads first
    uint4 xv[4], wv[4];
#pragma unroll
    for (int u = 0; u < 4; ++u) {
      xv[u] = xa[(k + 4 * u) * 4];
      wv[u] = wb[(k + 4 * u) * 4];
    }
#pragma unroll
    for (int u = 0; u < 4; ++u)
      acc = __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(bf16x8_t, xv[u]),
                                                    __builtin_bit_cast(bf16x8_t, wv[u]), acc,
                                                    0, 0, 0);
  }
  for (; k < nk; k += 4)
    acc = __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(bf16x8_t, xa[k * 4]),
                                                  __builtin_bit_cast(bf16x8_t, wb[k * 4]), acc,
                                                  0, 0, 0);
  // lane holds router row e0 + l%16 for tokens t0 + 4*(l/16) + r
#pragma unroll
  for (int r = 0; r < 4; ++r) part[wave][4 * kq + r][row] = acc[r];
  __syncthreads();
  if (wave == 0) {
    float *lg = a.logits + (int64_t)(la ? 1 : 0) * a.T * a.E;
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      const int tt = 4 * kq + r, t = t0 + tt, e = e0 + row;
      const float v = (part[0][tt][row] + part[1][tt][row]) + (part[2][tt][row] + part[3][tt][row]);
      if (t < a.T && e < a.E) lg[(int64_t)t * a.E + e] = v;
    }
  }
}

// one wave per selection task, after route_logits_mfma_kernel
__global__ __launch_bounds__(256) void route_select_kernel(RouteArgs a) {
  const int task = blockIdx.x * 4 + (threadIdx.x >> 6), lane = threadIdx.x & 63;
  if (task >= a.T * (a.Wn ? 2 : 1)) return;
  const TaskPre p = task_pre(a, task, lane);
  const float *lg = a.logits + ((int64_t)(task >= a.T ? 1 : 0) * a.T + task % a.T) * a.E;
  const float l0 = lg[min(lane, a.E - 1)], l1 = lg[min(lane + 64, a.E - 1)];
  select_task(a, task, lane, p, l0, l1);
}

__global__ void slot_lookup_kernel(const int32_t *table, int E,
                                   const int32_t *ids, int n, int32_t *refs,
                                   int32_t *miss_count) {
  const int i = blockIdx.x * blockDim.x + threadIdx.x;
  if (i >= n) return;
  const int e = ids[i];
  int32_t ref = 0;
  if (e < 0 || e >= E) {
    flag_error();
  } else {
    ref = table[e];
  }
  refs[i] = ref;
  if (miss_count && ref < 0) atomicAdd(miss_count, 1);
}

void launch_route(const RouteArgs &a, hipStream_t s) {
  if (a.T > kRouteMaxT) {
    const int eblocks = (a.E + 15) / 16;
    hipLaunchKernelGGL(route_logits_mfma_kernel, dim3((a.T + 15) / 16, eblocks * (a.Wn ? 2 : 1)),
                       dim3(256), 0, s, a);
    const int ntask = a.T * (a.Wn ? 2 : 1);
    hipLaunchKernelGGL(route_select_kernel, dim3((ntask + 3) / 4), dim3(256), 0, s, a);
    return;
  }
  const int nrows = a.E * (a.Wn ? 2 : 1);
  const int ntask = a.T * (a.Wn ? 2 : 1);
  const int nit = (a.D / 8 + 63) / 64;
  dim3 g((std::max(nrows, ntask) + 3) / 4), b(256);
  switch (nit) {
    case 1: hipLaunchKernelGGL(route_kernel<1>, g, b, 0, s, a); break;
    case 2: hipLaunchKernelGGL(route_kernel<2>, g, b, 0, s, a); break;
    case 3: hipLaunchKernelGGL(route_kernel<3>, g, b, 0, s, a); break;
    case 4: hipLaunchKernelGGL(route_kernel<4>, g, b, 0, s, a); break;
    case 5: hipLaunchKernelGGL(route_kernel<5>, g, b, 0, s, a); break;
    case 6: hipLaunchKernelGGL(route_kernel<6>, g, b, 0, s, a); break;
    case 7: hipLaunchKernelGGL(route_kernel<7>, g, b, 0, s, a); break;
    default: hipLaunchKernelGGL(route_kernel<8>, g, b, 0, s, a); break;
  }
}

void launch_slot_lookup(const int32_t *table, int E, const int32_t *ids, int n,
                        int32_t *refs, int32_t *miss_count, hipStream_t s) {
  if (n <= 0) return;
  hipLaunchKernelGGL(slot_lookup_kernel, dim3((n + 255) / 256), dim3(256), 0,
                     s, table, E, ids, n, refs, miss_count);
}

}  // namespace moe
