// Router, top-k, lookahead and slot lookup for a few tokens, one launch.
//
// Phase 1 (every workgroup): one wave per router row computes the fp32 dot
// x_t . W[e] for each token (bf16 pairs through v_dot2c_f32_bf16) and stores
// it to the workspace.  Rows 0..E-1 are this layer's router, rows E..2E-1 the
// next layer's router (lookahead), when present.
// Phase 2 (the last workgroup to finish, found with an acq_rel counter):
// bf16 logits, softmax / ranking, scores, lookahead ids and the slot-table
// lookup.  The counter is returned to zero by that workgroup, so the
// workspace needs zeroing only once.
//
// Reference semantics: top_k_experts (engine_v3.py:467-473), top_k_route
// (engine_120b.py:65-70), top_k_indices (engine_v3.py:476-483,
// engine_120b.py:73-75), slot lookup (engine_v3.py:548-552).  Ranking is
// value-descending with ties to the lower expert id (argpartition leaves the
// order of ties unspecified).
#include "launchers.h"

namespace moe {


// rank of element e among n values in LDS: count of values ranked before it
__device__ __forceinline__ int rank_of(const float *v, int n, int e) {
  const float me = v[e];
  int r = 0;
  for (int i = 0; i < n; ++i) {
    const float o = v[i];
    r += (o > me) || (o == me && i < e);
  }
  return r;
}

__global__ __launch_bounds__(256) void route_kernel(RouteArgs a) {
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int nrows = a.E * (a.Wn ? 2 : 1);
  const int row = blockIdx.x * 4 + wave;
  const int n8 = a.D / 8;  // uint4 per row

  if (row < nrows) {
    const bool nxt = row >= a.E;
    const int e = nxt ? row - a.E : row;
    const uint4 *w4 =
        reinterpret_cast<const uint4 *>((nxt ? a.Wn : a.W) + (int64_t)e * a.D);
    for (int t = 0; t < a.T; ++t) {
      const uint4 *x4 = reinterpret_cast<const uint4 *>(a.x + (int64_t)t * a.D);
      float acc = 0.f;
      for (int i = lane; i < n8; i += 64) {
        const uint4 w = w4[i], v = x4[i];
        acc = dot2_bf16(w.x, v.x, acc);
        acc = dot2_bf16(w.y, v.y, acc);
        acc = dot2_bf16(w.z, v.z, acc);
        acc = dot2_bf16(w.w, v.w, acc);
      }
      acc = group_sum<64>(acc);
      if (lane == 0) a.logits[((nxt ? 1 : 0) * a.T + t) * a.E + e] = acc;
    }
  }

  // ---- last workgroup does the selection --------------------------------
  __shared__ int s_last;
  __threadfence();
  __syncthreads();
  if (threadIdx.x == 0) {
    const uint32_t prev = __hip_atomic_fetch_add(
        a.counter, 1u, __ATOMIC_ACQ_REL, __HIP_MEMORY_SCOPE_AGENT);
    s_last = (prev == gridDim.x - 1);
  }
  __syncthreads();
  if (!s_last) return;
  __threadfence();

  __shared__ float v[2][kRouteMaxE];   // ranked quantity
  __shared__ float z[kRouteMaxE];      // bf16 logits of this layer
  __shared__ float red[8];
  __shared__ int sel[MOE_MAX_TOPK];
  const int E = a.E;
  const int tid = threadIdx.x;
  const bool router_thr = tid < E;                       // threads 0..E-1
  const bool la_thr = a.Wn && tid >= 128 && tid - 128 < E;  // 128..128+E-1

  for (int t = 0; t < a.T; ++t) {
    float zl = -INFINITY;
    if (router_thr) {
      float l = __hip_atomic_load(&a.logits[t * E + tid], __ATOMIC_RELAXED,
                                  __HIP_MEMORY_SCOPE_AGENT);
      if (a.bias) l += bf16_to_f32(a.bias[tid]);
      zl = round_bf16(l);
      z[tid] = zl;
    }
    if (la_thr) {
      const int e = tid - 128;
      float l = __hip_atomic_load(&a.logits[(a.T + t) * E + e],
                                  __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
      if (a.bias_n) l += bf16_to_f32(a.bias_n[e]);
      v[1][e] = round_bf16(l);
    }
    // softmax over all E for the SOFTMAX_TOPK rule (fp32, precise)
    if (a.mode == MOE_ROUTE_SOFTMAX_TOPK) {
      float m = zl;
      for (int off = 32; off >= 1; off >>= 1) m = fmaxf(m, __shfl_xor(m, off, 64));
      if (lane == 0) red[wave] = m;
      __syncthreads();
      m = fmaxf(fmaxf(red[0], red[1]), fmaxf(red[2], red[3]));
      __syncthreads();
      float ex = router_thr ? expf(zl - m) : 0.f;
      float s = group_sum<64>(ex);
      if (lane == 0) red[4 + wave] = s;
      __syncthreads();
      s = (red[4] + red[5]) + (red[6] + red[7]);
      if (router_thr) v[0][tid] = round_bf16(ex / s);
    } else if (router_thr) {
      v[0][tid] = zl;
    }
    __syncthreads();

    if (router_thr) {
      const int r = rank_of(v[0], E, tid);
      if (r < a.k) sel[r] = tid;
    }
    if (la_thr) {
      const int e = tid - 128;
      const int r = rank_of(v[1], E, e);
      if (r < a.kp) a.pred[t * a.kp + r] = e;
    }
    __syncthreads();

    if (tid == 0) {
      float sc[MOE_MAX_TOPK];
      if (a.mode == MOE_ROUTE_SOFTMAX_TOPK) {
        float tot = 0.f;
        for (int r = 0; r < a.k; ++r) {
          sc[r] = v[0][sel[r]];
          tot += sc[r];
        }
        if (a.renorm) {
          tot = round_bf16(tot);
          for (int r = 0; r < a.k; ++r) sc[r] = round_bf16(sc[r] / tot);
        }
      } else {
        const float m = z[sel[0]];
        float tot = 0.f;
        for (int r = 0; r < a.k; ++r) {
          sc[r] = expf(z[sel[r]] - m);
          tot += sc[r];
        }
        for (int r = 0; r < a.k; ++r) sc[r] = round_bf16(sc[r] / tot);
      }
      int misses = 0;
      for (int r = 0; r < a.k; ++r) {
        a.ids[t * a.k + r] = sel[r];
        a.scores[t * a.k + r] = sc[r];
        if (a.table) {
          const int32_t ref = a.table[sel[r]];
          a.slot_refs[t * a.k + r] = ref;
          misses += ref < 0;
        }
      }
      if (a.miss_count && misses) atomicAdd(a.miss_count, misses);
    }
    __syncthreads();
  }
  if (tid == 0)
    __hip_atomic_store(a.counter, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
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
  const int nrows = a.E * (a.Wn ? 2 : 1);
  hipLaunchKernelGGL(route_kernel, dim3((nrows + 3) / 4), dim3(256), 0, s, a);
}

void launch_slot_lookup(const int32_t *table, int E, const int32_t *ids, int n,
                        int32_t *refs, int32_t *miss_count, hipStream_t s) {
  if (n <= 0) return;
  hipLaunchKernelGGL(slot_lookup_kernel, dim3((n + 255) / 256), dim3(256), 0,
                     s, table, E, ids, n, refs, miss_count);
}

}  // namespace moe
