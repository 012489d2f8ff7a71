// Whole-token decode of an L-layer MoE stack in ONE cooperative launch.
//
// The three per-layer launches of the decode path (route, gate/up, down)
// cost ~2.5 us each of launch overhead on this part, more than the 21 MB a
// layer reads takes to stream.  Here a persistent grid of one workgroup per
// CU walks all layers; the phases of a layer are chained by device-scope
// counters (release on arrival, acquire on wait) instead of kernel
// boundaries:
//
//   R_l : router (+ next-layer lookahead) rows, one row per workgroup;
//         waits for D_{l-1} (the layer input depends on the previous output)
//   -   : every workgroup waits for R_l, then ranks the logits itself
//         (redundantly, identically) -- no extra hop to publish the choice
//   U_l : gate/up + activation, 24 rows of one routed expert per workgroup;
//         the workgroup's down-projection codes for phase D are issued to
//         the memory system before this phase's math
//   D_l : waits for U_l; down + score-weighted combine over the k experts,
//         8 output rows per workgroup
//
// Counters are monotonic across launches: launch number `epoch` (1, 2, ...)
// waits for epoch * arrivals, so the workspace is zeroed once.  Every wait is
// bounded: past the spin limit it sets the device error word and proceeds
// (wrong results, never a hang).  The cooperative launch guarantees that all
// workgroups are resident, so every wait is satisfiable.
//
// Semantics per layer are those of route_kernel + ffn_decode (see their
// files): top_k_experts / top_k_route (engine_v3.py:467-473,
// engine_120b.py:65-70), top_k_indices (engine_v3.py:476-483), slot lookup
// (engine_v3.py:548-552), the expert block (engine_v3.py:588-600).
#include "launchers.h"

namespace moe {

constexpr uint32_t kSpinLimit = 1u << 20;

struct StackArgs {
  PoolArgs pa;
  const uint16_t *x;      // [L][D] bf16 layer inputs
  const uint16_t *W;      // [L][E][D] bf16 routers
  const uint16_t *bias;   // [L][E] bf16 or null
  const int32_t *table;   // [L][E] slot refs
  uint16_t *y;            // [L][D] bf16 layer outputs
  int32_t *ids;           // [L][K]
  float *scores;          // [L][K]
  int32_t *refs_out;      // [L][K]
  int32_t *pred;          // [L][KP]
  int32_t *miss;          // [L]
  float *logits;          // ws [2][E]
  float *h;               // ws [K][F] bf16-valued floats
  uint32_t *cnt;          // ws [L][3][kSub] counters, 128 B apart
  int L, E, kp, mode, renorm, act;
  float alpha, limit;
  uint32_t epoch;
  uint64_t *trace;        // optional [kTraceWGs][L][kTracePoints] wall clock
};

// Phase trace: wall-clock stamps of thread 0 of the first kTraceWGs
// workgroups at each phase boundary of each layer.
constexpr int kTraceWGs = 8;
constexpr int kTracePoints = 12;
enum { TR_START, TR_R_WAITED, TR_R_ARRIVED, TR_SELECTED, TR_U_ARRIVED,
       TR_D_WAITED, TR_D_ARRIVED, TR_R_ALL, TR_LOGITS, TR_SOFTMAX, TR_TOPK };

__device__ __forceinline__ void trace_mark(const StackArgs &a, int l, int point) {
  if (a.trace && blockIdx.x < kTraceWGs && threadIdx.x == 0)
    a.trace[((size_t)blockIdx.x * a.L + l) * kTracePoints + point] = wall_clock64();
}
// Stamp once `dep` has been computed (keeps the clock read after its inputs).
__device__ __forceinline__ void trace_mark_after(const StackArgs &a, int l, int point,
                                                 float dep) {
  if (a.trace && blockIdx.x < kTraceWGs && threadIdx.x == 0) {
    __builtin_amdgcn_s_waitcnt(0);
    uint64_t t = wall_clock64();
    if (dep == 1.2345e-37f) t = 0;   // data dependence only
    a.trace[((size_t)blockIdx.x * a.L + l) * kTracePoints + point] = t;
  }
}

// A phase counter is kSub sub-counters on separate 128-byte lines (arrivals
// spread by workgroup id), so 256 arrivals do not queue on one address.
constexpr int kSub = 8;
constexpr int kCounterWords = kSub * 32;

// Counters of one layer: router rows, lookahead rows, the layer output, and
// one per routed expert for its activations h.
enum { CNT_R = 0, CNT_RL = 1, CNT_D = 2, CNT_U0 = 3 };
constexpr int kCountersPerLayer = CNT_U0 + 8;

__device__ __forceinline__ uint32_t *counter(const StackArgs &a, int l, int which) {
  return a.cnt + ((size_t)l * kCountersPerLayer + which) * kCounterWords;
}

// 16 bytes at device scope (4 x sc1 dword loads issued back to back).
__device__ __forceinline__ uint4 ld_dev16(const float *p) {
  uint4 r;
  r.x = __hip_atomic_load(reinterpret_cast<const uint32_t *>(p) + 0, __ATOMIC_RELAXED,
                          __HIP_MEMORY_SCOPE_AGENT);
  r.y = __hip_atomic_load(reinterpret_cast<const uint32_t *>(p) + 1, __ATOMIC_RELAXED,
                          __HIP_MEMORY_SCOPE_AGENT);
  r.z = __hip_atomic_load(reinterpret_cast<const uint32_t *>(p) + 2, __ATOMIC_RELAXED,
                          __HIP_MEMORY_SCOPE_AGENT);
  r.w = __hip_atomic_load(reinterpret_cast<const uint32_t *>(p) + 3, __ATOMIC_RELAXED,
                          __HIP_MEMORY_SCOPE_AGENT);
  return r;
}

// Data crossing workgroups (logits, h) moves through device-scope accesses
// (sc1: coherent across the XCDs without an L2 writeback or invalidate).
__device__ __forceinline__ void st_dev(float *p, float v) {
  __hip_atomic_store(p, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ float ld_dev(const float *p) {
  return __hip_atomic_load(p, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

// All threads of the workgroup: wait until the counter's sum >= target.
// Wave 0 polls the sub-counters (device scope); the barrier then releases
// the workgroup, whose later device-scope loads observe every store that was
// complete before the arrivals counted.  Bounded: past the spin limit, or as
// soon as any workgroup has flagged an error, it gives up (wrong results,
// never a hang).
// One whole wave: poll until the counter's sum >= target (no barrier).
__device__ __forceinline__ void wave_wait(const uint32_t *c, uint32_t target) {
  const int lane = threadIdx.x & 63;
  uint32_t spins = 0;
  while (true) {
    int v = (lane < kSub) ? (int)__hip_atomic_load(c + lane * 32, __ATOMIC_RELAXED,
                                                    __HIP_MEMORY_SCOPE_AGENT)
                          : 0;
    v += dpp_i<kDppQuadXor1>(v);
    v += dpp_i<kDppQuadXor2>(v);
    v += dpp_i<kDppHalfMirror>(v);
    const uint32_t sum = (uint32_t)__builtin_amdgcn_readfirstlane(v);
    if (sum >= target) break;
    __builtin_amdgcn_s_sleep(1);
    if (++spins > kSpinLimit ||
        __hip_atomic_load(&g_device_error, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT)) {
      if (lane == 0) flag_error();
      break;
    }
  }
}

__device__ __forceinline__ void wg_wait(const uint32_t *c, uint32_t target) {
  if (threadIdx.x < 64) wave_wait(c, target);
  __syncthreads();
}

// All threads of the workgroup, after their global stores: one arrival.
// Every thread waits for its own stores to complete before the barrier, so
// the relaxed increment is ordered after all of them.
__device__ __forceinline__ void wg_arrive(uint32_t *c) {
  __builtin_amdgcn_s_waitcnt(0);
  __syncthreads();
  if (threadIdx.x == 0)
    __hip_atomic_fetch_add(c + (blockIdx.x % kSub) * 32, 1u, __ATOMIC_RELAXED,
                           __HIP_MEMORY_SCOPE_AGENT);
}

template <int D, int F, int K, bool PBIAS>
struct StackCfg {
  static constexpr int NT = 512;                 // 8 waves
  // gate/up: SG 16 lanes per row, 4 rows per wave step, 6 waves -> 24 rows
  static constexpr int U = D / 32, NG = D / 64;
  static constexpr int SGU = 16, CPLU = U / SGU, RPSU = 64 / SGU, WAVES_U = 6;
  static constexpr int ROWS_U = WAVES_U * RPSU;
  static constexpr int ITEMS_U = K * (F / ROWS_U);
  static constexpr int SB_U4 = ROWS_U * NG * 2 / 16;
  // down: SG 8 lanes per row, 8 rows per wave, one wave per expert
  static constexpr int UF = F / 32, NGF = F / 64;
  static constexpr int SGD = 8, CPLD = (UF + SGD - 1) / SGD, RPSD = 64 / SGD;
  static constexpr int ROWS_D = RPSD;
  static constexpr int ITEMS_D = D / ROWS_D;
  static constexpr int SBD_U4 = ROWS_D * NGF * 2 / 16;
  static constexpr int NP = PBIAS ? 4 : 3;
  static_assert(U % SGU == 0, "gate/up rows split evenly over lanes");
  static_assert(F % ROWS_U == 0 && D % ROWS_D == 0, "row blocks");
  static_assert(K <= 8, "one wave per expert in the down phase");
  static_assert((ROWS_U * NG * 2) % 16 == 0 && (ROWS_D * NGF * 2) % 16 == 0, "scale blocks");
};

template <int D, int F, int K, bool PBIAS>
__global__ __launch_bounds__(512) void stack_decode_kernel(StackArgs a) {
  using C = StackCfg<D, F, K, PBIAS>;
  constexpr int NT = C::NT, U = C::U, NG = C::NG, SGU = C::SGU, CPLU = C::CPLU;
  constexpr int RPSU = C::RPSU, ROWS_U = C::ROWS_U, SB_U4 = C::SB_U4;
  constexpr int UF = C::UF, NGF = C::NGF, SGD = C::SGD, CPLD = C::CPLD;
  constexpr int RPSD = C::RPSD, ROWS_D = C::ROWS_D, SBD_U4 = C::SBD_U4, NP = C::NP;
  constexpr int XU4 = D / 8, HU4 = F / 8;
  constexpr int RIT = (XU4 + 63) / 64;       // router-row pieces per lane

  __shared__ uint4 act_l[4 * U];
  __shared__ float asum_l[U];
  __shared__ uint4 sbu_l[4][SB_U4];
  __shared__ uint4 hact_l[K][4 * UF];
  __shared__ float hsum_l[K][UF];
  __shared__ uint4 sbd_l[K][2 * SBD_U4];
  __shared__ float red_l[K][ROWS_D];
  __shared__ int sel_id[K];
  __shared__ float sel_sc[K];
  __shared__ int32_t sel_ref[K];

  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int wg = blockIdx.x;
  const uint32_t ep = a.epoch;

  for (int l = 0; l < a.L; ++l) {
    const bool has_next = l + 1 < a.L;
    const int nrows = a.E * (has_next ? 2 : 1);
    trace_mark(a, l, TR_START);
    // ------------------------------------------------------------ R_l ----
    if (wg < nrows) {
      const bool nxt = wg >= a.E;
      const int e = nxt ? wg - a.E : wg;
      const int lw = nxt ? l + 1 : l;
      // one wave per row, the lane partition and summation order of
      // route_kernel, so both paths produce bit-identical logits
      const uint4 *w4 = reinterpret_cast<const uint4 *>(a.W + ((size_t)lw * a.E + e) * D);
      uint4 wr[RIT];
      if (wave == 0) {
#pragma unroll
        for (int it = 0; it < RIT; ++it) {
          const int i = lane + it * 64;
          wr[it] = (i < XU4) ? load_stream16(w4 + i) : make_uint4(0, 0, 0, 0);
        }
      }
      if (l > 0) wg_wait(counter(a, l - 1, CNT_D), ep * C::ITEMS_D);
      trace_mark(a, l, TR_R_WAITED);
      if (wave == 0) {
        const uint4 *x4 = reinterpret_cast<const uint4 *>(a.x + (size_t)l * D);
        uint4 v[RIT];
#pragma unroll
        for (int it = 0; it < RIT; ++it) {
          const int i = lane + it * 64;
          v[it] = (i < XU4) ? x4[i] : make_uint4(0, 0, 0, 0);
        }
        float acc = 0.f;
#pragma unroll
        for (int it = 0; it < RIT; ++it) {
          acc = dot2_bf16(wr[it].x, v[it].x, acc);
          acc = dot2_bf16(wr[it].y, v[it].y, acc);
          acc = dot2_bf16(wr[it].z, v[it].z, acc);
          acc = dot2_bf16(wr[it].w, v[it].w, acc);
        }
        acc = group_sum<64>(acc);
        if (lane == 0) st_dev(a.logits + (nxt ? a.E : 0) + e, acc);
      }
      wg_arrive(counter(a, l, nxt ? CNT_RL : CNT_R));
      trace_mark(a, l, TR_R_ARRIVED);
    }
    // ------------------------------------------------------ selection ----
    // every workgroup needs this layer's router rows; only workgroup 0 waits
    // for the lookahead rows (it publishes the predicted ids)
    if (wave == 0 || (wave == 1 && has_next && wg == 0)) {
      const bool la = wave == 1;
      wave_wait(counter(a, l, la ? CNT_RL : CNT_R), ep * a.E);
      if (!la) trace_mark(a, l, TR_R_ALL);
      const int e0 = lane, e1 = lane + 64;
      const float *lg = a.logits + (la ? a.E : 0);
      const uint16_t *bias = a.bias ? a.bias + (size_t)(la ? l + 1 : l) * a.E : nullptr;
      float z0 = -INFINITY, z1 = -INFINITY;
      if (e0 < a.E) z0 = round_bf16(ld_dev(lg + e0) + (bias ? bf16_to_f32(bias[e0]) : 0.f));
      if (e1 < a.E) z1 = round_bf16(ld_dev(lg + e1) + (bias ? bf16_to_f32(bias[e1]) : 0.f));
      if (!la) trace_mark_after(a, l, TR_LOGITS, z0 + z1);
      float v0 = z0, v1 = z1;
      if (!la && a.mode == MOE_ROUTE_SOFTMAX_TOPK) {
        const float m = wave_max(fmaxf(z0, z1));
        const float x0 = (e0 < a.E) ? expf(z0 - m) : 0.f;
        const float x1 = (e1 < a.E) ? expf(z1 - m) : 0.f;
        const float s = group_sum<64>(x0 + x1);
        v0 = round_bf16(x0 / s);
        v1 = round_bf16(x1 / s);
      }
      if (!la) trace_mark_after(a, l, TR_SOFTMAX, v0 + v1);
      const int kk = la ? a.kp : K;
      bool s0, s1;
      int r0, r1;
      select_topk(e0 < a.E ? order_key(v0) : -1, e1 < a.E ? order_key(v1) : -1, kk, lane,
                  s0, s1, r0, r1);
      if (!la) trace_mark_after(a, l, TR_TOPK, (float)(r0 + r1));
      if (la) {
        if (s0) a.pred[(size_t)l * a.kp + r0] = e0;
        if (s1) a.pred[(size_t)l * a.kp + r1] = e1;
      } else {
        float sc0 = v0, sc1 = v1;
        if (a.mode == MOE_ROUTE_SOFTMAX_TOPK) {
          if (a.renorm) {
            const float tot = round_bf16(group_sum<64>((s0 ? v0 : 0.f) + (s1 ? v1 : 0.f)));
            sc0 = round_bf16(v0 / tot);
            sc1 = round_bf16(v1 / tot);
          }
        } else {
          const float m = wave_max(fmaxf(s0 ? z0 : -INFINITY, s1 ? z1 : -INFINITY));
          const float x0 = s0 ? expf(z0 - m) : 0.f;
          const float x1 = s1 ? expf(z1 - m) : 0.f;
          const float s = group_sum<64>(x0 + x1);
          sc0 = round_bf16(x0 / s);
          sc1 = round_bf16(x1 / s);
        }
        const int32_t *tab = a.table + (size_t)l * a.E;
        if (s0) {
          sel_id[r0] = e0;
          sel_sc[r0] = sc0;
          sel_ref[r0] = tab[e0];
        }
        if (s1) {
          sel_id[r1] = e1;
          sel_sc[r1] = sc1;
          sel_ref[r1] = tab[e1];
        }
      }
    }
    __syncthreads();
    if (wg == 0 && tid < K) {
      a.ids[(size_t)l * K + tid] = sel_id[tid];
      a.scores[(size_t)l * K + tid] = sel_sc[tid];
      a.refs_out[(size_t)l * K + tid] = sel_ref[tid];
      if (sel_ref[tid] < 0) atomicAdd(a.miss + l, 1);
    }

    trace_mark(a, l, TR_SELECTED);

    // ------------------------------------------------------------ U_l ----
    if (wg < C::ITEMS_U) {
      const int pj = wg / (F / ROWS_U), rb = wg % (F / ROWS_U);
      const int32_t ref = sel_ref[pj];
      const int row0 = rb * ROWS_U;
      const char *gw = resolve(a.pa, comp_index(PROJ_GATE, PART_W, NP), ref);
      const char *uw = resolve(a.pa, comp_index(PROJ_UP, PART_W, NP), ref);
      const bool ok = gw != nullptr;
      const bool uwave = wave < C::WAVES_U;
      const int uj = lane % SGU, usub = lane / SGU;
      // small loads first: x pieces and the block's scales/biases
      constexpr int XIT = (XU4 + NT - 1) / NT, SIT = (4 * SB_U4 + NT - 1) / NT;
      uint4 xr[XIT], sr[SIT];
      const uint4 *x4 = reinterpret_cast<const uint4 *>(a.x + (size_t)l * D);
#pragma unroll
      for (int it = 0; it < XIT; ++it) {
        const int i = it * NT + tid;
        xr[it] = (i < XU4) ? x4[i] : make_uint4(0, 0, 0, 0);
      }
      if (ok) {
#pragma unroll
        for (int it = 0; it < SIT; ++it) {
          const int i = it * NT + tid;
          const int p = i / SB_U4, o = i % SB_U4;
          const int part = (p & 1) ? PART_B : PART_S, proj = (p >> 1) ? PROJ_UP : PROJ_GATE;
          const char *sp = resolve(a.pa, comp_index(proj, part, NP), ref);
          sr[it] = (i < 4 * SB_U4)
                       ? reinterpret_cast<const uint4 *>(sp + (int64_t)row0 * NG * 2)[o]
                       : make_uint4(0, 0, 0, 0);
        }
      }
      uint4 cg[CPLU], cu[CPLU];
      const int urow = row0 + wave * RPSU + usub;
      if (ok && uwave) {
        const uint4 *g4 = reinterpret_cast<const uint4 *>(gw + (int64_t)urow * (D / 2));
        const uint4 *u4 = reinterpret_cast<const uint4 *>(uw + (int64_t)urow * (D / 2));
#pragma unroll
        for (int i = 0; i < CPLU; ++i) {
          cg[i] = load_stream16(g4 + i * SGU + uj);
          cu[i] = load_stream16(u4 + i * SGU + uj);
        }
      }
      if (ok) {
#pragma unroll
        for (int it = 0; it < SIT; ++it) {
          const int i = it * NT + tid;
          if (i < 4 * SB_U4) (&sbu_l[0][0])[i] = sr[it];
        }
      }
#pragma unroll
      for (int it = 0; it < XIT; ++it) {
        const int i = it * NT + tid;
        float s = 0.f;
        if (i < XU4) s = stage_piece<U>(act_l, i, xr[it]);
        s += dpp_f<kDppQuadXor1>(s);
        s += dpp_f<kDppQuadXor2>(s);
        if (i < XU4 && (i & 3) == 0) asum_l[i >> 2] = s;
      }
      __syncthreads();
      if (uwave) {
        float pg = 0.f, pu = 0.f;
        if (ok) {
          const uint16_t *sbh = reinterpret_cast<const uint16_t *>(&sbu_l[0][0]);
          constexpr int SBN = SB_U4 * 8;
          const int rl = wave * RPSU + usub;
#pragma unroll
          for (int i = 0; i < CPLU; ++i) {
            const int c = i * SGU + uj;
            const int g = rl * NG + (c >> 1);
            const float Sg = bf16_to_f32(sbh[g]), Bg = bf16_to_f32(sbh[SBN + g]);
            const float Su = bf16_to_f32(sbh[2 * SBN + g]), Bu = bf16_to_f32(sbh[3 * SBN + g]);
            const float xs = asum_l[c];
            pg += Sg * chunk_dot_lds<U>(cg[i], act_l, c) + (Bg - 128.f * Sg) * xs;
            pu += Su * chunk_dot_lds<U>(cu[i], act_l, c) + (Bu - 128.f * Su) * xs;
          }
        }
        pg = group_sum<SGU>(pg);
        pu = group_sum<SGU>(pu);
        if (uj == 0) {
          float hv = 0.f;
          if (ok) {
            if (PBIAS) {
              pg += bf16_to_f32(reinterpret_cast<const uint16_t *>(
                  resolve(a.pa, comp_index(PROJ_GATE, PART_BIAS, NP), ref))[urow]);
              pu += bf16_to_f32(reinterpret_cast<const uint16_t *>(
                  resolve(a.pa, comp_index(PROJ_UP, PART_BIAS, NP), ref))[urow]);
            }
            hv = apply_act(a.act, pg, pu, a.alpha, a.limit);
          } else if (lane == 0) {
            flag_error();
          }
          st_dev(a.h + (size_t)pj * F + urow, round_bf16(hv));   // h is bf16-valued
        }
      }
      wg_arrive(counter(a, l, CNT_U0 + pj));
      trace_mark(a, l, TR_U_ARRIVED);
    }

    // ------------------------------------------- D_l codes (prefetch) ----
    // this workgroup's down item: output rows wg*8 .. +8, wave = expert;
    // issued after the gate/up arrival (which waits for all of its own
    // memory operations) and before the wait for the activations
    const bool has_d = wg < C::ITEMS_D && wave < K;
    const int32_t dref = has_d ? sel_ref[wave] : 0;
    const char *dw = has_d ? resolve(a.pa, comp_index(PROJ_DOWN, PART_W, NP), dref) : nullptr;
    const int drow0 = wg * ROWS_D;
    const int dj = lane % SGD, dsub = lane / SGD;
    uint4 cd[CPLD];
    uint4 sdr[(2 * SBD_U4 + 63) / 64];
    if (dw != nullptr) {
#pragma unroll
      for (int it = 0; it < (2 * SBD_U4 + 63) / 64; ++it) {
        const int i = it * 64 + lane;
        const int p = i / SBD_U4, o = i % SBD_U4;
        const char *sp = resolve(a.pa, comp_index(PROJ_DOWN, p ? PART_B : PART_S, NP), dref);
        sdr[it] = (i < 2 * SBD_U4)
                      ? reinterpret_cast<const uint4 *>(sp + (int64_t)drow0 * NGF * 2)[o]
                      : make_uint4(0, 0, 0, 0);
      }
      const uint4 *d4 = reinterpret_cast<const uint4 *>(dw + (int64_t)(drow0 + dsub) * (F / 2));
#pragma unroll
      for (int i = 0; i < CPLD; ++i) {
        const int c = i * SGD + dj;
        cd[i] = (CPLD * SGD == UF || c < UF) ? load_stream16(d4 + c) : make_uint4(0, 0, 0, 0);
      }
    }

    // ------------------------------------------------------------ D_l ----
    if (wg < C::ITEMS_D) {
      if (wave < K) {
        // this wave's expert: its activations are complete when the expert's
        // gate/up workgroups have all arrived
        wave_wait(counter(a, l, CNT_U0 + wave), ep * (F / ROWS_U));
        if (wave == 0) trace_mark(a, l, TR_D_WAITED);
        uint4 *hact = hact_l[wave];
        float *hsum = hsum_l[wave];
        if (dw != nullptr) {
          uint4 *sbd = sbd_l[wave];
#pragma unroll
          for (int it = 0; it < (2 * SBD_U4 + 63) / 64; ++it) {
            const int i = it * 64 + lane;
            if (i < 2 * SBD_U4) sbd[i] = sdr[it];
          }
          const float *hrow = a.h + (size_t)wave * F;
#pragma unroll
          for (int it = 0; it < (HU4 + 63) / 64; ++it) {
            const int i = it * 64 + lane;
            float s = 0.f;
            if (i < HU4) {
              const uint4 lo = ld_dev16(hrow + 8 * i), hi = ld_dev16(hrow + 8 * i + 4);
              // bf16-valued floats: the high halves are the bf16 bit patterns
              const uint4 wds = make_uint4((lo.x >> 16) | (lo.y & 0xffff0000u),
                                           (lo.z >> 16) | (lo.w & 0xffff0000u),
                                           (hi.x >> 16) | (hi.y & 0xffff0000u),
                                           (hi.z >> 16) | (hi.w & 0xffff0000u));
              s = stage_piece<UF>(hact, i, wds);
            }
            s += dpp_f<kDppQuadXor1>(s);
            s += dpp_f<kDppQuadXor2>(s);
            if (i < HU4 && (i & 3) == 0) hsum[i >> 2] = s;
          }
        } else if (has_d && lane == 0) {
          flag_error();
        }
      }
      __syncthreads();
      if (wave < K) {
        float p = 0.f;
        if (dw != nullptr) {
          const uint16_t *sbh = reinterpret_cast<const uint16_t *>(sbd_l[wave]);
          constexpr int SBN = SBD_U4 * 8;
#pragma unroll
          for (int i = 0; i < CPLD; ++i) {
            const int c = i * SGD + dj;
            if (CPLD * SGD == UF || c < UF) {
              const int g = dsub * NGF + (c >> 1);
              const float Sd = bf16_to_f32(sbh[g]), Bd = bf16_to_f32(sbh[SBN + g]);
              p += Sd * chunk_dot_lds<UF>(cd[i], hact_l[wave], c) + (Bd - 128.f * Sd) * hsum_l[wave][c];
            }
          }
        }
        p = group_sum<SGD>(p);
        if (dj == 0) {
          if (PBIAS && dw != nullptr)
            p += bf16_to_f32(reinterpret_cast<const uint16_t *>(
                resolve(a.pa, comp_index(PROJ_DOWN, PART_BIAS, NP), dref))[drow0 + dsub]);
          red_l[wave][dsub] = (dw != nullptr) ? sel_sc[wave] * p : 0.f;
        }
      }
      __syncthreads();
      if (tid < ROWS_D) {
        float yv = 0.f;
        for (int w = 0; w < K; ++w) yv += red_l[w][tid];   // expert order
        a.y[(size_t)l * D + drow0 + tid] = (uint16_t)f32_to_bf16(yv);
      }
      wg_arrive(counter(a, l, CNT_D));
      trace_mark(a, l, TR_D_ARRIVED);
    }
  }
}

// ---------------------------------------------------------------------------
#define MOE_STACK_GEOM(D, F, K, PB)                                          \
  {D, F, K, PB,                                                              \
   (StackCfg<D, F, K, PB>::ITEMS_U > StackCfg<D, F, K, PB>::ITEMS_D          \
        ? StackCfg<D, F, K, PB>::ITEMS_U                                     \
        : StackCfg<D, F, K, PB>::ITEMS_D),                                   \
   reinterpret_cast<const void *>(&stack_decode_kernel<D, F, K, PB>)}

static const StackLaunch kStackTable[] = {
    MOE_STACK_GEOM(2048, 768, 8, false),   // Qwen3-30B-A3B: 256 workgroups
};

const StackLaunch *find_stack(int d_model, int d_ff, int k, int has_bias) {
  for (const auto &e : kStackTable)
    if (e.d_model == d_model && e.d_ff == d_ff && e.k == k && e.has_bias == (has_bias != 0))
      return &e;
  return nullptr;
}

hipError_t launch_stack(const StackLaunch *S, StackArgs &a, hipStream_t s) {
  void *args[] = {&a};
  return hipLaunchCooperativeKernel(S->func, dim3(S->nwg), dim3(512), args, 0, s);
}

}  // namespace moe
