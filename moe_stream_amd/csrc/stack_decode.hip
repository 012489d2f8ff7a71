// Whole-token decode of an L-layer MoE stack in ONE cooperative launch.
//
// The three per-layer launches of the decode path (route, gate/up, down)
// cost ~2.5 us each of launch overhead on this part, more than the 21 MB a
// layer reads takes to stream.  Here a persistent grid of one workgroup per
// CU walks all layers; the phases of a layer are chained by device-scope
// counters (a relaxed increment after the producer's stores completed;
// device-scope loads on the consumer side) instead of kernel boundaries.
//
// The lookahead router predicts layer l+1's experts during layer l
// (engine_v3.py:509-527).  Here that prediction stages the expert bytes:
// at the end of layer l every workgroup issues the register loads of the
// gate/up codes it will need in layer l+1 if the prediction is right, so
// the reads overlap the wait for the layer boundary; the down codes follow
// inside layer l+1, each wave's once its earlier work there is done (issued
// at layer l's end they would queue ahead of the boundary poll).  Per layer:
//
//   wait   : layer l-1 complete (its output is this layer's input)
//   split  : (expert position p = rank p of the prediction lives on XCD p:
//            the workgroups w with w % 8 == p) waves 0-5 gate/up + activation
//            for the PREDICTED expert at this workgroup's position (24 rows,
//            published XCD-locally), and waves 0-1 one 4-row task of
//            the two SPARE positions (lookahead ranks K, K+1; their bytes go
//            to LDS by direct-to-LDS loads while the predicted rows compute);
//            wave 6 one router row (+ the lookahead row), then the lookahead
//            ranking of layer l+1; wave 7 waits for all router rows and ranks
//            them (every workgroup redundantly, identically)
//   fix-up : routed experts that were not predicted get gate/up now
//   D      : the down rows (64 per workgroup, 8 per wave) of the routed
//            expert at the workgroup's position, its activations polled from
//            the XCD's L2; the score-weighted rows go out as that routing
//            rank's partial output, which the next layer combines in rank
//            order; then the gate/up staging loads of layer l+1
//
// Activations and the combine are indexed by routing rank, so results are
// bit-identical to route_kernel + ffn_decode whatever was predicted.
//
// Counters are monotonic across launches: launch number `epoch` (1, 2, ...)
// waits for epoch * arrivals, so the workspace is zeroed once; every counter
// receives its full count of arrivals in every layer, work or not.  Every
// wait is bounded: past the spin limit it sets the device error word and
// proceeds (wrong results, never a hang).  The cooperative launch guarantees
// that all workgroups are resident, so every wait is satisfiable.
//
// Semantics per layer are those of route_kernel + ffn_decode (see their
// files): top_k_experts / top_k_route (engine_v3.py:467-473,
// engine_120b.py:65-70), top_k_indices (engine_v3.py:476-483), slot lookup
// (engine_v3.py:548-552), the expert block (engine_v3.py:588-600).
#include <atomic>
#include <cstddef>

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
  char *ws;               // workspace (StackWs layout)
  int L, E, kp, mode, renorm, act;
  float alpha, limit;
  uint32_t epoch;
  uint64_t *trace;        // optional [kTraceWGs][L][kTracePoints] wall clock
};

// A field of the kernel's only argument (StackArgs, at offset 0 of the
// kernarg segment), read from the kernarg segment where it is used: the
// opaque offset keeps the compiler from loading it once and holding it in
// scalar registers for the whole kernel (this kernel runs at the scalar
// register limit, and a value held that way is spilled).  For fields the
// hot loops do not touch.
template <class T>
__device__ __forceinline__ T karg_load(size_t off) {
  typedef __attribute__((address_space(4))) const char kchar;
  typedef __attribute__((address_space(4))) const T kT;
  kchar *p = (kchar *)__builtin_amdgcn_kernarg_segment_ptr();
  asm volatile("" : "+s"(off));
  return *reinterpret_cast<kT *>(p + off);
}
#define KARG(field) karg_load<decltype(StackArgs::field)>(offsetof(StackArgs, field))

// Phase trace: wall-clock stamps of thread 0 of the first kTraceWGs
// workgroups at each phase boundary of each layer.
constexpr int kTraceWGs = 256;
constexpr int kTracePoints = 15;
enum { TR_START, TR_R_WAITED, TR_R_ARRIVED, TR_SELECTED, TR_U_ARRIVED,
       TR_D_WAITED, TR_D_ARRIVED, TR_R_ALL, TR_LOGITS, TR_SOFTMAX, TR_TOPK, TR_FIXED,
       TR_LOOKED, TR_SPARE1, TR_UROWS2 };

// Called by one wave at a time; its lane 0 stamps.
__device__ __forceinline__ void trace_mark(const StackArgs &a, int l, int point) {
  uint64_t *tr = KARG(trace);
  if (tr && blockIdx.x < kTraceWGs && (threadIdx.x & 63) == 0)
    tr[((size_t)blockIdx.x * a.L + l) * kTracePoints + point] = wall_clock64();
}
// Stamp once `dep` has been computed (keeps the clock read after its inputs).
__device__ __forceinline__ void trace_mark_after(const StackArgs &a, int l, int point,
                                                 float dep) {
  uint64_t *tr = KARG(trace);
  if (tr && blockIdx.x < kTraceWGs && (threadIdx.x & 63) == 0) {
    __builtin_amdgcn_s_waitcnt(0);
    uint64_t t = wall_clock64();
    if (dep == 1.2345e-37f) t = 0;   // data dependence only
    tr[((size_t)blockIdx.x * a.L + l) * kTracePoints + point] = t;
  }
}

// A phase counter is kSub sub-counters on separate 128-byte lines (arrivals
// spread by workgroup id), so 256 arrivals do not queue on one address.
constexpr int kSub = 8;
constexpr int kCounterWords = kSub * 32;

// Predicted experts beyond the K staged ones whose gate/up the workgroups
// compute speculatively from the pool each layer (lookahead ranks K ..
// K + kSpare - 1): a routed expert among them needs no fix-up pass.
constexpr int kSpare = 2;

// Widest layer output the per-rank partial outputs of the workspace hold.
constexpr int kStackMaxD = 2880;

// Workgroup w runs on XCD w % kXcds (the dispatcher deals workgroups to the
// XCDs round robin), so the workgroups with one value of w % kXcds share
// an L2: a plain store there is seen by an agent-scope load from any of
// them, without the round trip through the device-coherent path.
constexpr int kXcds = 8;

// Counters of one layer: the layer output (the layer boundary).  Router
// logits and expert activations carry their own flags instead.
enum { CNT_D = 0 };
constexpr int kCountersPerLayer = 1;
static_assert(kStackCounterBytesPerLayer == (size_t)kCountersPerLayer * kCounterWords * 4,
              "host-side workspace size");

// The flag a data entry exchanged between workgroups carries (router logits,
// expert activations): unique per (token, layer), so an entry left by an
// earlier token or layer never passes for a current one.
__device__ __forceinline__ uint32_t layer_flag(const StackArgs &a, int l) {
  return a.epoch * (uint32_t)a.L + (uint32_t)l;
}

// Router logits cross workgroups as flagged 8-byte entries, the fp32 logit in
// the low word and the layer flag in the high word: one device-scope store
// publishes a logit, and readers poll the entries themselves (no counter to
// arrive on, no load after the wait).
__device__ __forceinline__ void put_logit(uint64_t *slot, float v, uint32_t fl) {
  __hip_atomic_store(slot, (uint64_t)__float_as_uint(v) | ((uint64_t)fl << 32),
                     __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

// The workspace: one base address, the parts at offsets fixed by the
// geometry (the counters, whose size depends on the layer count, last).
//   abort word (256 B) | router + lookahead logits [2][kRouteMaxE], flagged
//   8-byte entries | activations of the predicted and spare experts
//   [K + kSpare][F/2] and of the fix-up slots [K][F/2] (2 bf16 + layer flag
//   per 8 bytes) | score-weighted down outputs per routing rank, 8 bytes
//   per entry (fp32, or fp32 + layer flag) [2 (layer parity)][K][kStackMaxD]
//   | counters [L][kSub], 128 B apart
template <int F, int K>
struct StackWs {
  static constexpr size_t al(size_t v) { return (v + 255) & ~(size_t)255; }
  static constexpr size_t kAbort = 0;
  static constexpr size_t kLgt = 256;
  static constexpr size_t kHpred = kLgt + al((size_t)2 * kRouteMaxE * 8);
  static constexpr size_t kHfix = kHpred + al((size_t)(K + kSpare) * (F / 2) * 8);
  static constexpr size_t kPart = kHfix + al((size_t)K * (F / 2) * 8);
  static constexpr size_t kCnt = kPart + al((size_t)2 * K * kStackMaxD * 8);
  static constexpr size_t bytes(int L) {
    return kCnt + (size_t)L * kCountersPerLayer * kCounterWords * 4;
  }
};

template <class W>
__device__ __forceinline__ uint32_t *counter(const StackArgs &a, int l, int which) {
  return reinterpret_cast<uint32_t *>(a.ws + W::kCnt) +
         ((size_t)l * kCountersPerLayer + which) * kCounterWords;
}

// The launch's abort word (in the workspace): the epoch of the launch in
// which some wait gave up.  A wait that keeps missing loads it every 64th
// poll (a normal wait ends long before, so it costs the fast path nothing),
// so once one wait has timed out the others stop soon instead of each
// running to the spin limit.  A value left by an earlier launch never equals
// the current epoch, so it cannot cut a new launch short.
struct Abort {
  uint32_t *word;
  uint32_t ep;
  // One whole wave, after its `spins`-th missed poll: true when it must stop
  // waiting (this launch gave up, or this wait ran past the spin limit).
  __device__ __forceinline__ bool gave_up(uint32_t spins) const {
    if ((spins & 63) == 0) {
      const uint32_t w = __hip_atomic_load(word, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
      if (__builtin_amdgcn_readfirstlane(w) == ep) return true;
    }
    if (spins > kSpinLimit) {
      if ((threadIdx.x & 63) == 0) {
        __hip_atomic_store(word, ep, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        flag_timeout();
      }
      return true;
    }
    return false;
  }
};

// One whole wave: poll until the counter's sum >= target (no barrier).
// Bounded: past the spin limit, or as soon as any workgroup has flagged an
// error, it gives up (wrong results, never a hang).  `lane`: the caller's
// lane index (a kernel may pass one it keeps from being hoisted).
__device__ __forceinline__ void wave_wait(const uint32_t *c, uint32_t target, const Abort &ab,
                                          int lane) {
  uint32_t spins = 0;
  while (true) {
    int v = (lane < kSub) ? (int)__hip_atomic_load(c + lane * 32, __ATOMIC_RELAXED,
                                                    __HIP_MEMORY_SCOPE_AGENT)
                          : 0;
    v += dpp_i<kDppQuadXor1>(v);
    v += dpp_i<kDppQuadXor2>(v);
    v += dpp_i<kDppHalfMirror>(v);
    const uint32_t sum = (uint32_t)__builtin_amdgcn_readfirstlane(v);
    // counters are monotonic modulo 2^32: compare the distance, not the values
    if ((int32_t)(sum - target) >= 0) break;
    if (ab.gave_up(++spins)) break;
    __builtin_amdgcn_s_sleep(1);
  }
}
__device__ __forceinline__ void wave_wait(const uint32_t *c, uint32_t target, const Abort &ab) {
  wave_wait(c, target, ab, threadIdx.x & 63);
}

// One whole wave: the logits of entries lane and lane + 64 of `slots` (n
// entries, n <= 128), polled until every present entry carries `fl`.
// Bounded like wave_wait.
__device__ __forceinline__ void get_logits(const uint64_t *slots, int n, uint32_t fl,
                                           const Abort &ab, float &z0, float &z1, int lane) {
  const int e0 = lane, e1 = lane + 64;
  const uint64_t *p0 = slots + min(e0, n - 1), *p1 = slots + min(e1, n - 1);
  uint32_t spins = 0;
  while (true) {
    const uint64_t v0 = __hip_atomic_load(p0, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    const uint64_t v1 = __hip_atomic_load(p1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    const bool ok = (e0 >= n || (uint32_t)(v0 >> 32) == fl) && (e1 >= n || (uint32_t)(v1 >> 32) == fl);
    z0 = __uint_as_float((uint32_t)v0);
    z1 = __uint_as_float((uint32_t)v1);
    if (__ballot(!ok) == 0) break;
    if (ab.gave_up(++spins)) break;
    __builtin_amdgcn_s_sleep(1);
  }
}
__device__ __forceinline__ void get_logits(const uint64_t *slots, int n, uint32_t fl,
                                           const Abort &ab, float &z0, float &z1) {
  get_logits(slots, n, fl, ab, z0, z1, threadIdx.x & 63);
}

// A workgroup barrier that orders LDS only: each wave's LDS operations
// complete, then the hardware barrier.  Unlike __syncthreads it does not
// wait for the wave's global loads and stores (its release fence makes the
// compiler wait for all of them: a device-scope store's acknowledgement
// takes ~0.5 us); for phases whose global data is exchanged only through
// flagged entries and counters.
__device__ __forceinline__ void lds_barrier() {
  __atomic_signal_fence(__ATOMIC_SEQ_CST);
  __builtin_amdgcn_s_waitcnt(0xc07f);   // lgkmcnt(0); vmcnt and expcnt not waited for
  __builtin_amdgcn_s_barrier();
  __atomic_signal_fence(__ATOMIC_SEQ_CST);
}

// All threads of the workgroup: wait until the counter's sum >= target.
// Wave `poll_wave` polls the sub-counters (device scope); the barrier then
// releases the workgroup, whose later device-scope loads observe every store
// that was complete before the arrivals counted.
__device__ __forceinline__ void wg_wait(const uint32_t *c, uint32_t target, int poll_wave,
                                        const Abort &ab) {
  if ((threadIdx.x >> 6) == poll_wave) wave_wait(c, target, ab);
  __syncthreads();
}

// One whole wave, after its own global stores: one arrival (phases in which
// only this wave stores).
__device__ __forceinline__ void wave_arrive(uint32_t *c) {
  __builtin_amdgcn_s_waitcnt(0);
  if ((threadIdx.x & 63) == 0)
    __hip_atomic_fetch_add(c + (blockIdx.x % kSub) * 32, 1u, __ATOMIC_RELAXED,
                           __HIP_MEMORY_SCOPE_AGENT);
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

template <int D, int F, int K, bool PBIAS, int ACT, int MODE, int RENORM>
struct StackCfg {
  static constexpr int D_ = D, F_ = F, K_ = K, ACT_ = ACT, MODE_ = MODE, RENORM_ = RENORM;
  static constexpr bool PBIAS_ = PBIAS;
  using Layout = PackedLayout<D, F, PBIAS>;   // the pool layout the kernel requires
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
  static constexpr int SIT = (4 * SB_U4 + NT - 1) / NT;   // gate/up scale pieces per thread
  static constexpr int SDIT = (2 * SBD_U4 + 63) / 64;     // down scale pieces per lane
  static_assert(U % SGU == 0, "gate/up rows split evenly over lanes");
  static_assert(F % ROWS_U == 0 && D % ROWS_D == 0, "row blocks");
  static_assert(K <= 8, "one wave per expert in the down phase");
  static_assert((ROWS_U * NG * 2) % 16 == 0 && (ROWS_D * NGF * 2) % 16 == 0, "scale blocks");
};

// The gated activation of the kernel's instantiation; the clamped form's
// alpha and limit come from the kernarg segment where they are used.
template <class C>
__device__ __forceinline__ float stack_act(float g, float u) {
  if (C::ACT_ == MOE_ACT_SWIGLU) return apply_act(MOE_ACT_SWIGLU, g, u, 0.f, 0.f);
  return apply_act(MOE_ACT_SWIGLU_CLAMP, g, u, KARG(alpha), KARG(limit));
}

// One whole wave, one row per 16 lanes (the row's activation in `hb` on
// each of its lanes): the 4 rows' bf16 activations as two flagged 8-byte
// entries (2 bf16 + layer flag) at hf[0], hf[1].
__device__ __forceinline__ void put_acts(uint64_t *hf, uint32_t hb, uint32_t fl) {
  const uint32_t h0 = __builtin_amdgcn_readlane(hb, 0), h1 = __builtin_amdgcn_readlane(hb, 16);
  const uint32_t h2 = __builtin_amdgcn_readlane(hb, 32), h3 = __builtin_amdgcn_readlane(hb, 48);
  if ((threadIdx.x & 63) == 0) {
    const uint64_t f = (uint64_t)fl << 32;
    __hip_atomic_store(hf, (uint64_t)(h0 | (h1 << 16)) | f, __ATOMIC_RELAXED,
                       __HIP_MEMORY_SCOPE_AGENT);
    __hip_atomic_store(hf + 1, (uint64_t)(h2 | (h3 << 16)) | f, __ATOMIC_RELAXED,
                       __HIP_MEMORY_SCOPE_AGENT);
  }
}

// put_acts for readers on this workgroup's XCD only: plain 8-byte stores,
// which stay in the XCD's L2 (agent-scope loads on the same XCD see them;
// workgroups on other XCDs must not read these entries).
__device__ __forceinline__ void put_acts_xcd(uint64_t *hf, uint32_t hb, uint32_t fl) {
  const uint32_t h0 = __builtin_amdgcn_readlane(hb, 0), h1 = __builtin_amdgcn_readlane(hb, 16);
  const uint32_t h2 = __builtin_amdgcn_readlane(hb, 32), h3 = __builtin_amdgcn_readlane(hb, 48);
  if ((threadIdx.x & 63) == 0) {
    const uint64_t f = (uint64_t)fl << 32;
    __hip_atomic_store(hf, (uint64_t)(h0 | (h1 << 16)) | f, __ATOMIC_RELAXED,
                       __HIP_MEMORY_SCOPE_WORKGROUP);
    __hip_atomic_store(hf + 1, (uint64_t)(h2 | (h3 << 16)) | f, __ATOMIC_RELAXED,
                       __HIP_MEMORY_SCOPE_WORKGROUP);
  }
}

// Gate/up rows of one expert for this workgroup's 24-row block, waves
// 0..WAVES_U-1: codes in cg/cu, scales staged in sbu_l, x staged in act_l
// and asum_l.  Returns the bf16 activation of this lane's row (its wave's
// RPSU = 4 rows go out with put_acts at hf + (row0 + wave * RPSU) / 2); an
// out-of-range ref flags an error and yields zeros.
template <class C>
__device__ __forceinline__ uint32_t u_rows(const StackArgs &a, int32_t ref, int row0,
                                           const uint4 (&cg)[C::CPLU],
                                           const uint4 (&cu)[C::CPLU], const uint4 *act_l,
                                           const float *asum_l,
                                           const uint4 (*sbu_l)[C::SB_U4]) {
  constexpr int U = C::U, NG = C::NG, SGU = C::SGU, CPLU = C::CPLU, RPSU = C::RPSU;
  constexpr int SB_U4 = C::SB_U4, NP = C::NP;
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int uj = lane % SGU, usub = lane / SGU;
  const bool ok = resolve_packed<typename C::Layout>(a.pa, comp_index(PROJ_GATE, PART_W, NP), ref) != nullptr;
  const int urow = row0 + wave * RPSU + usub;
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
  // every lane of a 16-lane row group holds that row's sums
  uint32_t hb = 0;
  if (ok) {
    if (C::PBIAS_) {
      pg += bf16_to_f32(reinterpret_cast<const uint16_t *>(
          resolve_packed<typename C::Layout>(a.pa, comp_index(PROJ_GATE, PART_BIAS, NP), ref))[urow]);
      pu += bf16_to_f32(reinterpret_cast<const uint16_t *>(
          resolve_packed<typename C::Layout>(a.pa, comp_index(PROJ_UP, PART_BIAS, NP), ref))[urow]);
    }
    hb = f32_to_bf16(stack_act<C>(pg, pu));
  } else if (lane == 0) {
    flag_error();
  }
  static_assert(RPSU == 4, "four rows per wave");
  return hb;
}

// One 4-row task, one whole wave: gate/up + activation of rows [4b, 4b+4)
// of one expert (16 lanes per row, as in u_rows) from its codes in cg/cu and
// its rows' scales in `sbw` (LDS, 4 arrays of 16 pieces: gate S, gate B,
// up S, up B); the 4 activations go out as two flagged 8-byte entries
// (2 bf16 + flag) at hf + 2b of the expert's [F/2] entries (put_acts of the
// returned activation).
template <class C>
__device__ __forceinline__ uint32_t task_rows(const StackArgs &a, int32_t ref, bool ok, int b,
                                          const uint4 (&cg)[C::CPLU], const uint4 (&cu)[C::CPLU],
                                          const uint4 *sbw, const uint4 *act_l,
                                          const float *asum_l, float gbv, float ubv) {
  constexpr int U = C::U, NG = C::NG, SGU = C::SGU, CPLU = C::CPLU;
  const int lane = threadIdx.x & 63, uj = lane % SGU, usub = lane / SGU;
  const uint16_t *sbh = reinterpret_cast<const uint16_t *>(sbw);
  constexpr int SBN = 4 * NG;   // bf16 per array: 4 rows x NG groups
  float pg = 0.f, pu = 0.f;
#pragma unroll
  for (int i = 0; i < CPLU; ++i) {
    const int c = i * SGU + uj;
    const int g = usub * NG + (c >> 1);
    const float Sg = bf16_to_f32(sbh[g]), Bg = bf16_to_f32(sbh[SBN + g]);
    const float Su = bf16_to_f32(sbh[2 * SBN + g]), Bu = bf16_to_f32(sbh[3 * SBN + g]);
    const float xs = asum_l[c];
    pg += Sg * chunk_dot_lds<U>(cg[i], act_l, c) + (Bg - 128.f * Sg) * xs;
    pu += Su * chunk_dot_lds<U>(cu[i], act_l, c) + (Bu - 128.f * Su) * xs;
  }
  pg = group_sum<SGU>(pg) + gbv;
  pu = group_sum<SGU>(pu) + ubv;
  uint32_t hb = 0;
  if (ok) hb = f32_to_bf16(stack_act<C>(pg, pu));
  else if (lane == 0) flag_error();
  return hb;
}

// The register loads of one 4-row task, lane by lane: its scale piece (lane
// -> scale array lane / 16, piece lane % 16 of the rows' 256-byte block),
// its rows' projection biases, and its gate and up code chunks, small loads
// first.  An out-of-range ref reads slot 0 (ok false; the task flags it).
template <class C>
struct TaskRegs {
  uint4 sv, cg[C::CPLU], cu[C::CPLU];
  float gbv, ubv;
  bool ok;
  __device__ __forceinline__ void load(const StackArgs &a, int32_t ref, int b) {
    constexpr int D = C::D_, NG = C::NG, SGU = C::SGU, CPLU = C::CPLU, NP = C::NP;
    static_assert(C::RPSU == 4 && SGU == 16 && NG * 2 * 4 == 16 * 16,
                  "a task: 4 rows of 16 lanes; its scales: 4 arrays of 16 pieces");
    const int lane = threadIdx.x & 63, uj = lane % SGU, usub = lane / SGU;
    const char *gw = resolve_packed_safe<typename C::Layout>(a.pa, comp_index(PROJ_GATE, PART_W, NP), ref, ok);
    const char *uw = resolve_packed_safe<typename C::Layout>(a.pa, comp_index(PROJ_UP, PART_W, NP), ref, ok);
    const char *gs = resolve_packed_safe<typename C::Layout>(a.pa, comp_index(PROJ_GATE, PART_S, NP), ref, ok);
    const char *gb = resolve_packed_safe<typename C::Layout>(a.pa, comp_index(PROJ_GATE, PART_B, NP), ref, ok);
    const char *us = resolve_packed_safe<typename C::Layout>(a.pa, comp_index(PROJ_UP, PART_S, NP), ref, ok);
    const char *ub = resolve_packed_safe<typename C::Layout>(a.pa, comp_index(PROJ_UP, PART_B, NP), ref, ok);
    const int arr = lane >> 4, row = 4 * b + usub;
    const char *sa = arr == 0 ? gs : arr == 1 ? gb : arr == 2 ? us : ub;
    sv = load16(reinterpret_cast<const uint4 *>(sa + (int64_t)(4 * b) * NG * 2) + (lane & 15));
    gbv = ubv = 0.f;
    if (C::PBIAS_) {
      bool okb;
      gbv = bf16_to_f32(reinterpret_cast<const uint16_t *>(
          resolve_packed_safe<typename C::Layout>(a.pa, comp_index(PROJ_GATE, PART_BIAS, NP), ref, okb))[row]);
      ubv = bf16_to_f32(reinterpret_cast<const uint16_t *>(
          resolve_packed_safe<typename C::Layout>(a.pa, comp_index(PROJ_UP, PART_BIAS, NP), ref, okb))[row]);
    }
    issue_order_fence();
    const uint4 *g4 = reinterpret_cast<const uint4 *>(gw + (int64_t)row * (D / 2)) + uj;
    const uint4 *u4 = reinterpret_cast<const uint4 *>(uw + (int64_t)row * (D / 2)) + uj;
#pragma unroll
    for (int i = 0; i < CPLU; ++i) {
      cg[i] = load_stream16(g4 + i * SGU);
      cu[i] = load_stream16(u4 + i * SGU);
    }
    issue_order_fence();
  }
  // the task from the loaded registers; `sbw`: this wave's 64 uint4 of LDS
  // for the rows' scales
  __device__ __forceinline__ void run(const StackArgs &a, int32_t ref, int b,
                                      const uint4 *act_l, const float *asum_l, uint4 *sbw,
                                      uint64_t *hf, uint32_t fl) const {
    sbw[threadIdx.x & 63] = sv;
    __atomic_signal_fence(__ATOMIC_SEQ_CST);
    __builtin_amdgcn_wave_barrier();
    __atomic_signal_fence(__ATOMIC_SEQ_CST);
    put_acts(hf + 2 * b, task_rows<C>(a, ref, ok, b, cg, cu, sbw, act_l, asum_l, gbv, ubv), fl);
  }
};

// LDS image of one 4-row task: pieces 0..CPLU-1 gate codes, CPLU..2CPLU-1 up
// codes, 2CPLU the scales (the layout of TaskRegs::sv), each 64 uint4 in
// lane order.
template <class C>
using TaskLds = uint4[2 * C::CPLU + 1][64];

// A 4-row task's pool bytes (TaskRegs' addresses) into `sl` by
// direct-to-LDS loads: no VGPRs; they complete in order with this wave's
// other loads.  An out-of-range ref reads slot 0 (ok false).
template <class C>
__device__ __forceinline__ bool task_stage_lds(const StackArgs &a, int32_t ref, int b,
                                               uint4 (*sl)[64]) {
  constexpr int D = C::D_, NG = C::NG, SGU = C::SGU, CPLU = C::CPLU, NP = C::NP;
  typedef __attribute__((address_space(3))) void lds_void;
  const int lane = threadIdx.x & 63, uj = lane % SGU, usub = lane / SGU;
  bool ok;
  const char *gw = resolve_packed_safe<typename C::Layout>(a.pa, comp_index(PROJ_GATE, PART_W, NP), ref, ok);
  const char *uw = resolve_packed_safe<typename C::Layout>(a.pa, comp_index(PROJ_UP, PART_W, NP), ref, ok);
  const char *gs = resolve_packed_safe<typename C::Layout>(a.pa, comp_index(PROJ_GATE, PART_S, NP), ref, ok);
  const char *gb = resolve_packed_safe<typename C::Layout>(a.pa, comp_index(PROJ_GATE, PART_B, NP), ref, ok);
  const char *us = resolve_packed_safe<typename C::Layout>(a.pa, comp_index(PROJ_UP, PART_S, NP), ref, ok);
  const char *ub = resolve_packed_safe<typename C::Layout>(a.pa, comp_index(PROJ_UP, PART_B, NP), ref, ok);
  const int arr = lane >> 4, row = 4 * b + usub;
  const char *sa = arr == 0 ? gs : arr == 1 ? gb : arr == 2 ? us : ub;
  const uint4 *g4 = reinterpret_cast<const uint4 *>(gw + (int64_t)row * (D / 2)) + uj;
  const uint4 *u4 = reinterpret_cast<const uint4 *>(uw + (int64_t)row * (D / 2)) + uj;
  __builtin_amdgcn_global_load_lds(
      reinterpret_cast<const uint4 *>(sa + (int64_t)(4 * b) * NG * 2) + (lane & 15),
      (lds_void *)&sl[2 * CPLU][0], 16, 0, 0);
#pragma unroll
  for (int i = 0; i < CPLU; ++i) {
    __builtin_amdgcn_global_load_lds(g4 + i * SGU, (lds_void *)&sl[i][0], 16, 0, 0);
    __builtin_amdgcn_global_load_lds(u4 + i * SGU, (lds_void *)&sl[CPLU + i][0], 16, 0, 0);
  }
  return ok;
}

// The gate/up waves' rows of the predicted expert (u_rows, when `urows`),
// with a spare task's bytes going to LDS beside them (task_stage_lds, when
// `spare`; returns its ok in sok).  The LDS operands are restrict pointers so
// the compiler knows u_rows' LDS reads cannot alias the direct-to-LDS loads
// and does not wait for those before them.
template <class C>
__device__ __forceinline__ uint32_t u_rows_with_spare(
    const StackArgs &a, bool urows, int32_t uref, int row0, const uint4 (&cg)[C::CPLU],
    const uint4 (&cu)[C::CPLU], const uint4 *__restrict__ act_l,
    const float *__restrict__ asum_l, const uint4 (*__restrict__ sbu_l)[C::SB_U4],
    bool spare, int32_t sref, int b, uint4 (*__restrict__ sl)[64], bool &sok) {
  // the staged codes u_rows is about to use are awaited here, for every
  // wave alike, so that no later wait for them also covers the spare loads
  __builtin_amdgcn_s_waitcnt(0);
  if (spare) sok = task_stage_lds<C>(a, sref, b, sl);
  return urows ? u_rows<C>(a, uref, row0, cg, cu, act_l, asum_l, sbu_l) : 0u;
}

// The task from the bytes task_stage_lds put in `sl`; returns the activation
// as task_rows.  The direct-to-LDS loads are awaited explicitly, with every
// LDS read kept after the wait: the compiler's own wait for them is not
// placed before all of these reads.
template <class C>
__device__ __forceinline__ uint32_t task_rows_lds(const StackArgs &a, int32_t ref, bool ok,
                                                  int b, const TaskLds<C> &sl,
                                                  const uint4 *act_l, const float *asum_l) {
  constexpr int CPLU = C::CPLU, NP = C::NP;
  const int lane = threadIdx.x & 63, usub = (lane & 63) / C::SGU;
  __builtin_amdgcn_s_waitcnt(0);
  issue_order_fence();
  float gbv = 0.f, ubv = 0.f;
  if (C::PBIAS_) {
    bool okb;
    gbv = bf16_to_f32(reinterpret_cast<const uint16_t *>(
        resolve_packed_safe<typename C::Layout>(a.pa, comp_index(PROJ_GATE, PART_BIAS, NP), ref, okb))[4 * b + usub]);
    ubv = bf16_to_f32(reinterpret_cast<const uint16_t *>(
        resolve_packed_safe<typename C::Layout>(a.pa, comp_index(PROJ_UP, PART_BIAS, NP), ref, okb))[4 * b + usub]);
  }
  uint4 cg[CPLU], cu[CPLU];
#pragma unroll
  for (int i = 0; i < CPLU; ++i) {
    cg[i] = sl[i][lane];
    cu[i] = sl[CPLU + i][lane];
  }
  return task_rows<C>(a, ref, ok, b, cg, cu, sl[2 * CPLU], act_l, asum_l, gbv, ubv);
}

// One fix-up task (a routed expert that was not predicted), straight from
// the pool.
template <class C>
__device__ __forceinline__ void fix_task(const StackArgs &a, int32_t ref, int b,
                                         const uint4 *act_l, const float *asum_l, uint4 *sbw,
                                         uint64_t *hf, uint32_t fl) {
  ref = __builtin_amdgcn_readfirstlane(ref);
  TaskRegs<C> r;
  r.load(a, ref, b);
  r.run(a, ref, b, act_l, asum_l, sbw, hf, fl);
}

// One whole wave: the F activations of one expert (`hf`, its F/2 flagged
// entries) as two 16-byte pieces
// per lane (pieces lane and lane + 64, 8 bf16 each), polled until every entry
// carries the flag `fl`.  Bounded like wave_wait.
template <int HU4>
__device__ __forceinline__ void get_acts(const uint64_t *hf, uint32_t fl, const Abort &ab,
                                         uint4 &p0, uint4 &p1) {
  const int lane = threadIdx.x & 63;
  const uint64_t *e0 = hf + 4 * min(lane, HU4 - 1), *e1 = hf + 4 * min(lane + 64, HU4 - 1);
  uint32_t spins = 0;
  while (true) {
    uint64_t v[8];
#pragma unroll
    for (int q = 0; q < 4; ++q) {
      v[q] = __hip_atomic_load(e0 + q, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
      v[4 + q] = __hip_atomic_load(e1 + q, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    }
    bool ok = true;
#pragma unroll
    for (int q = 0; q < 8; ++q) ok = ok && (uint32_t)(v[q] >> 32) == fl;
    p0 = make_uint4((uint32_t)v[0], (uint32_t)v[1], (uint32_t)v[2], (uint32_t)v[3]);
    p1 = make_uint4((uint32_t)v[4], (uint32_t)v[5], (uint32_t)v[6], (uint32_t)v[7]);
    if (__ballot(!ok) == 0) break;
    if (ab.gave_up(++spins)) break;
    __builtin_amdgcn_s_sleep(1);
  }
}

// One whole wave: pieces [PPW * w, PPW * w + PPW) of one expert's F
// activations (16-byte pieces of 8 bf16, 4 flagged entries each; lane j <
// PPW takes piece PPW * w + j), polled until each carries the flag `fl`.
// Lanes past PPW load the wave's first piece and do not wait on it.
template <int PPW>
__device__ __forceinline__ void acts_part_issue(const uint64_t *hf, int w, uint64_t (&v)[4]) {
  const int lane = threadIdx.x & 63;
  const uint64_t *e = hf + 4 * (PPW * w + (lane < PPW ? lane : 0));
#pragma unroll
  for (int q = 0; q < 4; ++q)
    v[q] = __hip_atomic_load(e + q, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
// get_acts_part from a first round already issued (acts_part_issue, into v):
// its flags checked, further rounds polled as needed.
template <int PPW>
__device__ __forceinline__ uint4 acts_part_finish(const uint64_t *hf, int w, uint32_t fl,
                                                  const Abort &ab, uint64_t (&v)[4]) {
  const bool mine = (threadIdx.x & 63) < PPW;
  uint32_t spins = 0;
  while (true) {
    bool ok = true;
#pragma unroll
    for (int q = 0; q < 4; ++q) ok = ok && (uint32_t)(v[q] >> 32) == fl;
    if (__ballot(mine && !ok) == 0) break;
    if (ab.gave_up(++spins)) break;
    __builtin_amdgcn_s_sleep(1);
    acts_part_issue<PPW>(hf, w, v);
  }
  return make_uint4((uint32_t)v[0], (uint32_t)v[1], (uint32_t)v[2], (uint32_t)v[3]);
}
template <int PPW>
__device__ __forceinline__ uint4 get_acts_part(const uint64_t *hf, int w, uint32_t fl,
                                               const Abort &ab) {
  uint64_t v[4];
  acts_part_issue<PPW>(hf, w, v);
  return acts_part_finish<PPW>(hf, w, fl, ab, v);
}

// Register loads of one workgroup's gate/up block (waves 0..WAVES_U-1: the
// codes of its rows; every thread: its share of the block's scales).
template <class C>
__device__ __forceinline__ void u_load(const StackArgs &a, int32_t ref, int row0,
                                       uint4 (&cg)[C::CPLU], uint4 (&cu)[C::CPLU],
                                       uint4 (&sr)[C::SIT]) {
  constexpr int D = C::D_, NG = C::NG, SGU = C::SGU, CPLU = C::CPLU, RPSU = C::RPSU;
  constexpr int SB_U4 = C::SB_U4, NP = C::NP, NT = C::NT;
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  // No branch around any load and no conditional load (either makes the
  // compiler wait for the loads before it): an out-of-range ref reads slot 0
  // (the phase that consumes the registers flags it), surplus lanes load a
  // clamped index.
  ref = __builtin_amdgcn_readfirstlane(ref);
  bool ok;
  const char *gw = resolve_packed_safe<typename C::Layout>(a.pa, comp_index(PROJ_GATE, PART_W, NP), ref, ok);
  const char *uw = resolve_packed_safe<typename C::Layout>(a.pa, comp_index(PROJ_UP, PART_W, NP), ref, ok);
  const char *sb[4] = {resolve_packed_safe<typename C::Layout>(a.pa, comp_index(PROJ_GATE, PART_S, NP), ref, ok),
                       resolve_packed_safe<typename C::Layout>(a.pa, comp_index(PROJ_GATE, PART_B, NP), ref, ok),
                       resolve_packed_safe<typename C::Layout>(a.pa, comp_index(PROJ_UP, PART_S, NP), ref, ok),
                       resolve_packed_safe<typename C::Layout>(a.pa, comp_index(PROJ_UP, PART_B, NP), ref, ok)};
#pragma unroll
  for (int it = 0; it < C::SIT; ++it) {
    const int i = min(it * NT + tid, 4 * SB_U4 - 1);
    const int p = i / SB_U4, o = i % SB_U4;
    const char *sp = p == 0 ? sb[0] : p == 1 ? sb[1] : p == 2 ? sb[2] : sb[3];
    sr[it] = load16(reinterpret_cast<const uint4 *>(sp + (int64_t)row0 * NG * 2) + o);
  }
  if (wave < C::WAVES_U) {
    const int uj = lane % SGU, usub = lane / SGU;
    const int urow = row0 + wave * RPSU + usub;
    const uint4 *g4 = reinterpret_cast<const uint4 *>(gw + (int64_t)urow * (D / 2));
    const uint4 *u4 = reinterpret_cast<const uint4 *>(uw + (int64_t)urow * (D / 2));
#pragma unroll
    for (int i = 0; i < CPLU; ++i) {
      cg[i] = load_stream16(g4 + i * SGU + uj);
      cu[i] = load_stream16(u4 + i * SGU + uj);
    }
  }
}

// Register loads of one wave's down rows (8 output rows) of one expert.
template <class C>
__device__ __forceinline__ void d_load(const StackArgs &a, int32_t ref, int drow0,
                                       uint4 (&cd)[C::CPLD], uint4 (&sdr)[C::SDIT]) {
  constexpr int F = C::F_, NGF = C::NGF, SGD = C::SGD, CPLD = C::CPLD, UF = C::UF;
  constexpr int SBD_U4 = C::SBD_U4, NP = C::NP;
  const int lane = threadIdx.x & 63;
  // (unconditional loads, as in u_load)
  ref = __builtin_amdgcn_readfirstlane(ref);
  bool ok;
  const char *dw = resolve_packed_safe<typename C::Layout>(a.pa, comp_index(PROJ_DOWN, PART_W, NP), ref, ok);
  const char *ds = resolve_packed_safe<typename C::Layout>(a.pa, comp_index(PROJ_DOWN, PART_S, NP), ref, ok);
  const char *db = resolve_packed_safe<typename C::Layout>(a.pa, comp_index(PROJ_DOWN, PART_B, NP), ref, ok);
#pragma unroll
  for (int it = 0; it < C::SDIT; ++it) {
    const int i = min(it * 64 + lane, 2 * SBD_U4 - 1);
    const int p = i / SBD_U4, o = i % SBD_U4;
    sdr[it] = load16(reinterpret_cast<const uint4 *>((p ? db : ds) + (int64_t)drow0 * NGF * 2) + o);
  }
  const int dj = lane % SGD, dsub = lane / SGD;
  const uint4 *d4 = reinterpret_cast<const uint4 *>(dw + (int64_t)(drow0 + dsub) * (F / 2));
#pragma unroll
  for (int i = 0; i < CPLD; ++i)   // surplus chunks (c >= UF) re-read the last one, unused
    cd[i] = load_stream16(d4 + min(i * SGD + dj, UF - 1));
}

template <int D, int F, int K, bool PBIAS, int ACT, int MODE, int RENORM>
__global__ __launch_bounds__(512) void stack_decode_kernel(StackArgs a) {
  using C = StackCfg<D, F, K, PBIAS, ACT, MODE, RENORM>;
  using WS = StackWs<F, K>;
  constexpr int NT = C::NT, U = C::U, SB_U4 = C::SB_U4;
  constexpr int UF = C::UF, NGF = C::NGF, SGD = C::SGD, CPLD = C::CPLD;
  constexpr int ROWS_D = C::ROWS_D, SBD_U4 = C::SBD_U4, NP = C::NP;
  constexpr int ROWS_U = C::ROWS_U, NPOS = F / ROWS_U;
  constexpr int XU4 = D / 8, HU4 = F / 8;
  constexpr int RIT = (XU4 + 63) / 64;       // router-row pieces per lane
  constexpr int XIT = (XU4 + NT - 1) / NT;
  constexpr int W_ROUTER = 6, W_RANK = 7;    // the router wave and the ranking wave
  static_assert(C::WAVES_U <= W_ROUTER && NT / 64 == 8, "wave roles");
  static_assert(C::ITEMS_U == K * NPOS, "one gate/up block per (position, row block)");
  constexpr int FT = F / 4;          // 4-row tasks per expert (fix-up, spares)
  constexpr int NWG = C::ITEMS_D;    // the grid
  static_assert(K * FT <= C::WAVES_U * NWG && kSpare <= K, "every task has a wave");
  // expert position p (gate/up and down rows) on the workgroups w with
  // w % K == p, i.e. on one XCD, so its activations stay in that XCD's L2
  constexpr int WPP = NWG / K;       // workgroups per position
  constexpr int DROWS_WG = D / WPP;  // a workgroup's down rows of its position
  static_assert(K == kXcds && NWG == K * NPOS && DROWS_WG == 8 * ROWS_D,
                "one position per XCD; 8 waves of ROWS_D down rows per workgroup");
  constexpr int PPW = HU4 / 8;       // activation pieces each wave polls
  static_assert(HU4 % 8 == 0 && PPW % 4 == 0 && PPW <= 64, "activation pieces per wave");
  static_assert(K * ROWS_D == 64 && D <= kStackMaxD, "the combine: one lane per (rank, row)");
  constexpr int W_COMB = C::WAVES_U - 1;   // the wave that combines the previous layer

  __shared__ uint4 act_l[4 * U];
  __shared__ float asum_l[U];
  __shared__ uint4 sbu_l[4][SB_U4];
  __shared__ uint4 hact_l[K][4 * UF];   // per wave: fix-up tasks' scale scratch
  __shared__ uint4 hact_s[4 * UF];      // the position's activations (down input)
  __shared__ float hsum_s[UF];
  __shared__ uint4 sbd_l[K][2 * SBD_U4];
  __shared__ float red_l[K][ROWS_D];
  __shared__ int sel_id[K];
  __shared__ float sel_sc[K];
  __shared__ int32_t sel_ref[K];
  __shared__ int pred_buf[2][K + kSpare];      // lookahead's best, rank order (slot l & 1)
  __shared__ int32_t pred_ref[2][K + kSpare];  // their slot refs (looked up by the ranking wave)
  __shared__ int pred_cnt[2];                  // staged positions (<= K)
  __shared__ int spare_cnt[2];                 // spare positions (<= kSpare)
  __shared__ int d_rank[K];          // D wave w: routing rank of its expert
  __shared__ int d_fix[K];           // D wave w: fix-up slot, or -1 (predicted at w)
  __shared__ int32_t miss_ref[K];    // fix-up slot -> slot ref
  __shared__ int miss_src[K];        // i-th unstaged routed expert: fix-up slot, or -1 - spare
  __shared__ int n_miss;
  __shared__ int staged[2];          // gate/up waves done staging x (slot l & 1)
  __shared__ TaskLds<C> spare_l[2];  // the spare tasks' bytes (waves 0 and 1)

  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int wg = blockIdx.x;
  const uint32_t ep = a.epoch;
  const Abort ab{reinterpret_cast<uint32_t *>(a.ws + WS::kAbort), ep};
  uint64_t *const lgt = reinterpret_cast<uint64_t *>(a.ws + WS::kLgt);
  uint64_t *const hpred = reinterpret_cast<uint64_t *>(a.ws + WS::kHpred);
  uint64_t *const hfix = reinterpret_cast<uint64_t *>(a.ws + WS::kHfix);
  float *const part = reinterpret_cast<float *>(a.ws + WS::kPart);
  const int upos = wg % K, urow0 = (wg / K) * ROWS_U;          // gate/up block
  const int dwrow = (wg / K) * DROWS_WG + wave * ROWS_D;       // this wave's down rows
  const int drow0 = wg * ROWS_D;                               // combined output rows
  const int dj = lane % SGD, dsub = lane / SGD;
  if (tid < 2) {
    pred_cnt[tid] = 0;               // layer 0 has no prediction
    spare_cnt[tid] = 0;
    staged[tid] = 0;
  }

  // staged registers, carried from the end of one layer into the next
  uint4 cg[C::CPLU], cu[C::CPLU], sr[C::SIT], cd[CPLD], sdr[C::SDIT];
#pragma unroll
  for (int i = 0; i < C::CPLU; ++i) cg[i] = cu[i] = make_uint4(0, 0, 0, 0);
#pragma unroll
  for (int i = 0; i < C::SIT; ++i) sr[i] = make_uint4(0, 0, 0, 0);
#pragma unroll
  for (int i = 0; i < CPLD; ++i) cd[i] = make_uint4(0, 0, 0, 0);
#pragma unroll
  for (int i = 0; i < C::SDIT; ++i) sdr[i] = make_uint4(0, 0, 0, 0);

  for (int l = 0; l < a.L; ++l) {
    const bool has_next = l + 1 < a.L;
    const int nrows = a.E * (has_next ? 2 : 1);
    const int32_t *tab = KARG(table) + (size_t)l * a.E;
    if (wave == 0) trace_mark(a, l, TR_START);
    // the router row's weights before the wait (wave 6)
    uint4 wr[RIT];
    const bool rrow = wave == W_ROUTER && wg < nrows;
    const bool rnxt = wg >= a.E;
    if (rrow) {
      const int e = rnxt ? wg - a.E : wg;
      const uint4 *w4 =
          reinterpret_cast<const uint4 *>(KARG(W) + ((size_t)(rnxt ? l + 1 : l) * a.E + e) * D);
#pragma unroll
      for (int it = 0; it < RIT; ++it) {
        const int i = lane + it * 64;
        wr[it] = (i < XU4) ? load_stream16(w4 + i) : make_uint4(0, 0, 0, 0);
      }
    }
    // ------------------------------------------------------ layer start ----
    // polled by the ranking wave: the one wave with no staging loads in
    // flight here (loads complete in order, so a poll issued behind staging
    // loads would return only after them); it issues its own down staging
    // right after
    if (l > 0) wg_wait(counter<WS>(a, l - 1, CNT_D), ep * C::ITEMS_D, W_RANK, ab);
    else __syncthreads();
    if (wave == 0) trace_mark(a, l, TR_R_WAITED);
    const int pcnt = pred_cnt[l & 1];
    const int *P = pred_buf[l & 1];
    if (wave == W_RANK && upos < pcnt) d_load<C>(a, pred_ref[l & 1][upos], dwrow, cd, sdr);
    // ------------------------------------------------------- role split ----
    uint32_t comb = 0;   // wave W_COMB: one partial output of layer l-1 per lane
    if (wave < W_ROUTER) {
      // stage x_l (pair order + 32-input sums) and the predicted block's
      // scales; the six gate/up waves then meet on an LDS counter, so the
      // router and ranking waves never wait for the staging
      static_assert(XIT == 1 && XU4 <= 64 * W_ROUTER && C::SIT == 1 &&
                        4 * SB_U4 <= 64 * W_ROUTER, "staging by the gate/up waves");
      // a spare task's pool bytes (task t: 4 rows of spare t / FT, on waves
      // 0 and 1) go to LDS by direct-to-LDS loads issued after x is staged
      // and the gate/up waves have met (a wait for x or the meeting's release
      // would otherwise wait for them too), so they land while the predicted
      // rows compute
      static_assert(kSpare * FT <= 2 * NWG, "spare tasks fit waves 0 and 1");
      const int ts = wave * NWG + wg;
      const bool spare = wave < 2 && ts < spare_cnt[l & 1] * FT;
      const int32_t sref =
          __builtin_amdgcn_readfirstlane(pred_ref[l & 1][K + min(ts / FT, kSpare - 1)]);
      bool sok = false;
      {
        const uint4 *x4 = reinterpret_cast<const uint4 *>(a.x + (size_t)l * D);
        float s = 0.f;
        if (tid < XU4) s = stage_piece<U>(act_l, tid, x4[tid]);
        s += dpp_f<kDppQuadXor1>(s);
        s += dpp_f<kDppQuadXor2>(s);
        if (tid < XU4 && (tid & 3) == 0) asum_l[tid >> 2] = s;
        if (upos < pcnt && tid < 4 * SB_U4) (&sbu_l[0][0])[tid] = sr[0];
      }
      if (lane == 0) {
        __hip_atomic_fetch_add(&staged[l & 1], 1, __ATOMIC_RELEASE, __HIP_MEMORY_SCOPE_WORKGROUP);
        while (__hip_atomic_load(&staged[l & 1], __ATOMIC_ACQUIRE, __HIP_MEMORY_SCOPE_WORKGROUP) <
               W_ROUTER)
          __builtin_amdgcn_s_sleep(1);
      }
      __builtin_amdgcn_wave_barrier();
      __atomic_signal_fence(__ATOMIC_SEQ_CST);
      // gate/up of the predicted expert at this workgroup's position, then
      // the spare task from LDS, and only then the two publishes (a store
      // between the direct-to-LDS loads and their wait would be waited for
      // too)
      const bool urows = wave < C::WAVES_U && upos < pcnt;
      const uint32_t hu = u_rows_with_spare<C>(a, urows, pred_ref[l & 1][upos], urow0, cg, cu,
                                               act_l, asum_l, sbu_l, spare, sref, ts % FT,
                                               spare_l[wave], sok);
      uint32_t hs = 0;
      if (spare) hs = task_rows_lds<C>(a, sref, sok, ts % FT, spare_l[wave], act_l, asum_l);
      if (urows)
        put_acts_xcd(hpred + (size_t)upos * (F / 2) + (urow0 + wave * C::RPSU) / 2, hu,
                     layer_flag(a, l));
      if (spare)
        put_acts(hpred + (size_t)(K + ts / FT) * (F / 2) + 2 * (ts % FT), hs, layer_flag(a, l));
      // this wave's down rows of the position's predicted expert, issued once
      // its gate/up work is done (at the previous layer's end they would
      // queue ahead of the boundary poll)
      if (upos < pcnt) d_load<C>(a, pred_ref[l & 1][upos], dwrow, cd, sdr);
      // layer l-1's score-weighted outputs of this workgroup's rows, complete
      // since this layer's start: loaded now, summed before the arrival
      if (wave == W_COMB && l > 0)
        comb = __hip_atomic_load(reinterpret_cast<const uint32_t *>(
                                     part + ((size_t)((l - 1) & 1) * K + lane / ROWS_D) *
                                                kStackMaxD + drow0 + lane % ROWS_D),
                                 __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
      if (wave == 0) trace_mark(a, l, TR_U_ARRIVED);
      if (wave == 1) trace_mark(a, l, TR_SPARE1);
      if (wave == 2) trace_mark(a, l, TR_UROWS2);
    } else if (wave == W_ROUTER) {
      // one router row (the lane partition and summation order of
      // route_kernel, so both paths produce bit-identical logits)
      if (rrow) {
        const int e = rnxt ? wg - a.E : wg;
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
        if (lane == 0) put_logit(lgt + (rnxt ? a.E : 0) + e, acc, layer_flag(a, l));
        trace_mark(a, l, TR_R_ARRIVED);
      }
      // this wave's down rows, loaded once its router row is out (its x
      // loads then have no staging loads ahead of them)
      if (upos < pcnt) d_load<C>(a, pred_ref[l & 1][upos], dwrow, cd, sdr);
      // lookahead ranking of layer l+1: raw bf16 logits of its router on x_l
      if (has_next) {
        const int e0 = lane, e1 = lane + 64;
        const uint16_t *bias0 = KARG(bias);
        const uint16_t *bias = bias0 ? bias0 + (size_t)(l + 1) * a.E : nullptr;
        const float b0 = bias ? bf16_to_f32(bias[min(e0, a.E - 1)]) : 0.f;   // before the wait
        const float b1 = bias ? bf16_to_f32(bias[min(e1, a.E - 1)]) : 0.f;
        const int32_t *tabn = KARG(table) + (size_t)(l + 1) * a.E;
        const int32_t t0 = tabn[min(e0, a.E - 1)], t1 = tabn[min(e1, a.E - 1)];
        float l0, l1;
        get_logits(lgt + a.E, a.E, layer_flag(a, l), ab, l0, l1);
        const float z0 = e0 < a.E ? round_bf16(l0 + b0) : -INFINITY;
        const float z1 = e1 < a.E ? round_bf16(l1 + b1) : -INFINITY;
        bool s0, s1;
        int r0, r1;
        // the caller's k_pred, and at least the K staged + kSpare spare
        // positions for this kernel's own speculation
        const int ksel = min(max(a.kp, K + kSpare), a.E);
        select_topk(e0 < a.E ? order_key(z0) : -1, e1 < a.E ? order_key(z1) : -1, ksel, lane,
                    s0, s1, r0, r1);
        if (wg == 0) {
          int32_t *pred = KARG(pred);
          if (s0 && r0 < a.kp) pred[(size_t)l * a.kp + r0] = e0;
          if (s1 && r1 < a.kp) pred[(size_t)l * a.kp + r1] = e1;
        }
        int *pn = pred_buf[(l + 1) & 1];
        int32_t *pr = pred_ref[(l + 1) & 1];
        if (s0 && r0 < K + kSpare) {
          pn[r0] = e0;
          pr[r0] = t0;
        }
        if (s1 && r1 < K + kSpare) {
          pn[r1] = e1;
          pr[r1] = t1;
        }
        if (lane == 0) {
          pred_cnt[(l + 1) & 1] = min(a.kp, K);
          spare_cnt[(l + 1) & 1] = min(kSpare, max(0, ksel - K));   // a wider k_pred: ranks
                                                                     // past K + kSpare unused
        }
        trace_mark(a, l, TR_LOOKED);
      }
    } else {
      // ---- routing: every workgroup ranks this layer's logits ----------
      const int e0 = lane, e1 = lane + 64;
      const uint16_t *bias0 = KARG(bias);
      const uint16_t *bias = bias0 ? bias0 + (size_t)l * a.E : nullptr;
      const float b0 = bias ? bf16_to_f32(bias[min(e0, a.E - 1)]) : 0.f;   // before the wait
      const float b1 = bias ? bf16_to_f32(bias[min(e1, a.E - 1)]) : 0.f;
      // every expert's slot ref, also before the wait (clamped, unconditional)
      const int32_t t0 = tab[min(e0, a.E - 1)], t1 = tab[min(e1, a.E - 1)];
      float l0, l1;
      // The first poll waits ~0.5 us (1,024 clocks): the router rows are
      // published ~0.5 us after the boundary, and polls of the 256 workgroups
      // issued before that only queue on the entries' lines ahead of the
      // rows' own stores and of the polls that will see them (measured:
      // every logit seen 0.6 us sooner, 3.2 % more tokens/s; waiting for this
      // workgroup's own router row instead was slower).
      __builtin_amdgcn_s_sleep(16);
      get_logits(lgt, a.E, layer_flag(a, l), ab, l0, l1);
      trace_mark(a, l, TR_R_ALL);
      const float z0 = e0 < a.E ? round_bf16(l0 + b0) : -INFINITY;
      const float z1 = e1 < a.E ? round_bf16(l1 + b1) : -INFINITY;
      trace_mark_after(a, l, TR_LOGITS, z0 + z1);
      float v0 = z0, v1 = z1;
      if (MODE == MOE_ROUTE_SOFTMAX_TOPK) {
        const float m = wave_max(fmaxf(z0, z1));
        const float x0 = (e0 < a.E) ? expf(z0 - m) : 0.f;
        const float x1 = (e1 < a.E) ? expf(z1 - m) : 0.f;
        const float s = group_sum<64>(x0 + x1);
        v0 = round_bf16(x0 / s);
        v1 = round_bf16(x1 / s);
      }
      trace_mark_after(a, l, TR_SOFTMAX, v0 + v1);
      bool s0, s1;
      int r0, r1;
      select_topk(e0 < a.E ? order_key(v0) : -1, e1 < a.E ? order_key(v1) : -1, K, lane,
                  s0, s1, r0, r1);
      trace_mark_after(a, l, TR_TOPK, (float)(r0 + r1));
      float sc0 = v0, sc1 = v1;
      if (MODE == MOE_ROUTE_SOFTMAX_TOPK) {
        if (RENORM) {
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
      if (s0) {
        sel_id[r0] = e0;
        sel_sc[r0] = sc0;
        sel_ref[r0] = t0;
      }
      if (s1) {
        sel_id[r1] = e1;
        sel_sc[r1] = sc1;
        sel_ref[r1] = t1;
      }
      // ---- which D wave takes which routed expert -----------------------
      // Predicted position w keeps its expert if it was routed (its codes
      // are staged there); the routed experts that were not predicted go,
      // in rank order, to the other positions in order (fix-up slots).
      __atomic_signal_fence(__ATOMIC_SEQ_CST);
      __builtin_amdgcn_wave_barrier();
      __atomic_signal_fence(__ATOMIC_SEQ_CST);
      const uint64_t below = lane ? (~0ull >> (64 - lane)) : 0ull;
      bool miss = false, routed = false;
      int rank_w = -1, sp = -1;
      int32_t ref_r = 0;
      const int nsp = spare_cnt[l & 1];
      if (lane < K) {
        // fixed trip counts, so every LDS read below issues in one batch
        int pv[K + kSpare], sv[K];
#pragma unroll
        for (int p = 0; p < K + kSpare; ++p) pv[p] = P[p];
#pragma unroll
        for (int r = 0; r < K; ++r) sv[r] = sel_id[r];
        const int er = sel_id[lane];   // routed expert of rank `lane`
        ref_r = sel_ref[lane];
        const int pw = lane < pcnt ? P[min(lane, K - 1)] : -1;   // predicted at position `lane`
        miss = true;
#pragma unroll
        for (int p = 0; p < K; ++p) miss = miss && !(p < pcnt && pv[p] == er);
#pragma unroll
        for (int q = 0; q < kSpare; ++q)
          if (q < nsp && pv[K + q] == er) sp = q;    // computed at a spare position
#pragma unroll
        for (int r = 0; r < K; ++r)
          if (pw >= 0 && sv[r] == pw) { routed = true; rank_w = r; }
      }
      // unstaged routed experts (rank order): a spare's activations are
      // ready; the others (true misses) get fix-up slots
      const uint64_t mm = __ballot(miss), fm = __ballot(lane < K && !routed);
      const uint64_t tm = __ballot(miss && sp < 0);
      if (miss && sp < 0) miss_ref[__popcll(tm & below)] = ref_r;
      if (miss) miss_src[__popcll(mm & below)] = sp >= 0 ? -1 - sp : __popcll(tm & below);
      if (lane < K) {
        if (routed) {
          d_rank[lane] = rank_w;
          d_fix[lane] = -1;
        } else {
          const int fi = __popcll(fm & below);
          uint64_t m = mm;
          for (int i = 0; i < fi; ++i) m &= m - 1;
          d_rank[lane] = (int)__builtin_ctzll(m);
          d_fix[lane] = fi;
        }
      }
      if (lane == 0) n_miss = __popcll(tm);
    }
    lds_barrier();   // the routing's results (LDS) for every wave
    // the first poll of the position's predicted activations, issued before
    // this phase's LDS and scalar reads: the down rows use it if the routing
    // kept that expert
    uint64_t pv4[4] = {0, 0, 0, 0};
    if (upos < pcnt) acts_part_issue<PPW>(hpred + (size_t)upos * (F / 2), wave, pv4);
    if (wave == 0) trace_mark(a, l, TR_SELECTED);
    if (tid == 0) {   // next layer's slots; nobody touches them before its start
      staged[(l + 1) & 1] = 0;
    }
    if (wg == 0 && tid < K) {
      KARG(ids)[(size_t)l * K + tid] = sel_id[tid];
      KARG(scores)[(size_t)l * K + tid] = sel_sc[tid];
      KARG(refs_out)[(size_t)l * K + tid] = sel_ref[tid];
      if (sel_ref[tid] < 0) atomicAdd(KARG(miss) + l, 1);
    }
    // this position's routed expert; its down rows, if it was not the
    // predicted one, loaded now so their latency overlaps the fix-up pass
    const int d_r = d_rank[upos], d_fx = d_fix[upos];
    const int32_t d_ref = sel_ref[d_r];
    if (d_fx >= 0) d_load<C>(a, d_ref, dwrow, cd, sdr);
    // ------------------------------------------ fix-up: unpredicted ----
    // Spread over the whole grid: task t = wave * (grid) + workgroup of the
    // gate/up waves computes 4 rows of fix-up slot t / FT, so one miss costs
    // each workgroup at most one wave's pass over 4 rows.
    {
      const int t = wave * NWG + wg;
      if (wave < C::WAVES_U && t < n_miss * FT)
        fix_task<C>(a, miss_ref[t / FT], t % FT, act_l, asum_l, hact_l[wave],
                    hfix + (size_t)(t / FT) * (F / 2), layer_flag(a, l));
      if (wave == 0) trace_mark(a, l, TR_FIXED);
    }
    // ------------------------------------------------------------ D_l ----
    // The position's routed expert, ROWS_D rows per wave: each wave polls
    // PPW pieces of its activations (XCD-local entries for the predicted
    // expert) into the shared LDS copy, then its rows' score-weighted outputs
    // go to the rank's partial output row (summed in rank order by the
    // combine, after the layer).
    {
      const int r = d_r, fx = d_fx;
      const int32_t dref = d_ref;
      const char *dw = resolve_packed<typename C::Layout>(a.pa, comp_index(PROJ_DOWN, PART_W, NP), dref);
      if (dw != nullptr) {
        uint4 *sbd = sbd_l[wave];
#pragma unroll
        for (int it = 0; it < C::SDIT; ++it) {
          const int i = it * 64 + lane;
          if (i < 2 * SBD_U4) sbd[i] = sdr[it];
        }
        const int src = fx < 0 ? 0 : miss_src[fx];
        const uint64_t *hf = fx < 0    ? hpred + (size_t)upos * (F / 2)
                             : src >= 0 ? hfix + (size_t)src * (F / 2)
                                        : hpred + (size_t)(K - 1 - src) * (F / 2);
        const uint4 pc = fx < 0 ? acts_part_finish<PPW>(hf, wave, layer_flag(a, l), ab, pv4)
                                : get_acts_part<PPW>(hf, wave, layer_flag(a, l), ab);
        if (wave == 0) trace_mark(a, l, TR_D_WAITED);
        const int i = PPW * wave + lane;
        float s = 0.f;
        if (lane < PPW) s = stage_piece<UF>(hact_s, i, pc);
        s += dpp_f<kDppQuadXor1>(s);
        s += dpp_f<kDppQuadXor2>(s);
        if (lane < PPW && (i & 3) == 0) hsum_s[i >> 2] = s;
      } else if (wave == 0 && lane == 0) {
        flag_error();
      }
      __syncthreads();   // every wave's pieces staged
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
            p += Sd * chunk_dot_lds<UF>(cd[i], hact_s, c) + (Bd - 128.f * Sd) * hsum_s[c];
          }
        }
      }
      p = group_sum<SGD>(p);
      if (dj == 0) {
        if (PBIAS && dw != nullptr)
          p += bf16_to_f32(reinterpret_cast<const uint16_t *>(
              resolve_packed<typename C::Layout>(a.pa, comp_index(PROJ_DOWN, PART_BIAS, NP), dref))[dwrow + dsub]);
        const float v = (dw != nullptr) ? sel_sc[r] * p : 0.f;
        __hip_atomic_store(reinterpret_cast<uint32_t *>(
                               part + ((size_t)(l & 1) * K + r) * kStackMaxD + dwrow + dsub),
                           __float_as_uint(v), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
      }
    }
    // the combine of layer l-1 (its partials were loaded during this layer):
    // ROWS_D output rows, the k ranks summed in rank order
    if (wave == W_COMB && l > 0) {
      red_l[lane / ROWS_D][lane % ROWS_D] = __uint_as_float(comb);
      __atomic_signal_fence(__ATOMIC_SEQ_CST);
      __builtin_amdgcn_wave_barrier();
      __atomic_signal_fence(__ATOMIC_SEQ_CST);
      if (lane < ROWS_D) {
        float yv = 0.f;
        for (int w = 0; w < K; ++w) yv += red_l[w][lane];   // rank order
        KARG(y)[(size_t)(l - 1) * D + drow0 + lane] = (uint16_t)f32_to_bf16(yv);
      }
    }
    wg_arrive(counter<WS>(a, l, CNT_D));
    if (wave == 0) trace_mark(a, l, TR_D_ARRIVED);
    // ----------------------------- staging loads of layer l+1's prediction
    // (its down rows are staged during layer l+1: the ranking wave's after
    // the boundary, the router wave's after its router row, the gate/up
    // waves' after their gate/up rows)
    if (has_next) {
      const int pc = pred_cnt[(l + 1) & 1];
      const int32_t *Rn = pred_ref[(l + 1) & 1];
      if (upos < pc) u_load<C>(a, Rn[upos], urow0, cg, cu, sr);
    }
  }
  // the last layer's outputs: its partials are complete once every
  // workgroup has arrived
  wg_wait(counter<WS>(a, a.L - 1, CNT_D), ep * C::ITEMS_D, W_RANK, ab);
  if (wave == W_COMB) {
    const float v = __uint_as_float(__hip_atomic_load(
        reinterpret_cast<const uint32_t *>(part + ((size_t)((a.L - 1) & 1) * K + lane / ROWS_D) *
                                                      kStackMaxD + drow0 + lane % ROWS_D),
        __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT));
    red_l[lane / ROWS_D][lane % ROWS_D] = v;
    __atomic_signal_fence(__ATOMIC_SEQ_CST);
    __builtin_amdgcn_wave_barrier();
    __atomic_signal_fence(__ATOMIC_SEQ_CST);
    if (lane < ROWS_D) {
      float yv = 0.f;
      for (int w = 0; w < K; ++w) yv += red_l[w][lane];   // rank order
      KARG(y)[(size_t)(a.L - 1) * D + drow0 + lane] = (uint16_t)f32_to_bf16(yv);
    }
  }
}

}  // namespace moe

#include "stack_wide.hip"

namespace moe {

// ---------------------------------------------------------------------------
#define MOE_STACK_GEOM(D, F, K, PB, ACT, MODE, RN)                            \
  {D, F, K, PB, ACT, MODE, RN,                                               \
   (StackCfg<D, F, K, PB, ACT, MODE, RN>::ITEMS_U >                          \
            StackCfg<D, F, K, PB, ACT, MODE, RN>::ITEMS_D                    \
        ? StackCfg<D, F, K, PB, ACT, MODE, RN>::ITEMS_U                      \
        : StackCfg<D, F, K, PB, ACT, MODE, RN>::ITEMS_D),                    \
   StackWs<F, K>::kCnt,                                                      \
   reinterpret_cast<const void *>(&stack_decode_kernel<D, F, K, PB, ACT, MODE, RN>)}

// Qwen3-30B-A3B: 256 workgroups; softmax top-k with and without renorm
#define MOE_STACK_WIDE(D, F, K, PB, ACT, MODE, RN)                            \
  {D, F, K, PB, ACT, MODE, RN, WideCfg<D, F, K, PB, ACT, MODE, RN>::NWG,     \
   StackWs<F, K>::kCnt,                                                      \
   reinterpret_cast<const void *>(&stack_wide_kernel<D, F, K, PB, ACT, MODE, RN>)}

static const StackLaunch kStackTable[] = {
    MOE_STACK_GEOM(2048, 768, 8, false, MOE_ACT_SWIGLU, MOE_ROUTE_SOFTMAX_TOPK, 1),
    MOE_STACK_GEOM(2048, 768, 8, false, MOE_ACT_SWIGLU, MOE_ROUTE_SOFTMAX_TOPK, 0),
    // gpt-oss-120b: 256 workgroups (240 with gate/up rows, 180 with down rows)
    MOE_STACK_WIDE(2880, 2880, 4, true, MOE_ACT_SWIGLU_CLAMP, MOE_ROUTE_TOPK_SOFTMAX, 0),
};
constexpr int kStackKernels = sizeof(kStackTable) / sizeof(kStackTable[0]);

const StackLaunch *find_stack(int d_model, int d_ff, int k, int has_bias, int act, int mode,
                              int renorm) {
  for (const auto &e : kStackTable)
    if (e.d_model == d_model && e.d_ff == d_ff && e.k == k &&
        e.has_bias == (has_bias != 0) && e.act == act &&
        (mode < 0 || (e.mode == mode &&
                      (mode != MOE_ROUTE_SOFTMAX_TOPK || e.renorm == (renorm != 0)))))
      return &e;
  return nullptr;
}

// Every workgroup of the kernel waits for every other, so the whole grid
// must be resident at once.  The cooperative launch guarantees that.  An
// ordinary launch (the caller's choice, `ordinary`) costs ~16 us less per
// token to dispatch and places every workgroup only while no other kernel
// holds CUs of the device: it is taken when the kernel's occupancy lets one
// device hold the grid (checked once per device and kernel), else the launch
// is cooperative anyway.  The kernel's waits are bounded, so an ordinary
// launch that could not place its whole grid ends with the timeout bit in
// the device error word, never a hang.
hipError_t launch_stack(const StackLaunch *S, StackArgs &a, bool ordinary, hipStream_t s) {
  void *args[] = {&a};
  if (ordinary) {
    constexpr int kMaxDevices = 64;
    static std::atomic<int> fits[kMaxDevices][kStackKernels];   // 0 unknown, 1 yes, 2 no
    int dev = 0;
    hipError_t e = hipGetDevice(&dev);
    if (e != hipSuccess) return e;
    const int ki = (int)(S - kStackTable);
    int f = (dev >= 0 && dev < kMaxDevices) ? fits[dev][ki].load() : 2;
    if (f == 0) {
      int per_cu = 0, cus = 0;
      e = hipOccupancyMaxActiveBlocksPerMultiprocessor(&per_cu, S->func, 512, 0);
      if (e == hipSuccess)
        e = hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev);
      if (e != hipSuccess) return e;
      f = (int64_t)per_cu * cus >= S->nwg ? 1 : 2;
      fits[dev][ki].store(f);
    }
    if (f == 1) return hipLaunchKernel(S->func, dim3(S->nwg), dim3(512), args, 0, s);
  }
  return hipLaunchCooperativeKernel(S->func, dim3(S->nwg), dim3(512), args, 0, s);
}

}  // namespace moe
