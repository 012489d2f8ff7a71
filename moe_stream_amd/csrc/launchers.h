// Host-side launchers of the gfx950 kernels, shared by the C ABI layer.
#pragma once

#include "common.h"

namespace moe {

// ---- batch-1 / small-T expert block (ffn_decode.hip) ----------------------
// Small-T grouped kernels: up to this many (token, expert) pairs per call,
// member tokens of a slot staged this many at a time.
constexpr int kSmallMaxPairs = 256;
constexpr int kSmallTokensPerPass = 8;
struct FfnLaunch {
  int d_model, d_ff, has_bias;
  int up_rows_wg, up_threads;  // gate/up kernel: rows and threads per WG
  int down_rows_wg;            // down kernel: output rows per WG
  int down_small_waves;        // grouped down kernel: waves per WG
  void (*up)(dim3, dim3, hipStream_t, const PoolArgs &, const RefList &,
             const uint16_t *, int, uint16_t *, int, float, float);
  void (*down)(dim3, dim3, hipStream_t, const PoolArgs &, const RefList &,
               const float *, const uint16_t *, int, uint16_t *, float *);
  size_t (*down_lds)(int k);   // dynamic LDS bytes of the down kernel
  void (*up_small)(dim3, dim3, hipStream_t, const PoolArgs &, const int32_t *, int,
                   const uint16_t *, int, uint16_t *, int, float, float);
  void (*down_small)(dim3, dim3, size_t, hipStream_t, const PoolArgs &, const int32_t *,
                     const float *, const uint16_t *, int, int, uint16_t *, float *);
  size_t (*down_small_lds)(int P);   // dynamic LDS bytes of the grouped down kernel
};
const FfnLaunch *find_ffn(int d_model, int d_ff, int has_bias);
void launch_ffn_up(const FfnLaunch *L, const PoolArgs &pa, const RefList &refs,
                   const uint16_t *x, int T, int k, uint16_t *h, int act,
                   float alpha, float limit, hipStream_t s);
void launch_ffn_down(const FfnLaunch *L, const PoolArgs &pa,
                     const RefList &refs, const float *scores, int T, int k,
                     const uint16_t *h, uint16_t *out, float *out32,
                     hipStream_t s);
void launch_ffn_decode(const FfnLaunch *L, const PoolArgs &pa,
                       const RefList &refs, const float *scores,
                       const uint16_t *x, int T, int k, uint16_t *h,
                       uint16_t *out, float *out32, int act, float alpha,
                       float limit, hipStream_t s);

// ---- router / top-k / lookahead / slot lookup (route.hip) -----------------
constexpr int kRouteMaxE = 128;
constexpr int kRouteMaxT = 16;
constexpr uint32_t kRouteSpinLimit = 1u << 20;   // polls before a router wait gives up
// the router workspace's arrival word (32-bit index from the sequence word:
// its own 128-byte line inside the 256-byte header); zero between launches
constexpr int kRouteArrivedWord = 32;

struct RouteArgs {
  const uint16_t *x;
  const uint16_t *W;
  const uint16_t *bias;
  const uint16_t *Wn;
  const uint16_t *bias_n;
  int32_t *ids;
  float *scores;
  int32_t *pred;
  const int32_t *table;
  int32_t *slot_refs;
  int32_t *miss_count;
  float *logits;      // [2][T][E] fp32 workspace (many tokens)
  uint64_t *flagged;  // [2][T][E] (flag << 32 | fp32 logit) workspace (T <= kRouteMaxT)
  uint32_t *counter;  // workspace word: the last launch's flag (T <= kRouteMaxT)
  int T, D, E, mode, renorm, k, kp;
};
void launch_route(const RouteArgs &a, hipStream_t s);

// ---- multi-token grouped MFMA expert block (grouped.hip) ------------------
constexpr int kGroupMaxKeys = 16256;    // n_slots + n_records: LDS histogram <= 64 KiB
constexpr int kGroupedMaxWGs = 2048;    // grid cap; workgroups loop over items
struct GroupedLaunch {
  int d_model, d_ff, has_bias;
  int nb_up, nb_down;   // output features per work item of gate/up and of down
  // (with nb_up a multiple of 64 gate/up writes h in the down kernel's input
  // order with its 64-input row sums, else h as it is)
  void (*gate_up)(dim3, hipStream_t, const PoolArgs &, const uint16_t *, const float *, int,
                  const int32_t *, const int4 *, const int32_t *, uint16_t *, float *, int,
                  float, float);
  void (*down)(dim3, hipStream_t, const PoolArgs &, const uint16_t *, const float *,
               const float *, const int32_t *, const int4 *, const int32_t *, float *);
};
struct GroupedWs {
  int64_t max_tiles;
  size_t off_perm, off_tiles, off_ntiles, off_h, off_yp, off_xq, off_rsx, off_hq, off_rsh, total;
};
const GroupedLaunch *find_grouped(int d_model, int d_ff, int has_bias);
GroupedWs grouped_ws(int64_t T, int k, int D, int F);
void launch_grouped(const GroupedLaunch *G, const PoolArgs &pa, const int32_t *refs,
                    const float *scores, const uint16_t *x, int T, int k, uint16_t *out,
                    float *out32, char *ws, int act, float alpha, float limit,
                    hipStream_t s);

// ---- whole-token persistent decode (stack_decode.hip) ---------------------
struct StackArgs;
struct StackLaunch {
  int d_model, d_ff, k, has_bias, act, mode, renorm, nwg;
  size_t ws_fixed;   // workspace bytes before the per-layer counters
  const void *func;
};
constexpr size_t kStackCounterBytesPerLayer = 8 * 32 * 4;   // kSub lines of 32 words
const StackLaunch *find_stack(int d_model, int d_ff, int k, int has_bias, int act, int mode,
                              int renorm);
hipError_t launch_stack(const StackLaunch *S, StackArgs &a, bool ordinary, hipStream_t s);
void launch_slot_lookup(const int32_t *table, int E, const int32_t *ids, int n,
                        int32_t *refs, int32_t *miss_count, hipStream_t s);

}  // namespace moe
