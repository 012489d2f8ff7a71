// Whole-token decode in ONE launch for wide experts (gpt-oss-120b: hidden =
// expert intermediate = 2880, top-4, projection biases, clamped SwiGLU,
// top-k-then-softmax routing).
//
// The launch, the workspace, the exchanges and the routing are those of
// stack_decode_kernel (one workgroup per CU, all resident; router logits and
// expert activations cross workgroups as flagged 8-byte entries; the layer
// boundary is a counter; bounded waits).  What differs is where a layer's
// 55 MB of expert rows wait for their turn, so that HBM streams while the
// chain of dependent steps runs:
//
//   gate/up  240 workgroups x 48 rows of the expert PREDICTED at the
//            workgroup's position w % K (60 workgroups per position), held
//            in the registers of waves 0-3 (one per SIMD, 12 rows each); the
//            next layer's are loaded as soon as this layer's gate/up is done
//   down     240 workgroups x 48 output rows of the expert at their position
//            w % K (60 workgroups per position, 12 rows per down wave),
//            staged in LDS (84 KiB of codes and scales) by direct-to-LDS
//            loads of waves 4-7 once the routing is known
//   router   wave 6: one router row (+ the lookahead row), then the
//            lookahead ranking of layer l+1
//   routing  wave 7: the layer boundary, x staged in LDS, the ranking of
//            the routed experts, which position holds which rank
//   fix-up   a routed expert that was not predicted takes the position of a
//            predicted expert that was not routed: its gate/up rows are
//            spread over the whole grid (two rows per gate/up wave and task,
//            straight from the pool) and its down rows are staged by that
//            position's down waves once the routing is known
//   D        the four gate/up waves collect a quarter each of the
//            activations of the workgroup's position into LDS (they have no
//            loads in flight, so their polls return at once); waves 4-7 run
//            16 down rows each and publish the score-weighted rows as
//            flagged per-rank entries; wave 7 arrives
//   combine  wave 5 of the next layer (idle until the routing) sums the
//            previous layer's per-rank rows in rank order and stores them
//            (the last layer's after the kernel's final boundary)
//
// Every row is summed over the lanes and in the order of ffn_decode's
// gpt-oss instantiation (gate/up: 32 lanes per row; down: 16 lanes per row)
// and the combine runs in rank order, so the outputs are bit-identical to
// route_kernel + ffn_decode per layer.  Each workgroup polls the activations
// of one expert (11.5 KB), not of all K.
//
// Semantics per layer: top_k_route (engine_120b.py:65-70), top_k_indices
// (engine_120b.py:73-75), the gpt-oss expert block with projection biases
// and the clamped SwiGLU (engine_120b.py:132-145).

namespace moe {

template <int D, int F, int K, bool PBIAS, int ACT, int MODE, int RENORM>
struct WideCfg {
  static constexpr int D_ = D, F_ = F, K_ = K, ACT_ = ACT, MODE_ = MODE, RENORM_ = RENORM;
  static constexpr bool PBIAS_ = PBIAS;
  using Layout = PackedLayout<D, F, PBIAS>;
  static constexpr int NT = 512, NWG = 256;
  // gate/up: 32 lanes per row, 2 rows per wave step, 4 waves x 6 steps
  static constexpr int U = D / 32, NG = D / 64;
  static constexpr int SGU = 32, CPLU = (U + SGU - 1) / SGU, RPSU = 64 / SGU;
  static constexpr int WAVES_U = 4, RSTEPS_U = 6, ROWS_U = WAVES_U * RSTEPS_U * RPSU;
  static constexpr int NPOS = F / ROWS_U;              // workgroups per position
  static constexpr int ITEMS_U = K * NPOS;
  static constexpr int SB_U4 = ROWS_U * NG * 2 / 16;   // 16-byte pieces per scale array
  static constexpr int SUI_ALL = (4 * SB_U4 + 63) / 64;  // scale loads (1 KiB each)
  static constexpr int SUI = (SUI_ALL + WAVES_U - 1) / WAVES_U;   // per gate/up wave
  // down: 16 lanes per row, 4 rows per step, 3 steps per wave (12 rows), 4
  // waves per workgroup: 48 rows, so the K positions' rows take 240
  // workgroups (as gate/up does) instead of 180 at 16 rows per wave
  static constexpr int UF = F / 32, NGF = F / 64;
  static constexpr int SGD = 16, CPLD = (UF + SGD - 1) / SGD, RPSD = 64 / SGD;
  static constexpr int RSTEPS_D = 3, ROWS_D = RSTEPS_D * RPSD;   // rows per down wave
  static constexpr int WAVES_D = 4, ROWS_DWG = WAVES_D * ROWS_D;   // rows per workgroup
  static constexpr int ITEMS_D = K * (D / ROWS_DWG);               // down workgroups
  static constexpr int CROWS = D / ITEMS_D;                         // combined rows per workgroup
  // a down wave's scales (ROWS_D * NGF halfwords per array) start 8-byte
  // aligned: its image is the 16-byte pieces from the aligned address below,
  // one piece more than the rows need (the halfword offset DOFF(row0) skips
  // the lead-in)
  static constexpr int SBD_U4 = (ROWS_D * NGF * 2 + 8 + 15) / 16;
  static constexpr int DCI = RSTEPS_D * CPLD;          // code loads per position (1 KiB each)
  static constexpr int DSI = (2 * SBD_U4 + 63) / 64;   // scale loads per position
  static constexpr int NP = PBIAS ? 4 : 3;
  static constexpr int XU4 = D / 8, HU4 = F / 8;
  static constexpr int HPL = (HU4 + 63) / 64;          // activation pieces per lane
  static constexpr int HPW = (HU4 / WAVES_U + 3) / 4 * 4;   // ... per gate/up wave (whole chunks)
  static constexpr int HPWL = (HPW + 63) / 64;              // ... per lane of it
  static constexpr int XPL = (XU4 + 63) / 64;          // x pieces per lane (one wave)
  static_assert(F % ROWS_U == 0 && D % ROWS_DWG == 0 && D % ITEMS_D == 0, "row blocks");
  static_assert(K * CROWS <= 64 && WAVES_U * HPW >= HU4, "combine lanes, activation quarters");
  static_assert(ITEMS_U <= NWG && ITEMS_D <= NWG, "one item per workgroup");
  static_assert((ROWS_U * NG * 2) % 16 == 0 && (ROWS_D * NGF * 2) % 8 == 0, "scale pieces");
  // the last wave's image ends inside the scale array
  static_assert((((D - ROWS_D) * NGF * 2) & ~15) + SBD_U4 * 16 <= D * NGF * 2, "scale image");
  // halfword offset of row row0's scales in its wave's image
  static __device__ __forceinline__ int doff(int row0) { return (row0 * NGF) & 7; }
  static_assert(K == 4 && WAVES_U == 4 && NT / 64 == 8,
                "a down wave per position beside each gate/up wave; two positions per staging wave");
};

template <class C>
__device__ __forceinline__ float wide_act(float g, float u) {
  if (C::ACT_ == MOE_ACT_SWIGLU) return apply_act(MOE_ACT_SWIGLU, g, u, 0.f, 0.f);
  return apply_act(MOE_ACT_SWIGLU_CLAMP, g, u, KARG(alpha), KARG(limit));
}

typedef __attribute__((address_space(3))) void wide_lds_void;

// chunk_dot_lds with the chunk's 4 activation pieces already in registers
// (the same products in the same order).
__device__ __forceinline__ float chunk_dot_regs(const uint4 &c, const uint4 (&xa)[4]) {
  float acc = 0.f;
  const uint32_t w[4] = {c.x, c.y, c.z, c.w};
#pragma unroll
  for (int q = 0; q < 4; ++q) {
    const uint32_t xv[4] = {xa[q].x, xa[q].y, xa[q].z, xa[q].w};
    uint32_t p[4];
    codes_to_bf16x2(w[q], p);
#pragma unroll
    for (int m = 0; m < 4; ++m) acc = dot2_bf16(p[m], xv[m], acc);
  }
  return acc;
}

// One whole wave: 16 bytes per lane from `g` (the lane's own address) into
// LDS at `lds` + 16 * lane, through no registers (the load completes in
// order with this wave's other loads).
__device__ __forceinline__ void dma16(const void *g, void *lds) {
  __builtin_amdgcn_global_load_lds(g, (wide_lds_void *)lds, 16, 0, 0);
}

// One whole wave: the F activations of one expert (its F/2 flagged entries
// at hf) as HPL 16-byte pieces per lane (piece lane + 64 i, 8 bf16 each),
// polled until every entry carries `fl`.  Bounded.
template <int HU4, int HPL>
__device__ __forceinline__ void get_acts_wide(int tid, const uint64_t *hf, uint32_t fl,
                                              const Abort &ab, uint4 (&p)[HPL]) {
  const int lane = tid & 63;
  uint32_t spins = 0;
  // a piece whose 4 entries all carried the flag is kept and not read again:
  // later rounds read only what was missing (every workgroup re-reading all
  // of its pieces per round loads the path the polls share)
  static_assert(HPL <= 32, "one bit per piece");
  uint32_t got = 0;   // bit i: piece i complete
  while (true) {
    bool ok = true;
#pragma unroll
    for (int i = 0; i < HPL; ++i) {
      if ((got >> i) & 1u) continue;
      const uint64_t *e = hf + 4 * min(lane + 64 * i, HU4 - 1);
      uint64_t v[4];
#pragma unroll
      for (int q = 0; q < 4; ++q)
        v[q] = __hip_atomic_load(e + q, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
      bool ok_i = true;
#pragma unroll
      for (int q = 0; q < 4; ++q) ok_i = ok_i && (uint32_t)(v[q] >> 32) == fl;
      p[i] = make_uint4((uint32_t)v[0], (uint32_t)v[1], (uint32_t)v[2], (uint32_t)v[3]);
      got |= (uint32_t)ok_i << i;
      ok = ok && ok_i;
    }
    if (__ballot(!ok) == 0) break;
    if (ab.gave_up(++spins)) break;
    __builtin_amdgcn_s_sleep(1);
  }
}

// As get_acts_wide for NE experts at once (their pieces polled together,
// so one round trip covers all of them).
template <int HU4, int HPL, int NE>
__device__ __forceinline__ void get_acts_multi(int tid, const uint64_t *const (&hf)[NE],
                                               uint32_t fl, const Abort &ab,
                                               uint4 (&p)[NE][HPL]) {
  const int lane = tid & 63;
  uint32_t spins = 0;
  while (true) {
    bool ok = true;
#pragma unroll
    for (int n = 0; n < NE; ++n) {
#pragma unroll
      for (int i = 0; i < HPL; ++i) {
        const uint64_t *e = hf[n] + 4 * min(lane + 64 * i, HU4 - 1);
        uint64_t v[4];
#pragma unroll
        for (int q = 0; q < 4; ++q)
          v[q] = __hip_atomic_load(e + q, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
#pragma unroll
        for (int q = 0; q < 4; ++q) ok = ok && (uint32_t)(v[q] >> 32) == fl;
        p[n][i] = make_uint4((uint32_t)v[0], (uint32_t)v[1], (uint32_t)v[2], (uint32_t)v[3]);
      }
    }
    if (__ballot(!ok) == 0) break;
    if (ab.gave_up(++spins)) break;
    __builtin_amdgcn_s_sleep(1);
  }
}

// One whole wave: pieces [HPW * w, HPW * w + HPW) of one expert's F
// activations (its F/2 flagged entries at hf; lane i takes pieces
// HPW * w + i + 64 j, j < HPWL), polled until every one of them carries `fl`.
// Lanes past the quarter re-read a clamped piece and do not wait on it; a
// piece that arrived is not read again.  Bounded.
template <int HU4, int HPW, int HPWL>
__device__ __forceinline__ void get_acts_quarter(int tid, const uint64_t *hf, int w, uint32_t fl,
                                                 const Abort &ab, uint4 (&p)[HPWL]) {
  const int lane = tid & 63;
  uint32_t spins = 0;
  uint32_t got = 0;   // bit j: piece j of this lane complete (or not this lane's)
#pragma unroll
  for (int j = 0; j < HPWL; ++j) {
    const int k = lane + 64 * j;
    if (k >= HPW || HPW * w + k >= HU4) got |= 1u << j;
  }
  while (true) {
#pragma unroll
    for (int j = 0; j < HPWL; ++j) {
      if ((got >> j) & 1u) continue;
      const uint64_t *e = hf + 4 * min(HPW * w + lane + 64 * j, HU4 - 1);
      uint64_t v[4];
#pragma unroll
      for (int q = 0; q < 4; ++q)
        v[q] = __hip_atomic_load(e + q, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
      bool ok = true;
#pragma unroll
      for (int q = 0; q < 4; ++q) ok = ok && (uint32_t)(v[q] >> 32) == fl;
      p[j] = make_uint4((uint32_t)v[0], (uint32_t)v[1], (uint32_t)v[2], (uint32_t)v[3]);
      got |= (uint32_t)ok << j;
    }
    if (__ballot(got != (1u << HPWL) - 1u) == 0) break;
    if (ab.gave_up(++spins)) break;
    __builtin_amdgcn_s_sleep(1);
  }
}

// The lane index, made opaque at each use: what is derived from it (LDS and
// global addresses, lane-0 masks) is computed where it is used instead of
// being held in registers across the layer loop (this kernel runs at the
// register limit, and values held that way are spilled to scratch).
__device__ __forceinline__ int wide_lane() {
  int t = threadIdx.x;
  asm volatile("" : "+v"(t));
  return t & 63;
}

// One whole wave (lane = rank * CROWS + row): the layer's combined output
// rows [crow0, crow0 + CROWS) from the K per-rank flagged entries of `part`
// (polled until each carries `fl`), summed in rank order through `red`.
template <int K, int CROWS>
__device__ __forceinline__ void wide_combine(const uint64_t *part, int crow0, uint32_t fl,
                                             const Abort &ab, float (*red)[CROWS],
                                             uint16_t *y) {
  const int lane = wide_lane();
  const int r = min(lane / CROWS, K - 1), i = lane % CROWS;
  const bool mine = lane < K * CROWS;
  const uint64_t *e = part + (size_t)r * kStackMaxD + crow0 + i;
  uint64_t v = __hip_atomic_load(e, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  uint32_t spins = 0;
  while (__ballot(mine && (uint32_t)(v >> 32) != fl) != 0) {
    if (ab.gave_up(++spins)) break;
    __builtin_amdgcn_s_sleep(1);
    v = __hip_atomic_load(e, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  }
  if (mine) red[r][i] = __uint_as_float((uint32_t)v);
  __atomic_signal_fence(__ATOMIC_SEQ_CST);
  __builtin_amdgcn_wave_barrier();
  __atomic_signal_fence(__ATOMIC_SEQ_CST);
  if (lane < CROWS) {
    float yv = 0.f;
    for (int w = 0; w < K; ++w) yv += red[w][lane];   // rank order
    y[crow0 + lane] = (uint16_t)f32_to_bf16(yv);
  }
}

// One whole wave: wait until the LDS word `w` holds `fl` (set by another
// wave of the workgroup, which always sets it).
__device__ __forceinline__ void lds_wait_flag(const uint32_t *w, uint32_t fl) {
  if (wide_lane() == 0) {
    while (__hip_atomic_load(w, __ATOMIC_ACQUIRE, __HIP_MEMORY_SCOPE_WORKGROUP) != fl)
      __builtin_amdgcn_s_sleep(1);
  }
  __builtin_amdgcn_wave_barrier();
  __atomic_signal_fence(__ATOMIC_SEQ_CST);
}
__device__ __forceinline__ void lds_set_flag(uint32_t *w, uint32_t fl) {
  __atomic_signal_fence(__ATOMIC_SEQ_CST);
  if (wide_lane() == 0) __hip_atomic_store(w, fl, __ATOMIC_RELEASE, __HIP_MEMORY_SCOPE_WORKGROUP);
}

// Gate/up rows of expert `ref` for this workgroup's 48-row block, per wave
// (4 waves: 6 steps of 2 rows each).  load: the codes into registers and,
// by direct-to-LDS loads, the block's four scale arrays (gate S, gate B, up
// S, up B) into sbu and its gate and up projection biases into ubias, spread
// over the 4 waves; the caller waits for every wave's loads before run.
// run: the rows, with x in act_l/asum_l, each step's 2 activations published
// as one flagged entry at hf + row / 2.
template <class C>
struct WideU {
  uint4 cg[C::RSTEPS_U][C::CPLU], cu[C::RSTEPS_U][C::CPLU];
  bool ok;
  __device__ __forceinline__ void load(int tid, const StackArgs &a, int32_t ref, int row0,
                                       uint4 *sbu, uint32_t *ubias) {
    constexpr int D = C::D_, NG = C::NG, SGU = C::SGU, CPLU = C::CPLU, RPSU = C::RPSU;
    constexpr int U = C::U, NP = C::NP, SB_U4 = C::SB_U4, ROWS_U = C::ROWS_U;
    const int lane = tid & 63, wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int uj = lane % SGU, usub = lane / SGU;
    ref = __builtin_amdgcn_readfirstlane(ref);
    // No branch around any load (an out-of-range ref reads slot 0 and clears
    // ok; surplus lanes read a clamped index), so nothing waits for them here.
    const char *gw = resolve_packed_safe<typename C::Layout>(a.pa, comp_index(PROJ_GATE, PART_W, NP), ref, ok);
    const char *uw = resolve_packed_safe<typename C::Layout>(a.pa, comp_index(PROJ_UP, PART_W, NP), ref, ok);
    const char *sb[4] = {resolve_packed_safe<typename C::Layout>(a.pa, comp_index(PROJ_GATE, PART_S, NP), ref, ok),
                         resolve_packed_safe<typename C::Layout>(a.pa, comp_index(PROJ_GATE, PART_B, NP), ref, ok),
                         resolve_packed_safe<typename C::Layout>(a.pa, comp_index(PROJ_UP, PART_S, NP), ref, ok),
                         resolve_packed_safe<typename C::Layout>(a.pa, comp_index(PROJ_UP, PART_B, NP), ref, ok)};
    // scale pieces: load j (1 KiB) on wave j % 4
#pragma unroll
    for (int it = 0; it < C::SUI; ++it) {
      const int j = it * C::WAVES_U + wave;
      if (j < C::SUI_ALL) {
        const int i = min(j * 64 + lane, 4 * SB_U4 - 1);
        const int p = i / SB_U4, o = i % SB_U4;
        const char *sp = p == 0 ? sb[0] : p == 1 ? sb[1] : p == 2 ? sb[2] : sb[3];
        dma16(reinterpret_cast<const uint4 *>(sp + (int64_t)row0 * NG * 2) + o, sbu + j * 64);
      }
    }
    if (C::PBIAS_ && wave == 0) {
      // 4 bytes per lane: lanes 0..23 the gate biases of the 48 rows, lanes
      // 24..47 the up biases, the rest a clamped copy
      bool okb;
      const char *gbias = resolve_packed_safe<typename C::Layout>(a.pa, comp_index(PROJ_GATE, PART_BIAS, NP), ref, okb);
      const char *ubias_g = resolve_packed_safe<typename C::Layout>(a.pa, comp_index(PROJ_UP, PART_BIAS, NP), ref, okb);
      constexpr int W = ROWS_U / 2;   // 4-byte words per bias block
      const int w = min(lane, 2 * W - 1);
      const char *src = (w < W ? gbias : ubias_g) + (int64_t)row0 * 2 + (w % W) * 4;
      __builtin_amdgcn_global_load_lds(src, (wide_lds_void *)ubias, 4, 0, 0);
    }
    issue_order_fence();
    // uniform base + 32-bit lane offset: the loads take the base in scalar
    // registers (one VGPR of offset per load instead of a 64-bit address)
#pragma unroll
    for (int st = 0; st < C::RSTEPS_U; ++st) {
      const int row = row0 + (wave * C::RSTEPS_U + st) * RPSU + usub;
#pragma unroll
      for (int i = 0; i < CPLU; ++i) {   // surplus chunks (c >= U) re-read the last one, unused
        const uint32_t off = (uint32_t)(row * (D / 2) + min(i * SGU + uj, U - 1) * 16);
        cg[st][i] = load_stream16(reinterpret_cast<const uint4 *>(gw + off));
        cu[st][i] = load_stream16(reinterpret_cast<const uint4 *>(uw + off));
      }
    }
    issue_order_fence();
  }
  // No value for the registers (where no load follows, so that the last
  // expert's codes are not kept alive, in registers, through the layer).
  __device__ __forceinline__ void forget() {
#pragma unroll
    for (int st = 0; st < C::RSTEPS_U; ++st) {
#pragma unroll
      for (int i = 0; i < C::CPLU; ++i) {
        cg[st][i].x = __builtin_nondeterministic_value(cg[st][i].x);
        cg[st][i].y = __builtin_nondeterministic_value(cg[st][i].y);
        cg[st][i].z = __builtin_nondeterministic_value(cg[st][i].z);
        cg[st][i].w = __builtin_nondeterministic_value(cg[st][i].w);
        cu[st][i].x = __builtin_nondeterministic_value(cu[st][i].x);
        cu[st][i].y = __builtin_nondeterministic_value(cu[st][i].y);
        cu[st][i].z = __builtin_nondeterministic_value(cu[st][i].z);
        cu[st][i].w = __builtin_nondeterministic_value(cu[st][i].w);
      }
    }
  }
  // the rows from the loaded registers; `sbh`: the block's scales in LDS,
  // `bh`: its gate biases then up biases (bf16).  Chunk-outer: a chunk's
  // activations are read from LDS once for all 6 steps (each row still sums
  // its chunks in ascending order).
  __device__ __forceinline__ void run(int tid, const uint4 *act_l, const float *asum_l,
                                      const uint16_t *sbh, const uint16_t *bh, uint64_t *hf,
                                      int row0, uint32_t fl) const {
    constexpr int U = C::U, NG = C::NG, SGU = C::SGU, CPLU = C::CPLU, RPSU = C::RPSU;
    constexpr int SBN = C::SB_U4 * 8, ROWS_U = C::ROWS_U, RS = C::RSTEPS_U;
    const int lane = tid & 63, wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int uj = lane % SGU, usub = lane / SGU;
    const int rl0 = wave * RS * RPSU + usub;   // row of step st: rl0 + st * RPSU
    float pg[RS], pu[RS];
#pragma unroll
    for (int st = 0; st < RS; ++st) pg[st] = pu[st] = 0.f;
#pragma unroll
    for (int i = 0; i < CPLU; ++i) {
      const int c = i * SGU + uj;
      if (CPLU * SGU == U || c < U) {
        uint4 xa[4];
#pragma unroll
        for (int q = 0; q < 4; ++q) xa[q] = act_l[q * U + c];
        const float xs = asum_l[c];
#pragma unroll
        for (int st = 0; st < RS; ++st) {
          const int g = (rl0 + st * RPSU) * NG + (c >> 1);
          const float Sg = bf16_to_f32(sbh[0 * SBN + g]), Bg = bf16_to_f32(sbh[1 * SBN + g]);
          const float Su = bf16_to_f32(sbh[2 * SBN + g]), Bu = bf16_to_f32(sbh[3 * SBN + g]);
          pg[st] += Sg * chunk_dot_regs(cg[st][i], xa) + (Bg - 128.f * Sg) * xs;
          pu[st] += Su * chunk_dot_regs(cu[st][i], xa) + (Bu - 128.f * Su) * xs;
        }
      }
    }
#pragma unroll
    for (int st = 0; st < RS; ++st) {
      const int rl = rl0 + st * RPSU;
      float g = group_sum<SGU>(pg[st]);
      float u = group_sum<SGU>(pu[st]);
      if (C::PBIAS_) {
        g += bf16_to_f32(bh[rl]);
        u += bf16_to_f32(bh[ROWS_U + rl]);
      }
      uint32_t hb = 0;
      if (ok) hb = f32_to_bf16(wide_act<C>(g, u));
      else if (lane == 0) flag_error();
      // rows rl (lanes 0-31) and rl + 1 (lanes 32-63) as one flagged entry
      static_assert(RPSU == 2, "two rows per wave step");
      const uint32_t h0 = __builtin_amdgcn_readlane(hb, 0), h1 = __builtin_amdgcn_readlane(hb, 32);
      if (lane == 0)
        __hip_atomic_store(hf + (row0 + rl) / 2, (uint64_t)(h0 | (h1 << 16)) | ((uint64_t)fl << 32),
                           __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    }
  }
};

// One whole wave: fix-up task t of expert `ref`, i.e. its gate/up rows 2t
// (lanes 0-31) and 2t + 1 (lanes 32-63) straight from the pool, published as
// the flagged entry hf[t].  The lane partition, the chunk order and the
// arithmetic are WideU::run's for one step, so a row computed here is
// bit-identical to the same row computed by its position's workgroup.
template <class C>
struct WideFix {   // one fix-up task's operands in registers
  uint32_t sv[4][C::CPLU];
  uint4 cg[C::CPLU], cu[C::CPLU];
  float gbv, ubv;
  bool ok;
};

// The loads of task t (every load unconditional: surplus chunks re-read the
// last one, unused).
template <class C>
__device__ __forceinline__ void wide_fix_load(int lane, const StackArgs &a, int32_t ref, int t,
                                              WideFix<C> &o) {
  constexpr int D = C::D_, U = C::U, NG = C::NG, SGU = C::SGU, CPLU = C::CPLU, NP = C::NP;
  using Lay = typename C::Layout;
  const int uj = lane % SGU, usub = lane / SGU;
  const int row = 2 * t + usub;
  ref = __builtin_amdgcn_readfirstlane(ref);
  bool ok = true;
  const char *gw = resolve_packed_safe<Lay>(a.pa, comp_index(PROJ_GATE, PART_W, NP), ref, ok);
  const char *uw = resolve_packed_safe<Lay>(a.pa, comp_index(PROJ_UP, PART_W, NP), ref, ok);
  const uint16_t *sp[4] = {
      reinterpret_cast<const uint16_t *>(resolve_packed_safe<Lay>(a.pa, comp_index(PROJ_GATE, PART_S, NP), ref, ok)),
      reinterpret_cast<const uint16_t *>(resolve_packed_safe<Lay>(a.pa, comp_index(PROJ_GATE, PART_B, NP), ref, ok)),
      reinterpret_cast<const uint16_t *>(resolve_packed_safe<Lay>(a.pa, comp_index(PROJ_UP, PART_S, NP), ref, ok)),
      reinterpret_cast<const uint16_t *>(resolve_packed_safe<Lay>(a.pa, comp_index(PROJ_UP, PART_B, NP), ref, ok))};
#pragma unroll
  for (int i = 0; i < CPLU; ++i) {
    const int g = row * NG + (min(i * SGU + uj, U - 1) >> 1);
#pragma unroll
    for (int j = 0; j < 4; ++j) o.sv[j][i] = sp[j][g];
  }
  o.gbv = 0.f;
  o.ubv = 0.f;
  if (C::PBIAS_) {
    bool okb;
    o.gbv = bf16_to_f32(reinterpret_cast<const uint16_t *>(
        resolve_packed_safe<Lay>(a.pa, comp_index(PROJ_GATE, PART_BIAS, NP), ref, okb))[row]);
    o.ubv = bf16_to_f32(reinterpret_cast<const uint16_t *>(
        resolve_packed_safe<Lay>(a.pa, comp_index(PROJ_UP, PART_BIAS, NP), ref, okb))[row]);
  }
#pragma unroll
  for (int i = 0; i < CPLU; ++i) {
    const uint32_t off = (uint32_t)(row * (D / 2) + min(i * SGU + uj, U - 1) * 16);
    o.cg[i] = load_stream16(reinterpret_cast<const uint4 *>(gw + off));
    o.cu[i] = load_stream16(reinterpret_cast<const uint4 *>(uw + off));
  }
  o.ok = ok;
}

// Gate/up rows 2t, 2t+1 of a fix-up expert from its loaded operands, with the
// lane partition and summation order of WideU::run; published as one flagged
// entry of the expert's activations.
template <class C>
__device__ __forceinline__ void wide_fix_compute(int lane, int t, const WideFix<C> &o,
                                                 const uint4 *act_l, const float *asum_l,
                                                 uint64_t *hf, uint32_t fl) {
  constexpr int U = C::U, SGU = C::SGU, CPLU = C::CPLU;
  const int uj = lane % SGU;
  float pg = 0.f, pu = 0.f;
#pragma unroll
  for (int i = 0; i < CPLU; ++i) {
    const int c = i * SGU + uj;
    if (CPLU * SGU == U || c < U) {
      uint4 xa[4];
#pragma unroll
      for (int q = 0; q < 4; ++q) xa[q] = act_l[q * U + c];
      const float xs = asum_l[c];
      const float Sg = bf16_to_f32(o.sv[0][i]), Bg = bf16_to_f32(o.sv[1][i]);
      const float Su = bf16_to_f32(o.sv[2][i]), Bu = bf16_to_f32(o.sv[3][i]);
      pg += Sg * chunk_dot_regs(o.cg[i], xa) + (Bg - 128.f * Sg) * xs;
      pu += Su * chunk_dot_regs(o.cu[i], xa) + (Bu - 128.f * Su) * xs;
    }
  }
  float g = group_sum<SGU>(pg);
  float u = group_sum<SGU>(pu);
  if (C::PBIAS_) {
    g += o.gbv;
    u += o.ubv;
  }
  uint32_t hb = 0;
  if (o.ok) hb = f32_to_bf16(wide_act<C>(g, u));
  else if (lane == 0) flag_error();
  static_assert(C::RPSU == 2, "two rows per task");
  const uint32_t h0 = __builtin_amdgcn_readlane(hb, 0), h1 = __builtin_amdgcn_readlane(hb, 32);
  if (lane == 0)
    __hip_atomic_store(hf + t, (uint64_t)(h0 | (h1 << 16)) | ((uint64_t)fl << 32),
                       __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

// One whole wave: the down rows of expert `ref` for one down wave's 12-row
// block into the LDS image of one position by direct-to-LDS loads: codes as
// [step][chunk][lane] (the lane's 16 bytes of row step * 4 + lane / 16),
// then the scale and bias arrays' pieces (S | B).
template <class C>
__device__ __forceinline__ void wide_d_stage(int lane, const StackArgs &a, int32_t ref, int drow0,
                                             uint4 (*code)[64], uint4 (*sc)[64]) {
  constexpr int F = C::F_, NGF = C::NGF, SGD = C::SGD, CPLD = C::CPLD, UF = C::UF;
  constexpr int SBD_U4 = C::SBD_U4, NP = C::NP, RPSD = C::RPSD;
  const int dj = lane % SGD, dsub = lane / SGD;
  ref = __builtin_amdgcn_readfirstlane(ref);
  bool ok;
  const char *dw = resolve_packed_safe<typename C::Layout>(a.pa, comp_index(PROJ_DOWN, PART_W, NP), ref, ok);
  const char *ds = resolve_packed_safe<typename C::Layout>(a.pa, comp_index(PROJ_DOWN, PART_S, NP), ref, ok);
  const char *db = resolve_packed_safe<typename C::Layout>(a.pa, comp_index(PROJ_DOWN, PART_B, NP), ref, ok);
  const int64_t sb0 = ((int64_t)drow0 * NGF * 2) & ~(int64_t)15;   // 16-byte aligned
#pragma unroll
  for (int it = 0; it < C::DSI; ++it) {
    const int i = min(it * 64 + lane, 2 * SBD_U4 - 1);
    const int p = i / SBD_U4, o = i % SBD_U4;
    dma16(reinterpret_cast<const uint4 *>((p ? db : ds) + sb0) + o, &sc[it][0]);
  }
#pragma unroll
  for (int st = 0; st < C::RSTEPS_D; ++st) {
#pragma unroll
    for (int i = 0; i < CPLD; ++i) {
      const uint32_t off =
          (uint32_t)((drow0 + st * RPSD + dsub) * (F / 2) + min(i * SGD + dj, UF - 1) * 16);
      dma16(dw + off, &code[st * CPLD + i][0]);
    }
  }
}

// One wave: an arrival on a monotonic LDS counter, after this wave's LDS
// accesses before it.
__device__ __forceinline__ void lds_arrive(uint32_t *c) {
  __atomic_signal_fence(__ATOMIC_SEQ_CST);
  if (wide_lane() == 0)
    __hip_atomic_fetch_add(c, 1u, __ATOMIC_RELEASE, __HIP_MEMORY_SCOPE_WORKGROUP);
}
// One wave: wait until the monotonic LDS counter reaches `target` (its
// arrivals are made by waves that always make them).
__device__ __forceinline__ void lds_wait_count(const uint32_t *c, uint32_t target) {
  if (wide_lane() == 0) {
    while ((int32_t)(__hip_atomic_load(c, __ATOMIC_ACQUIRE, __HIP_MEMORY_SCOPE_WORKGROUP) -
                     target) < 0)
      __builtin_amdgcn_s_sleep(1);
  }
  __builtin_amdgcn_wave_barrier();
  __atomic_signal_fence(__ATOMIC_SEQ_CST);
}

// The down rows of position p for one down wave's 12-row block (rows
// row0...), from the LDS images (codes and scales staged by direct-to-LDS
// loads, activations and biases staged by the polling waves), chunk-outer: a
// chunk's activations are read once for the 3 steps, and each row still sums its
// chunks in ascending order.  Writes the score-weighted rows to red.
template <class C>
__device__ __forceinline__ void wide_down_rows(int lane, const StackArgs &a, int32_t dref,
                                               int row0, float sc, const uint4 (*code)[64],
                                               const uint16_t *sbh, const uint4 *hact,
                                               const float *hsum, const float *dbias,
                                               float *red) {
  constexpr int UF = C::UF, NGF = C::NGF, SGD = C::SGD, CPLD = C::CPLD, RPSD = C::RPSD;
  constexpr int SBN = C::SBD_U4 * 8, RS = C::RSTEPS_D, NP = C::NP;
  bool dok;
  resolve_packed_safe<typename C::Layout>(a.pa, comp_index(PROJ_DOWN, PART_W, NP), dref, dok);
  const int dj = lane % SGD, dsub = lane / SGD;
  float pv[RS];
#pragma unroll
  for (int st = 0; st < RS; ++st) pv[st] = 0.f;
  // A software pipeline over the (chunk, row) steps: the code word and the
  // scales of step n + 1 are read while step n computes, and the next
  // chunk's activations during the chunk's last row, so the LDS latency
  // hides behind a row of arithmetic instead of a wait before every row.
  // Lanes past the last chunk read a clamped (valid) chunk and add nothing.
  uint4 xa[2][4], cd[2];
  uint32_t sv[2], bv[2];
  float xs[2];
  auto fetch_x = [&](int i, int b) {
    const int c = min(i * SGD + dj, UF - 1);
#pragma unroll
    for (int q = 0; q < 4; ++q) xa[b][q] = hact[q * UF + c];
    xs[b] = hsum[c];
  };
  auto fetch_row = [&](int i, int st, int b) {
    const int c = min(i * SGD + dj, UF - 1);
    const int g = C::doff(row0) + (st * RPSD + dsub) * NGF + (c >> 1);
    cd[b] = code[st * CPLD + i][lane];
    sv[b] = sbh[g];
    bv[b] = sbh[SBN + g];
  };
  fetch_x(0, 0);
  fetch_row(0, 0, 0);
#pragma unroll
  for (int i = 0; i < CPLD; ++i) {
    const int c = i * SGD + dj;
    const bool in = CPLD * SGD == UF || c < UF;
#pragma unroll
    for (int st = 0; st < RS; ++st) {
      const int n = i * RS + st, b = n & 1;
      if (st + 1 < RS) fetch_row(i, st + 1, b ^ 1);
      else if (i + 1 < CPLD) {
        fetch_row(i + 1, 0, b ^ 1);
        fetch_x(i + 1, (i + 1) & 1);
      }
      // (the scheduler would otherwise sink the reads next to their use)
      __builtin_amdgcn_sched_barrier(0);
      if (in) {
        const float Sd = bf16_to_f32(sv[b]), Bd = bf16_to_f32(bv[b]);
        pv[st] += Sd * chunk_dot_regs(cd[b], xa[i & 1]) + (Bd - 128.f * Sd) * xs[i & 1];
      }
    }
  }
#pragma unroll
  for (int st = 0; st < RS; ++st) {
    const int rl = st * RPSD + dsub;
    const float v = group_sum<SGD>(pv[st]);
    if (dj == 0) red[rl] = dok ? sc * (v + (C::PBIAS_ ? dbias[rl] : 0.f)) : 0.f;
  }
  if (!dok && lane == 0) flag_error();
}

template <int D, int F, int K, bool PBIAS, int ACT, int MODE, int RENORM>
__global__ __launch_bounds__(512) void stack_wide_kernel(StackArgs a) {
  using C = WideCfg<D, F, K, PBIAS, ACT, MODE, RENORM>;
  using WS = StackWs<F, K>;
  constexpr int U = C::U, UF = C::UF, SBD_U4 = C::SBD_U4, NP = C::NP;
  constexpr int ROWS_U = C::ROWS_U, ROWS_D = C::ROWS_D, NPOS = C::NPOS;
  constexpr int XU4 = C::XU4, HU4 = C::HU4, HPL = C::HPL, XPL = C::XPL, NWG = C::NWG;
  constexpr int RIT = (XU4 + 63) / 64;
  constexpr int W_DMA = 4, W_ROUTER = 6, W_RANK = 7;
  static_assert(C::WAVES_U == W_DMA && C::NT / 64 == 8, "wave roles");
  (void)SBD_U4;

  __shared__ uint4 act_l[4 * U];
  __shared__ float asum_l[U];
  __shared__ uint4 sbu_l[C::SUI_ALL * 64];    // gate/up scales (gate S | gate B | up S | up B)
  __shared__ uint32_t ubias_l[64];            // gate/up projection biases (bf16 pairs)
  __shared__ uint4 dcode_l[C::WAVES_D][C::DCI][64];   // down codes of each down wave's rows
  __shared__ uint4 dsc_l[C::WAVES_D][C::DSI][64];     // their scales (S | B)
  __shared__ uint4 hact_l[4 * UF];                    // the position's activations
  __shared__ float hsum_l[UF];
  __shared__ float dbias_l[C::WAVES_D][ROWS_D];
  __shared__ float dred_l[C::WAVES_D][ROWS_D];        // each down wave's score-weighted rows
  __shared__ float red_l[K][C::CROWS];                // the combine's per-rank rows
  __shared__ int sel_id[K];
  __shared__ float sel_sc[K];
  __shared__ int32_t sel_ref[K];
  __shared__ int pred_buf[2][K];       // lookahead's best, rank order (slot l & 1)
  __shared__ int32_t pred_ref[2][K];   // their slot refs
  __shared__ int pred_cnt[2];          // predicted positions (<= K)
  __shared__ int pos_fix[K];           // position p runs a fix-up of this rank, or -1
  __shared__ int pos_rank[K];          // routing rank whose activations position p holds
  __shared__ int fix_pos[K];           // the positions running a fix-up, in order
  __shared__ int n_fix;                // ... how many
  // monotonic: WAVES_U + 1 arrivals per layer (the gate/up waves' loads
  // landed, x staged); layer l's meeting waits for (WAVES_U + 1) * (l + 1).
  // A wave arrives for layer l + 1 only after layer l's meeting (gate/up
  // waves) or after every wave's layer-l arrival on dsync (wave 7), so the
  // count reaches that target exactly when layer l's arrivals are in.
  __shared__ uint32_t staged;
  // layer flags (the value layer_flag(l) once the event of layer l happened)
  __shared__ uint32_t lstart;          // the layer boundary was seen (wave 7)
  __shared__ uint32_t routed;          // the routing and positions are known (wave 7)
  __shared__ uint32_t looked;          // layer l+1's prediction is in pred_* (wave 6)
  __shared__ uint32_t hcnt;            // monotonic: WAVES_U per layer (activation quarters staged)
  __shared__ uint32_t dpre;            // monotonic: 2 per layer (waves 4 and 5 done with the
                                       // predicted expert's down rows)
  // monotonic counters
  __shared__ uint32_t dsync;           // 8 arrivals per layer: every wave is done with it

  const int tid0 = threadIdx.x;
  const int wg = blockIdx.x;
  const uint32_t ep = a.epoch;
  const Abort ab{reinterpret_cast<uint32_t *>(a.ws + WS::kAbort), ep};
  uint64_t *const lgt = reinterpret_cast<uint64_t *>(a.ws + WS::kLgt);
  uint64_t *const hpred = reinterpret_cast<uint64_t *>(a.ws + WS::kHpred);
  uint64_t *const hfix = reinterpret_cast<uint64_t *>(a.ws + WS::kHfix);
  uint64_t *const part = reinterpret_cast<uint64_t *>(a.ws + WS::kPart);
  const bool uact = wg < C::ITEMS_U, dact = wg < C::ITEMS_D;
  static_assert(C::ITEMS_U % K == 0 && C::ITEMS_D % K == 0 && C::ITEMS_U / K == NPOS,
                "positions dealt round robin over the workgroups");
  const int upos = wg % K, urow0 = (wg / K) * ROWS_U;            // gate/up block
  const int drow0 = dact ? (wg / K) * C::ROWS_DWG : 0;           // down rows (position upos)
  const int crow0 = dact ? wg * C::CROWS : 0;                    // combined output rows
  constexpr int W_COMB = W_DMA + 1;   // combines the previous layer (idle until the routing)
  {
    const uint32_t none = layer_flag(a, 0) - 1u;   // no flag of this launch
    if (tid0 < 2) pred_cnt[tid0] = 0;   // layer 0 has no prediction
    if (tid0 == 0) {
      routed = lstart = looked = none;
      dsync = staged = hcnt = dpre = 0;
    }
  }
  __syncthreads();

  // gate/up registers of the predicted expert, loaded one layer ahead
  WideU<C> ur = {};

  // Roles per layer, ordered by LDS flags and counters rather than
  // workgroup barriers: a wave issuing a large batch of loads is held at its
  // load instructions until the memory queues drain, and a barrier would
  // hold every other wave with it.
  for (int l = 0; l < a.L; ++l) {
    // the thread index made opaque once per layer: addresses derived from it
    // are computed inside the layer, not held in registers across all layers
    int tid = tid0;
    asm volatile("" : "+v"(tid));
    const int lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const bool has_next = l + 1 < a.L;
    const uint32_t fl = layer_flag(a, l);
    if (wave == 0) trace_mark(a, l, TR_START);
    if (wave < C::WAVES_U) {
      // ---- gate/up of the predicted expert (loaded during the previous
      // layer): every wave's loads landed, x staged (wave 7), then the rows
      __builtin_amdgcn_s_waitcnt(0);
      lds_arrive(&staged);
      lds_wait_count(&staged, (uint32_t)(C::WAVES_U + 1) * (uint32_t)(l + 1));
      if (uact && upos < pred_cnt[l & 1])
        ur.run(tid, act_l, asum_l, reinterpret_cast<const uint16_t *>(sbu_l),
               reinterpret_cast<const uint16_t *>(ubias_l), hpred + (size_t)upos * (F / 2),
               urow0, fl);
      if (wave == 0) trace_mark(a, l, TR_U_ARRIVED);
      lds_wait_flag(&routed, fl);
      if (wave == 0) trace_mark(a, l, TR_SELECTED);
      if (wg == 0 && tid < K) {
        KARG(ids)[(size_t)l * K + tid] = sel_id[tid];
        KARG(scores)[(size_t)l * K + tid] = sel_sc[tid];
        KARG(refs_out)[(size_t)l * K + tid] = sel_ref[tid];
        if (sel_ref[tid] < 0) atomicAdd(KARG(miss) + l, 1);
      }
      // ---- fix-up: a position whose predicted expert was not routed takes
      // a routed expert that was not predicted.  Its gate/up rows are spread
      // over the whole grid (task t = wave * NWG + workgroup: rows 2t, 2t+1
      // of the fix-up in t / (F / 2)), straight from the pool, so one miss
      // costs each gate/up wave about one task instead of a 48-row pass on
      // the position's own workgroups (its down rows are staged by its down
      // waves like the others)
      {
        constexpr int FT = F / 2;
        constexpr int STRIDE = C::WAVES_U * NWG;
        const int nf = n_fix;
        // two tasks at a time: the second one's loads in flight while the
        // first one computes
        for (int t = wave * NWG + wg; t < nf * FT; t += 2 * STRIDE) {
          const int p0 = fix_pos[t / FT], t2 = t + STRIDE;
          WideFix<C> f0;
          wide_fix_load<C>(lane, a, sel_ref[pos_rank[p0]], t % FT, f0);
          if (t2 < nf * FT) {
            const int p1 = fix_pos[t2 / FT];
            WideFix<C> f1;
            wide_fix_load<C>(lane, a, sel_ref[pos_rank[p1]], t2 % FT, f1);
            wide_fix_compute<C>(lane, t % FT, f0, act_l, asum_l, hfix + (size_t)p0 * FT, fl);
            wide_fix_compute<C>(lane, t2 % FT, f1, act_l, asum_l, hfix + (size_t)p1 * FT, fl);
          } else {
            wide_fix_compute<C>(lane, t % FT, f0, act_l, asum_l, hfix + (size_t)p0 * FT, fl);
          }
        }
      }
      if (wave == 0) trace_mark(a, l, TR_FIXED);
      // ---- gate/up wave w polls quarter w of the activations of the
      // workgroup's position and stages it for the down waves: it has no
      // loads in flight here, while the down waves' polls would return only
      // after their direct-to-LDS down-row loads (loads complete in order)
      if (uact) {
        const bool fix = pos_fix[upos] >= 0;
        uint4 pv[C::HPWL];
        get_acts_quarter<HU4, C::HPW, C::HPWL>(tid, (fix ? hfix : hpred) + (size_t)upos * (F / 2),
                                               wave, fl, ab, pv);
        if (dact) {
#pragma unroll
          for (int it = 0; it < C::HPWL; ++it) {
            const int k = lane + 64 * it, i = C::HPW * wave + k;
            const bool mine = k < C::HPW && i < HU4;
            float sm = 0.f;
            if (mine) sm = stage_piece<UF>(hact_l, i, pv[it]);
            sm += dpp_f<kDppQuadXor1>(sm);
            sm += dpp_f<kDppQuadXor2>(sm);
            if (mine && (i & 3) == 0) hsum_l[i >> 2] = sm;
          }
        }
        lds_arrive(&hcnt);
        if (wave == 2) trace_mark(a, l, TR_D_WAITED);
      }
      lds_arrive(&dsync);
      // ---- gate/up loads of layer l+1's prediction, once this workgroup's
      // activation polls are done (loads queued ahead of them would delay
      // them); in flight through the down pass and the layer boundary
      // (wave 6 publishes layer l+1's prediction under `looked`; it always
      // does when there is a next layer)
      if (has_next && uact) lds_wait_flag(&looked, fl);
      if (has_next && uact && upos < pred_cnt[(l + 1) & 1]) {
        lds_wait_count(&hcnt, (uint32_t)C::WAVES_U * (uint32_t)(l + 1));
        ur.load(tid, a, pred_ref[(l + 1) & 1][upos], urow0, sbu_l, ubias_l);
      } else {
        ur.forget();
      }
    } else {
      ur.forget();
      if (wave < W_ROUTER) {
        // wave 5: the previous layer's output rows, complete once its
        // boundary is passed (the entries' flags confirm each)
        lds_wait_flag(&lstart, fl);
        if (wave == W_COMB && dact && l > 0)
          wide_combine<K, C::CROWS>(part + (size_t)((l - 1) & 1) * K * kStackMaxD, crow0,
                                    layer_flag(a, l - 1), ab, red_l, KARG(y) + (size_t)(l - 1) * D);
        // waves 4 and 5, idle until the routing: the down rows of the
        // expert predicted at this position, all four quarters (wave 4
        // quarters 0 and 2, wave 5 quarters 1 and 3), then an arrival once
        // they landed
        if (dact && upos < pred_cnt[l & 1]) {
          const int32_t pref = __builtin_amdgcn_readfirstlane(pred_ref[l & 1][upos]);
#pragma unroll
          for (int h = 0; h < 2; ++h) {
            const int qq = (wave - W_DMA) + 2 * h;
            wide_d_stage<C>(lane, a, pref, drow0 + qq * ROWS_D, dcode_l[qq], dsc_l[qq]);
            if (PBIAS && lane < ROWS_D) {
              const uint16_t *dbias = reinterpret_cast<const uint16_t *>(resolve_packed<typename C::Layout>(
                  a.pa, comp_index(PROJ_DOWN, PART_BIAS, NP), pref));
              dbias_l[qq][lane] = dbias ? bf16_to_f32(dbias[drow0 + qq * ROWS_D + lane]) : 0.f;
            }
          }
          __builtin_amdgcn_s_waitcnt(0);
        }
        lds_arrive(&dpre);
        lds_wait_flag(&routed, fl);
      } else if (wave == W_ROUTER) {
        // ---- one router row (the lane partition and summation order of
        // route_kernel: bit-identical logits), its weights loaded before the
        // layer boundary; then the lookahead ranking of layer l+1
        const int nrows = a.E * (has_next ? 2 : 1);
        const bool rrow = wg < nrows, rnxt = wg >= a.E;
        uint4 wr[RIT] = {};
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
        lds_wait_flag(&lstart, fl);
        if (rrow) {
          const int e = rnxt ? wg - a.E : wg;
          const uint4 *x4 = reinterpret_cast<const uint4 *>(KARG(x) + (size_t)l * D);
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
          if (lane == 0) put_logit(lgt + (rnxt ? a.E : 0) + e, acc, fl);
          trace_mark(a, l, TR_R_ARRIVED);
        }
        if (has_next) {
          // raw bf16 logits of layer l+1's router on x_l
          const int e0 = lane, e1 = lane + 64;
          const uint16_t *bias0 = KARG(bias);
          const uint16_t *bias = bias0 ? bias0 + (size_t)(l + 1) * a.E : nullptr;
          const float b0 = bias ? bf16_to_f32(bias[min(e0, a.E - 1)]) : 0.f;
          const float b1 = bias ? bf16_to_f32(bias[min(e1, a.E - 1)]) : 0.f;
          const int32_t *tabn = KARG(table) + (size_t)(l + 1) * a.E;
          const int32_t t0 = tabn[min(e0, a.E - 1)], t1 = tabn[min(e1, a.E - 1)];
          float l0, l1;
          get_logits(lgt + a.E, a.E, fl, ab, l0, l1, wide_lane());
          const float z0 = e0 < a.E ? round_bf16(l0 + b0) : -INFINITY;
          const float z1 = e1 < a.E ? round_bf16(l1 + b1) : -INFINITY;
          bool s0, s1;
          int r0, r1;
          const int ksel = min(max(a.kp, K), a.E);
          select_topk(e0 < a.E ? order_key(z0) : -1, e1 < a.E ? order_key(z1) : -1, ksel, lane,
                      s0, s1, r0, r1);
          if (wg == 0) {
            int32_t *pred = KARG(pred);
            if (s0 && r0 < a.kp) pred[(size_t)l * a.kp + r0] = e0;
            if (s1 && r1 < a.kp) pred[(size_t)l * a.kp + r1] = e1;
          }
          int *pn = pred_buf[(l + 1) & 1];
          int32_t *pr = pred_ref[(l + 1) & 1];
          if (s0 && r0 < K) {
            pn[r0] = e0;
            pr[r0] = t0;
          }
          if (s1 && r1 < K) {
            pn[r1] = e1;
            pr[r1] = t1;
          }
          if (lane == 0) pred_cnt[(l + 1) & 1] = min(a.kp, K);
          lds_set_flag(&looked, fl);
        }
        lds_wait_flag(&routed, fl);
      } else {
        // ---- the layer boundary, x_l into LDS, the routing -------------
        if (l > 0) wave_wait(counter<WS>(a, l - 1, CNT_D), ep * NWG, ab, wide_lane());
        lds_set_flag(&lstart, fl);
        trace_mark(a, l, TR_R_WAITED);
        {
          const uint4 *x4 = reinterpret_cast<const uint4 *>(KARG(x) + (size_t)l * D);
          uint4 xv[XPL];
#pragma unroll
          for (int it = 0; it < XPL; ++it) xv[it] = load16(x4 + min(lane + 64 * it, XU4 - 1));
#pragma unroll
          for (int it = 0; it < XPL; ++it) {
            const int i = lane + 64 * it;
            float sm = 0.f;
            if (i < XU4) sm = stage_piece<U>(act_l, i, xv[it]);
            sm += dpp_f<kDppQuadXor1>(sm);
            sm += dpp_f<kDppQuadXor2>(sm);
            if (i < XU4 && (i & 3) == 0) asum_l[i >> 2] = sm;
          }
          lds_arrive(&staged);
        }
        const int pcnt = pred_cnt[l & 1];
        const int e0 = lane, e1 = lane + 64;
        const uint16_t *bias0 = KARG(bias);
        const uint16_t *bias = bias0 ? bias0 + (size_t)l * a.E : nullptr;
        const float b0 = bias ? bf16_to_f32(bias[min(e0, a.E - 1)]) : 0.f;
        const float b1 = bias ? bf16_to_f32(bias[min(e1, a.E - 1)]) : 0.f;
        const int32_t *tab = KARG(table) + (size_t)l * a.E;
        const int32_t t0 = tab[min(e0, a.E - 1)], t1 = tab[min(e1, a.E - 1)];
        float l0, l1;
        get_logits(lgt, a.E, fl, ab, l0, l1, wide_lane());
        trace_mark(a, l, TR_R_ALL);
        const float z0 = e0 < a.E ? round_bf16(l0 + b0) : -INFINITY;
        const float z1 = e1 < a.E ? round_bf16(l1 + b1) : -INFINITY;
        float v0 = z0, v1 = z1;
        if (MODE == MOE_ROUTE_SOFTMAX_TOPK) {
          const float m = wave_max(fmaxf(z0, z1));
          const float x0 = (e0 < a.E) ? expf(z0 - m) : 0.f;
          const float x1 = (e1 < a.E) ? expf(z1 - m) : 0.f;
          const float sum = group_sum<64>(x0 + x1);
          v0 = round_bf16(x0 / sum);
          v1 = round_bf16(x1 / sum);
        }
        bool s0, s1;
        int r0, r1;
        select_topk(e0 < a.E ? order_key(v0) : -1, e1 < a.E ? order_key(v1) : -1, K, lane, s0,
                    s1, r0, r1);
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
          const float sum = group_sum<64>(x0 + x1);
          sc0 = round_bf16(x0 / sum);
          sc1 = round_bf16(x1 / sum);
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
        __atomic_signal_fence(__ATOMIC_SEQ_CST);
        __builtin_amdgcn_wave_barrier();
        __atomic_signal_fence(__ATOMIC_SEQ_CST);
        // position p keeps rank r when its predicted expert was routed at r;
        // the routed experts that were not predicted go, in rank order, to
        // the remaining positions in order (fix-ups)
        const uint64_t below = lane ? (~0ull >> (64 - lane)) : 0ull;
        int prank = -1;      // lane = position: the rank of its predicted expert
        bool hit = false;    // lane = rank: its expert was predicted
        if (lane < K) {
          int sv[K], pv[K];
#pragma unroll
          for (int r = 0; r < K; ++r) sv[r] = sel_id[r];
#pragma unroll
          for (int p = 0; p < K; ++p) pv[p] = p < pcnt ? pred_buf[l & 1][p] : -1;
#pragma unroll
          for (int r = 0; r < K; ++r)
            if (lane < pcnt && sv[r] == pv[lane]) prank = r;
#pragma unroll
          for (int p = 0; p < K; ++p)
            if (p < pcnt && pv[p] == sv[lane]) hit = true;
        }
        const uint64_t free_m = __ballot(lane < K && prank < 0);   // positions needing a fix-up
        const uint64_t miss_m = __ballot(lane < K && !hit);         // ranks needing a fix-up
        if (lane < K && prank < 0) fix_pos[__popcll(free_m & below)] = lane;
        if (lane == 0) n_fix = __popcll(free_m);
        if (lane < K) {
          if (prank >= 0) {
            pos_rank[lane] = prank;
            pos_fix[lane] = -1;
          } else {
            // the i-th free position takes the i-th missed rank
            const int fi = __popcll(free_m & below);
            uint64_t m = miss_m;
            for (int i = 0; i < fi; ++i) m &= m - 1;
            const int r = (int)__builtin_ctzll(m);
            pos_rank[lane] = r;
            pos_fix[lane] = r;
          }
        }
        lds_set_flag(&routed, fl);
      }
      // ---- down wave q = wave - 4: 12 rows of the expert at the
      // workgroup's position into LDS by direct-to-LDS loads (issued once
      // the routing is known), its down biases, then (the activations
      // staged by the gate/up waves) the rows, published as flagged entries
      // of the expert's rank
      const int q = wave - W_DMA;
      const int r = pos_rank[upos];
      const int32_t dref = __builtin_amdgcn_readfirstlane(sel_ref[r]);
      const int qrow0 = drow0 + q * ROWS_D;
      // the rows staged by waves 4 and 5 at the layer start (their loads
      // landed) are the routed expert's when the position kept its
      // prediction; otherwise this wave stages its own, after those loads
      // (they write the same LDS)
      if (dact) lds_wait_count(&dpre, 2u * (uint32_t)(l + 1));
      if (wave == W_DMA) trace_mark(a, l, TR_SOFTMAX);   // (slot reused: predicted rows in)
      if (dact && !(upos < pred_cnt[l & 1] && pos_fix[upos] < 0)) {
        wide_d_stage<C>(lane, a, dref, qrow0, dcode_l[q], dsc_l[q]);
        if (PBIAS && lane < ROWS_D) {
          const uint16_t *dbias = reinterpret_cast<const uint16_t *>(resolve_packed<typename C::Layout>(
              a.pa, comp_index(PROJ_DOWN, PART_BIAS, NP), dref));
          dbias_l[q][lane] = dbias ? bf16_to_f32(dbias[qrow0 + lane]) : 0.f;
        }
      }
      if (dact) {
        __builtin_amdgcn_s_waitcnt(0);   // this wave's direct-to-LDS loads landed
        if (wave == W_DMA) trace_mark(a, l, TR_LOOKED);   // (slot reused)
        lds_wait_count(&hcnt, (uint32_t)C::WAVES_U * (uint32_t)(l + 1));   // the activations
        if (wave == W_DMA) trace_mark(a, l, TR_SPARE1);   // (slot reused)
        __atomic_signal_fence(__ATOMIC_SEQ_CST);
        wide_down_rows<C>(lane, a, dref, qrow0, sel_sc[r], dcode_l[q],
                          reinterpret_cast<const uint16_t *>(&dsc_l[q][0][0]), hact_l, hsum_l,
                          dbias_l[q], dred_l[q]);
        __atomic_signal_fence(__ATOMIC_SEQ_CST);
        __builtin_amdgcn_wave_barrier();
        __atomic_signal_fence(__ATOMIC_SEQ_CST);
        if (lane < ROWS_D)
          __hip_atomic_store(part + ((size_t)(l & 1) * K + r) * kStackMaxD + qrow0 + lane,
                             (uint64_t)__float_as_uint(dred_l[q][lane]) | ((uint64_t)fl << 32),
                             __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        if (wave == W_DMA) trace_mark(a, l, TR_LOGITS);   // (slot reused: down rows done)
        if (wave == W_RANK) trace_mark(a, l, TR_UROWS2);  // (slot reused)
      }
      lds_arrive(&dsync);
    }
    // ---- wave 7: once every wave is done with layer l, arrive.  Every
    // entry this workgroup read in layer l has been read, and its per-rank
    // output rows carry the layer's flag, so the arrival needs no wait for
    // its stores.
    if (wave == W_RANK) {
      lds_wait_count(&dsync, 8u * (uint32_t)(l + 1));
      if (lane == 0)
        __hip_atomic_fetch_add(counter<WS>(a, l, CNT_D) + (wg % kSub) * 32, 1u,
                               __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
      trace_mark(a, l, TR_D_ARRIVED);
    }
  }
  // the last layer's output rows, after every workgroup has arrived
  if ((threadIdx.x >> 6) == W_RANK) {
    wave_wait(counter<WS>(a, a.L - 1, CNT_D), ep * NWG, ab);
    if (dact)
      wide_combine<K, C::CROWS>(part + (size_t)((a.L - 1) & 1) * K * kStackMaxD, crow0,
                                layer_flag(a, a.L - 1), ab, red_l, KARG(y) + (size_t)(a.L - 1) * D);
  }
}

}  // namespace moe
