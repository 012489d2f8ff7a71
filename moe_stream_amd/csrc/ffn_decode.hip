// Batch-1 / small-T expert block for gfx950: a bandwidth-bound dequant-GEMV
// in two kernels.
//
//   ffn_gate_up : for every (token, routed expert) pair and every row r of
//                 d_ff, gate_r . x and up_r . x from the 4-bit codes, then the
//                 gated activation; h[pair, r] stored as bf16.
//   ffn_down    : for every token and output row r of d_model, the k routed
//                 experts' down_r . h_j, scaled by the routing scores and
//                 summed in expert order (deterministic, no atomics).
//
// Math (reference: the factorised group form of kernels.py:104-106,141-145):
//   w(o,i) = S[o,g]*q(o,i) + B[o,g], g = i/64
//   row . x = sum_chunks S*sum((128+q)*x) + (B - 128*S)*sum(x)
// where a chunk is 32 consecutive inputs (half a quant group, one 16-byte
// load of codes).  The 128 offset comes from decoding codes as the bf16
// numbers 128+q (see codes_to_bf16x2); products and sums run in fp32 through
// v_dot2c_f32_bf16.
//
// Work mapping: SG lanes share one weight row; lane j of a row reads 16-byte
// chunks j, j+SG, j+2SG, ... so each load instruction of a wave covers
// 64/SG rows with SG*16 contiguous bytes each.  Every lane issues all of its
// code loads first; while they are in flight the workgroup stages the
// activations (already rearranged into the pair order of the decoded codes,
// with per-chunk sums) and the rows' scales and biases in LDS with coalesced
// 16-byte loads.  Row sums are an SG-lane butterfly.
#include "launchers.h"

namespace moe {

__device__ int g_device_error = 0;

// Stage one 16-byte piece (8 activations, index i of the row) into LDS in
// pair order: act[q*U + c] holds pieces q=0..3 of chunk c, so the lanes of a
// row, which read consecutive chunks, hit consecutive 16-byte LDS slots.
// Returns the 8-value partial sum; the caller reduces it over the 4 pieces
// of a chunk (4 consecutive lanes).
template <int U>
__device__ __forceinline__ float stage_piece(uint4 *act, int i, uint4 a) {
  const int c = i >> 2, q = i & 3;
  uint32_t in[4] = {a.x, a.y, a.z, a.w}, out[4];
  x_pairs(in, out);
  act[q * U + c] = make_uint4(out[0], out[1], out[2], out[3]);
  float s = 0.f;
#pragma unroll
  for (int m = 0; m < 4; ++m) s += bf16_to_f32(in[m] & 0xffffu) + bf16_to_f32(in[m] >> 16);
  return s;
}

// sum((128+q)*x) over one 16-byte chunk of codes (32 inputs), activations
// from LDS in pair order.
template <int U>
__device__ __forceinline__ float chunk_dot_lds(const uint4 &c, const uint4 *act,
                                               int chunk) {
  float acc = 0.f;
  const uint32_t w[4] = {c.x, c.y, c.z, c.w};
#pragma unroll
  for (int q = 0; q < 4; ++q) {
    const uint4 xa = act[q * U + chunk];
    const uint32_t xv[4] = {xa.x, xa.y, xa.z, xa.w};
    uint32_t p[4];
    codes_to_bf16x2(w[q], p);
#pragma unroll
    for (int m = 0; m < 4; ++m) acc = dot2_bf16(p[m], xv[m], acc);
  }
  return acc;
}

// A chunk's 32 codes decoded once (4 words -> 16 packed bf16 pairs, the
// order of chunk_dot_lds), for several activation vectors.
__device__ __forceinline__ void decode_chunk(const uint4 &c, uint32_t (&p)[16]) {
  const uint32_t w[4] = {c.x, c.y, c.z, c.w};
#pragma unroll
  for (int q = 0; q < 4; ++q) {
    uint32_t t[4];
    codes_to_bf16x2(w[q], t);
#pragma unroll
    for (int m = 0; m < 4; ++m) p[4 * q + m] = t[m];
  }
}
// chunk_dot_lds over pre-decoded codes: the same products in the same order.
template <int U>
__device__ __forceinline__ float chunk_dot_dec(const uint32_t (&p)[16], const uint4 *act,
                                               int chunk) {
  float acc = 0.f;
#pragma unroll
  for (int q = 0; q < 4; ++q) {
    const uint4 xa = act[q * U + chunk];
    const uint32_t xv[4] = {xa.x, xa.y, xa.z, xa.w};
#pragma unroll
    for (int m = 0; m < 4; ++m) acc = dot2_bf16(p[4 * q + m], xv[m], acc);
  }
  return acc;
}

__device__ __forceinline__ float apply_act(int act, float g, float u,
                                           float alpha, float limit) {
  if (act == MOE_ACT_SWIGLU) {
    return (g / (1.f + expf(-g))) * u;  // silu(g)*u, engine_v3.py:597
  }
  // clamped SwiGLU, engine_120b.py:143 (HANDOFF.md:886-887)
  g = fminf(g, limit);
  u = fminf(fmaxf(u, -limit), limit);
  return g * (1.f / (1.f + expf(-alpha * g))) * (u + 1.f);
}

// ---------------------------------------------------------------------------
// gate/up + activation
// ---------------------------------------------------------------------------
template <int D, int F, int SG, int WAVES, int RSTEPS, bool PBIAS>
__global__ __launch_bounds__(WAVES * 64) void ffn_gate_up_kernel(
    PoolArgs pa, const RefList refs,
    const uint16_t *__restrict__ x, int k, uint16_t *__restrict__ h, int act,
    float alpha, float limit) {
  constexpr int U = D / 32;                 // 16-byte code chunks per row
  constexpr int CPL = (U + SG - 1) / SG;    // chunks per lane
  constexpr int RPS = 64 / SG;              // rows per wave step
  constexpr int ROWS_WG = WAVES * RSTEPS * RPS;
  constexpr int WG_PER_PAIR = F / ROWS_WG;
  constexpr int NG = D / 64;                // quant groups per row
  constexpr int NP = PBIAS ? 4 : 3;
  constexpr int NT = WAVES * 64;
  constexpr int XU4 = D / 8;                // 16-byte pieces of x
  constexpr int SB_U4 = ROWS_WG * NG * 2 / 16;  // 16-byte pieces per scale block
  static_assert(F % ROWS_WG == 0, "rows per workgroup must divide d_ff");
  static_assert((ROWS_WG * NG * 2) % 16 == 0, "scale block must be 16-byte pieces");

  __shared__ uint4 act_l[4 * U];
  __shared__ float asum_l[U];
  __shared__ uint4 sb_l[4][SB_U4];          // gate S, gate B, up S, up B

  const int pair = blockIdx.x / WG_PER_PAIR;
  const int rb = blockIdx.x % WG_PER_PAIR;
  const int tid = threadIdx.x;
  const int lane = tid & 63, wave = tid >> 6;
  const int rsub = lane / SG, j = lane % SG;
  const int t = pair / k;
  const int32_t ref = refs[pair];
  const int row0 = rb * ROWS_WG;

  const char *gw = resolve(pa, comp_index(PROJ_GATE, PART_W, NP), ref);
  if (gw == nullptr) {  // uniform over the workgroup
    if (tid == 0) flag_error();
    for (int r = tid; r < ROWS_WG; r += NT) h[(int64_t)pair * F + row0 + r] = 0;
    return;
  }
  const char *uw = resolve(pa, comp_index(PROJ_UP, PART_W, NP), ref);

  // 1. the small loads first (activations, scales/biases: 16 bytes per
  //    thread), so that staging them into LDS only waits for them and not
  //    for the code stream issued after them (loads retire in order)
  constexpr int XIT = (XU4 + NT - 1) / NT;
  constexpr int SIT = (4 * SB_U4 + NT - 1) / NT;
  uint4 xr[XIT], sr[SIT];
  {
    const uint4 *x4 = reinterpret_cast<const uint4 *>(x + (int64_t)t * D);
    // every thread loads (clamped indices, surplus ignored): conditional
    // loads would be waited for before the code stream is issued
#pragma unroll
    for (int it = 0; it < XIT; ++it) xr[it] = load16(x4 + min(it * NT + tid, XU4 - 1));
    // (selected by conditionals, not through an indexed array: a pointer
    // picked out of a private array loses its global address space, and
    // the flat load that results is waited for together with every load
    // issued after it)
    const char *gs = resolve(pa, comp_index(PROJ_GATE, PART_S, NP), ref);
    const char *gb = resolve(pa, comp_index(PROJ_GATE, PART_B, NP), ref);
    const char *us = resolve(pa, comp_index(PROJ_UP, PART_S, NP), ref);
    const char *ub = resolve(pa, comp_index(PROJ_UP, PART_B, NP), ref);
#pragma unroll
    for (int it = 0; it < SIT; ++it) {
      const int i = min(it * NT + tid, 4 * SB_U4 - 1);
      const int p = i / SB_U4, o = i % SB_U4;
      const char *sp = p == 0 ? gs : p == 1 ? gb : p == 2 ? us : ub;
      sr[it] = load16(reinterpret_cast<const uint4 *>(sp + (int64_t)row0 * NG * 2) + o);
    }
  }
  // the rows' projection biases, also ahead of the code stream
  float gbv[RSTEPS], ubv[RSTEPS];
#pragma unroll
  for (int s = 0; s < RSTEPS; ++s) gbv[s] = ubv[s] = 0.f;
  if (PBIAS) {
    const uint16_t *gbias = reinterpret_cast<const uint16_t *>(
        resolve(pa, comp_index(PROJ_GATE, PART_BIAS, NP), ref));
    const uint16_t *ubias = reinterpret_cast<const uint16_t *>(
        resolve(pa, comp_index(PROJ_UP, PART_BIAS, NP), ref));
#pragma unroll
    for (int s = 0; s < RSTEPS; ++s) {
      const int row = row0 + (wave * RSTEPS + s) * RPS + rsub;
      gbv[s] = bf16_to_f32(gbias[row]);
      ubv[s] = bf16_to_f32(ubias[row]);
    }
  }

  // 2. every code load of this lane (the scheduling barriers keep the
  //    small loads ahead of the code stream, and the staging behind it)
  issue_order_fence();
  uint4 cg[RSTEPS][CPL], cu[RSTEPS][CPL];
#pragma unroll
  for (int s = 0; s < RSTEPS; ++s) {
    const int row = row0 + (wave * RSTEPS + s) * RPS + rsub;
    const uint4 *g4 = reinterpret_cast<const uint4 *>(gw + (int64_t)row * (D / 2));
    const uint4 *u4 = reinterpret_cast<const uint4 *>(uw + (int64_t)row * (D / 2));
#pragma unroll
    for (int i = 0; i < CPL; ++i) {   // surplus chunks (c >= U) re-read the last one, unused
      const int c = min(i * SG + j, U - 1);
      cg[s][i] = load_stream16(g4 + c);
      cu[s][i] = load_stream16(u4 + c);
    }
  }
  issue_order_fence();
  // 3. stage scales/biases and the activations (pair order + chunk sums)
#pragma unroll
  for (int it = 0; it < SIT; ++it) {
    const int i = it * NT + tid;
    if (i < 4 * SB_U4) (&sb_l[0][0])[i] = sr[it];
  }
#pragma unroll
  for (int it = 0; it < XIT; ++it) {
    const int i = it * NT + tid;
    float s = 0.f;
    if (i < XU4) s = stage_piece<U>(act_l, i, xr[it]);
    s += dpp_f<kDppQuadXor1>(s);   // the 4 pieces of a chunk: 4 adjacent lanes
    s += dpp_f<kDppQuadXor2>(s);
    if (i < XU4 && (i & 3) == 0) asum_l[i >> 2] = s;
  }
  __syncthreads();

  const uint16_t *sbh = reinterpret_cast<const uint16_t *>(&sb_l[0][0]);
  constexpr int SBN = SB_U4 * 8;  // bf16 per scale block
  // 4. dot products, row sums, activation
#pragma unroll
  for (int s = 0; s < RSTEPS; ++s) {
    const int rl = (wave * RSTEPS + s) * RPS + rsub;  // row inside the WG
    float pg = 0.f, pu = 0.f;
#pragma unroll
    for (int i = 0; i < CPL; ++i) {
      const int c = i * SG + j;
      if (CPL * SG == U || c < U) {
        const int g = rl * NG + (c >> 1);
        const float Sg = bf16_to_f32(sbh[0 * SBN + g]), Bg = bf16_to_f32(sbh[1 * SBN + g]);
        const float Su = bf16_to_f32(sbh[2 * SBN + g]), Bu = bf16_to_f32(sbh[3 * SBN + g]);
        const float xs = asum_l[c];
        pg += Sg * chunk_dot_lds<U>(cg[s][i], act_l, c) + (Bg - 128.f * Sg) * xs;
        pu += Su * chunk_dot_lds<U>(cu[s][i], act_l, c) + (Bu - 128.f * Su) * xs;
      }
    }
    pg = group_sum<SG>(pg);
    pu = group_sum<SG>(pu);
    if (j == 0) {
      const int row = row0 + rl;
      pg += gbv[s];   // 0 without projection bias
      pu += ubv[s];
      h[(int64_t)pair * F + row] = (uint16_t)f32_to_bf16(apply_act(act, pg, pu, alpha, limit));
    }
  }
}

// ---------------------------------------------------------------------------
// down + weighted combine; one wave per routed expert, blockDim = 64*k.
// Dynamic LDS per wave: h in pair order (4*U pieces), chunk sums (U floats),
// scales and biases of the workgroup's rows; then the combine buffer.
// ---------------------------------------------------------------------------
template <int D, int F, int SG, int RSTEPS>
struct DownLds {
  static constexpr int U = F / 32;
  static constexpr int RPS = 64 / SG;
  static constexpr int ROWS_WG = RSTEPS * RPS;
  static constexpr int NG = F / 64;
  static constexpr int SB_U4 = ROWS_WG * NG * 2 / 16;
  static constexpr int ACT_BYTES = 4 * U * 16;
  static constexpr int SUM_BYTES = ((U * 4 + 15) / 16) * 16;
  static constexpr int SB_BYTES = 2 * SB_U4 * 16;
  static constexpr int WAVE_BYTES = ACT_BYTES + SUM_BYTES + SB_BYTES;
  static constexpr size_t bytes(int k) {
    return (size_t)k * WAVE_BYTES + (size_t)MOE_MAX_TOPK * ROWS_WG * 4;
  }
};

template <int D, int F, int SG, int RSTEPS, bool PBIAS>
__global__ __launch_bounds__(64 * MOE_MAX_TOPK) void ffn_down_kernel(
    PoolArgs pa, const RefList refs,
    const float *__restrict__ scores, const uint16_t *__restrict__ h, int k,
    uint16_t *__restrict__ out, float *__restrict__ out32) {
  using LY = DownLds<D, F, SG, RSTEPS>;
  constexpr int U = LY::U;
  constexpr int CPL = (U + SG - 1) / SG;
  constexpr int RPS = LY::RPS;
  constexpr int ROWS_WG = LY::ROWS_WG;
  constexpr int WG_PER_TOK = D / ROWS_WG;
  constexpr int NG = LY::NG;
  constexpr int NP = PBIAS ? 4 : 3;
  constexpr int SB_U4 = LY::SB_U4;
  constexpr int HU4 = F / 8;
  static_assert(D % ROWS_WG == 0, "rows per workgroup must divide d_model");
  static_assert((ROWS_WG * NG * 2) % 16 == 0, "scale block must be 16-byte pieces");

  extern __shared__ uint4 dyn_lds[];
  const int t = blockIdx.x / WG_PER_TOK;
  const int rb = blockIdx.x % WG_PER_TOK;
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int rsub = lane / SG, j = lane % SG;
  // wave-uniform: the slot's addresses resolve in scalar registers
  const int pair = __builtin_amdgcn_readfirstlane(t * k + wave);
  const int32_t ref = __builtin_amdgcn_readfirstlane(refs[pair]);
  const float score = scores[pair];
  const int row0 = rb * ROWS_WG;

  char *wbase = reinterpret_cast<char *>(dyn_lds) + (size_t)wave * LY::WAVE_BYTES;
  uint4 *act_l = reinterpret_cast<uint4 *>(wbase);
  float *asum_l = reinterpret_cast<float *>(wbase + LY::ACT_BYTES);
  uint4 *sb_l = reinterpret_cast<uint4 *>(wbase + LY::ACT_BYTES + LY::SUM_BYTES);
  float *red = reinterpret_cast<float *>(reinterpret_cast<char *>(dyn_lds) +
                                         (size_t)k * LY::WAVE_BYTES);

  // an out-of-range ref reads slot 0, flags the error and contributes 0
  bool ok;
  const char *dw = resolve_safe(pa, comp_index(PROJ_DOWN, PART_W, NP), ref, ok);
  const char *sp = resolve_safe(pa, comp_index(PROJ_DOWN, PART_S, NP), ref, ok);
  const char *bp = resolve_safe(pa, comp_index(PROJ_DOWN, PART_B, NP), ref, ok);
  if (!ok && lane == 0) flag_error();
  // small loads first (h of this expert, the rows' scales/biases), then the
  // code stream; staging then waits only for the former.  No branch around
  // any load and every lane loads (indices clamped, surplus lanes ignored
  // later): a conditional load would be waited for before the code stream.
  constexpr int HIT = (HU4 + 63) / 64;
  constexpr int SIT = (2 * SB_U4 + 63) / 64;
  uint4 hr[HIT], sr[SIT], cd[RSTEPS][CPL];
  const uint4 *h4 = reinterpret_cast<const uint4 *>(h + (int64_t)pair * F);
#pragma unroll
  for (int it = 0; it < HIT; ++it) hr[it] = load16(h4 + min(it * 64 + lane, HU4 - 1));
#pragma unroll
  for (int it = 0; it < SIT; ++it) {
    const int i = min(it * 64 + lane, 2 * SB_U4 - 1);
    const int p = i / SB_U4, o = i % SB_U4;
    sr[it] = load16(reinterpret_cast<const uint4 *>((p ? bp : sp) + (int64_t)row0 * NG * 2) + o);
  }
  float dbv[RSTEPS];
#pragma unroll
  for (int s = 0; s < RSTEPS; ++s) dbv[s] = 0.f;
  if (PBIAS) {
    bool okb;
    const uint16_t *dbias = reinterpret_cast<const uint16_t *>(
        resolve_safe(pa, comp_index(PROJ_DOWN, PART_BIAS, NP), ref, okb));
#pragma unroll
    for (int s = 0; s < RSTEPS; ++s) dbv[s] = bf16_to_f32(dbias[row0 + s * RPS + rsub]);
  }
  issue_order_fence();
#pragma unroll
  for (int s = 0; s < RSTEPS; ++s) {
    const int row = row0 + s * RPS + rsub;
    const uint4 *d4 = reinterpret_cast<const uint4 *>(dw + (int64_t)row * (F / 2));
#pragma unroll
    for (int i = 0; i < CPL; ++i)   // surplus chunks (c >= U) re-read the last one, unused
      cd[s][i] = load_stream16(d4 + min(i * SG + j, U - 1));
  }
  issue_order_fence();
#pragma unroll
  for (int it = 0; it < SIT; ++it) {
    const int i = it * 64 + lane;
    if (i < 2 * SB_U4) sb_l[i] = sr[it];
  }
#pragma unroll
  for (int it = 0; it < HIT; ++it) {
    const int i = it * 64 + lane;
    float s = 0.f;
    if (i < HU4) s = stage_piece<U>(act_l, i, hr[it]);
    s += dpp_f<kDppQuadXor1>(s);
    s += dpp_f<kDppQuadXor2>(s);
    if (i < HU4 && (i & 3) == 0) asum_l[i >> 2] = s;
  }
  __syncthreads();

  const uint16_t *sbh = reinterpret_cast<const uint16_t *>(sb_l);
  constexpr int SBN = SB_U4 * 8;
#pragma unroll
  for (int s = 0; s < RSTEPS; ++s) {
    const int rl = s * RPS + rsub;
    float p = 0.f;
#pragma unroll
    for (int i = 0; i < CPL; ++i) {
      const int c = i * SG + j;
      if (CPL * SG == U || c < U) {
        const int g = rl * NG + (c >> 1);
        const float Sd = bf16_to_f32(sbh[g]), Bd = bf16_to_f32(sbh[SBN + g]);
        p += Sd * chunk_dot_lds<U>(cd[s][i], act_l, c) + (Bd - 128.f * Sd) * asum_l[c];
      }
    }
    p = group_sum<SG>(p);
    if (j == 0) red[wave * ROWS_WG + rl] = ok ? score * (p + dbv[s]) : 0.f;
  }
  __syncthreads();
  for (int r = threadIdx.x; r < ROWS_WG; r += blockDim.x) {
    float y = 0.f;
    for (int w = 0; w < k; ++w) y += red[w * ROWS_WG + r];  // expert order
    const int64_t o = (int64_t)t * D + row0 + r;
    if (out) out[o] = (uint16_t)f32_to_bf16(y);
    if (out32) out32[o] = y;
  }
}

// ---------------------------------------------------------------------------
// Small-T grouped variants (2 <= T, T*k <= kSmallMaxPairs): the T*k routed
// pairs are grouped by slot reference, so each distinct expert's codes are
// read once per call and applied to every token routed to it (a speculative
// verification of T = gamma+1 tokens routes many of its tokens to the same
// hot experts).  Each (pair, row) dot product is computed exactly as in the
// per-pair kernels above (same lane split and summation order), so results
// are bit-identical to them.
// ---------------------------------------------------------------------------

// gate/up: workgroup (pair p, row block).  The workgroup of the FIRST pair
// of each slot reference computes that slot's rows for all pairs sharing it
// (its members), tokens staged MB at a time; the others exit at once.
template <int D, int F, int SG, int WAVES, int RSTEPS, bool PBIAS>
__global__ __launch_bounds__(WAVES * 64) void ffn_gate_up_small_kernel(
    PoolArgs pa, const int32_t *__restrict__ refs, int P, const uint16_t *__restrict__ x,
    int k, uint16_t *__restrict__ h, int act, float alpha, float limit) {
  constexpr int U = D / 32, CPL = (U + SG - 1) / SG, RPS = 64 / SG;
  constexpr int ROWS_WG = WAVES * RSTEPS * RPS, WG_PER_PAIR = F / ROWS_WG;
  constexpr int NG = D / 64, NP = PBIAS ? 4 : 3, NT = WAVES * 64, XU4 = D / 8;
  constexpr int SB_U4 = ROWS_WG * NG * 2 / 16;
  constexpr int MB = kSmallTokensPerPass;
  constexpr int XIT = (XU4 + NT - 1) / NT, SIT = (4 * SB_U4 + NT - 1) / NT;
  static_assert(F % ROWS_WG == 0 && (ROWS_WG * NG * 2) % 16 == 0, "row blocks");

  __shared__ uint4 act_l[MB][4 * U];
  __shared__ float asum_l[MB][U];
  __shared__ uint4 sb_l[4][SB_U4];
  __shared__ uint64_t eq_l[kSmallMaxPairs / 64];
  __shared__ int mem_l[kSmallMaxPairs];

  const int pair = blockIdx.x / WG_PER_PAIR, rb = blockIdx.x % WG_PER_PAIR;
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int rsub = lane / SG, j = lane % SG;
  const int row0 = rb * ROWS_WG;
  const int32_t ref = __builtin_amdgcn_readfirstlane(refs[pair]);
  // 1. the pairs sharing this slot reference, in pair order
  for (int w = wave; w < kSmallMaxPairs / 64; w += WAVES) {
    const int i = 64 * w + lane;
    const uint64_t b = __ballot(i < P && refs[min(i, P - 1)] == ref);
    if (lane == 0) eq_l[w] = b;
  }
  __syncthreads();
  int first = -1, nm = 0;
#pragma unroll
  for (int w = 0; w < kSmallMaxPairs / 64; ++w) {
    const uint64_t b = eq_l[w];
    if (first < 0 && b) first = 64 * w + (int)__builtin_ctzll(b);
    nm += __popcll(b);
  }
  if (first != pair) return;        // another workgroup serves this slot (uniform)
  for (int i = tid; i < P; i += NT) {
    const uint64_t b = eq_l[i >> 6];
    if ((b >> (i & 63)) & 1) {
      int pos = __popcll(b & ((i & 63) ? (~0ull >> (64 - (i & 63))) : 0ull));
      for (int w = 0; w < (i >> 6); ++w) pos += __popcll(eq_l[w]);
      mem_l[pos] = i;
    }
  }
  const char *gw = resolve(pa, comp_index(PROJ_GATE, PART_W, NP), ref);
  if (gw == nullptr) {   // uniform: zeros for every member, the error flagged
    __syncthreads();
    if (tid == 0) flag_error();
    for (int i = tid; i < nm * ROWS_WG; i += NT)
      h[(int64_t)mem_l[i / ROWS_WG] * F + row0 + i % ROWS_WG] = 0;
    return;
  }
  const char *uw = resolve(pa, comp_index(PROJ_UP, PART_W, NP), ref);
  __syncthreads();   // mem_l complete
  // 2. small loads first (the first pass's activations, the rows' scales and
  //    projection biases), then every code load (as the per-pair kernel)
  uint4 xr[MB][XIT], sr[SIT];
  auto load_x = [&](int b0) {
#pragma unroll
    for (int b = 0; b < MB; ++b) {
      const int q = mem_l[min(b0 + b, nm - 1)];   // clamped: unconditional loads
      const uint4 *x4 = reinterpret_cast<const uint4 *>(x + (int64_t)(q / k) * D);
#pragma unroll
      for (int it = 0; it < XIT; ++it) xr[b][it] = load16(x4 + min(it * NT + tid, XU4 - 1));
    }
  };
  load_x(0);
  {
    const char *gs = resolve(pa, comp_index(PROJ_GATE, PART_S, NP), ref);
    const char *gb = resolve(pa, comp_index(PROJ_GATE, PART_B, NP), ref);
    const char *us = resolve(pa, comp_index(PROJ_UP, PART_S, NP), ref);
    const char *ub = resolve(pa, comp_index(PROJ_UP, PART_B, NP), ref);
#pragma unroll
    for (int it = 0; it < SIT; ++it) {
      const int i = min(it * NT + tid, 4 * SB_U4 - 1);
      const int p = i / SB_U4, o = i % SB_U4;
      const char *sp = p == 0 ? gs : p == 1 ? gb : p == 2 ? us : ub;
      sr[it] = load16(reinterpret_cast<const uint4 *>(sp + (int64_t)row0 * NG * 2) + o);
    }
  }
  float gbv[RSTEPS], ubv[RSTEPS];
#pragma unroll
  for (int st = 0; st < RSTEPS; ++st) gbv[st] = ubv[st] = 0.f;
  if (PBIAS) {
    const uint16_t *gbias = reinterpret_cast<const uint16_t *>(
        resolve(pa, comp_index(PROJ_GATE, PART_BIAS, NP), ref));
    const uint16_t *ubias = reinterpret_cast<const uint16_t *>(
        resolve(pa, comp_index(PROJ_UP, PART_BIAS, NP), ref));
#pragma unroll
    for (int st = 0; st < RSTEPS; ++st) {
      const int row = row0 + (wave * RSTEPS + st) * RPS + rsub;
      gbv[st] = bf16_to_f32(gbias[row]);
      ubv[st] = bf16_to_f32(ubias[row]);
    }
  }
  issue_order_fence();
  uint4 cg[RSTEPS][CPL], cu[RSTEPS][CPL];
#pragma unroll
  for (int st = 0; st < RSTEPS; ++st) {
    const int row = row0 + (wave * RSTEPS + st) * RPS + rsub;
    const uint4 *g4 = reinterpret_cast<const uint4 *>(gw + (int64_t)row * (D / 2));
    const uint4 *u4 = reinterpret_cast<const uint4 *>(uw + (int64_t)row * (D / 2));
#pragma unroll
    for (int i = 0; i < CPL; ++i) {
      const int c = min(i * SG + j, U - 1);
      cg[st][i] = load_stream16(g4 + c);
      cu[st][i] = load_stream16(u4 + c);
    }
  }
  issue_order_fence();
#pragma unroll
  for (int it = 0; it < SIT; ++it) {
    const int i = it * NT + tid;
    if (i < 4 * SB_U4) (&sb_l[0][0])[i] = sr[it];
  }
  const uint16_t *sbh = reinterpret_cast<const uint16_t *>(&sb_l[0][0]);
  constexpr int SBN = SB_U4 * 8;
  // 3. passes of up to MB member tokens: stage, then every row for each
  for (int b0 = 0; b0 < nm; b0 += MB) {
    if (b0 > 0) {
      __syncthreads();   // the previous pass's reads of act_l are done
      load_x(b0);
    }
#pragma unroll
    for (int b = 0; b < MB; ++b) {
#pragma unroll
      for (int it = 0; it < XIT; ++it) {
        const int i = it * NT + tid;
        float sm = 0.f;
        if (i < XU4) sm = stage_piece<U>(act_l[b], i, xr[b][it]);
        sm += dpp_f<kDppQuadXor1>(sm);
        sm += dpp_f<kDppQuadXor2>(sm);
        if (i < XU4 && (i & 3) == 0) asum_l[b][i >> 2] = sm;
      }
    }
    __syncthreads();
    const int nb = min(MB, nm - b0);
#pragma unroll
    for (int st = 0; st < RSTEPS; ++st) {
      const int rl = (wave * RSTEPS + st) * RPS + rsub;
      // chunk by chunk: the codes decoded once, then applied to every token
      // of the pass (per token the same sums in the same order as above)
      float pg[MB], pu[MB];
#pragma unroll
      for (int b = 0; b < MB; ++b) pg[b] = pu[b] = 0.f;
#pragma unroll
      for (int i = 0; i < CPL; ++i) {
        const int c = i * SG + j;
        if (CPL * SG == U || c < U) {
          const int g = rl * NG + (c >> 1);
          const float Sg = bf16_to_f32(sbh[0 * SBN + g]), Bg = bf16_to_f32(sbh[1 * SBN + g]);
          const float Su = bf16_to_f32(sbh[2 * SBN + g]), Bu = bf16_to_f32(sbh[3 * SBN + g]);
          uint32_t dg[16], du[16];
          decode_chunk(cg[st][i], dg);
          decode_chunk(cu[st][i], du);
#pragma unroll
          for (int b = 0; b < MB; ++b) {
            if (b < nb) {
              const float xs = asum_l[b][c];
              pg[b] += Sg * chunk_dot_dec<U>(dg, act_l[b], c) + (Bg - 128.f * Sg) * xs;
              pu[b] += Su * chunk_dot_dec<U>(du, act_l[b], c) + (Bu - 128.f * Su) * xs;
            }
          }
        }
      }
#pragma unroll
      for (int b = 0; b < MB; ++b) {
        if (b < nb) {
          float g2 = group_sum<SG>(pg[b]), u2 = group_sum<SG>(pu[b]);
          if (j == 0) {
            g2 += gbv[st];
            u2 += ubv[st];
            h[(int64_t)mem_l[b0 + b] * F + row0 + rl] =
                (uint16_t)f32_to_bf16(apply_act(act, g2, u2, alpha, limit));
          }
        }
      }
    }
  }
}

// down + weighted combine: workgroup = one block of output rows, NW waves.
// Wave w takes the slot references r with r mod NW == w; for each of them it
// loads the block's rows once and applies them to every pair routed there
// (each pair's h staged in the wave's LDS in turn), writing the pair's
// score-weighted rows; then the rows of each token are summed over its k
// pairs in rank order (as the per-pair kernel sums over its waves).
template <int D, int F, int SG, int RSTEPS, int NW>
struct SmallDownLds {
  using W = DownLds<D, F, SG, RSTEPS>;
  static constexpr size_t bytes(int P) {
    return (size_t)NW * W::WAVE_BYTES + (size_t)P * W::ROWS_WG * 4;
  }
};

template <int D, int F, int SG, int RSTEPS, bool PBIAS, int NW>
__global__ __launch_bounds__(NW * 64) void ffn_down_small_kernel(
    PoolArgs pa, const int32_t *__restrict__ refs, const float *__restrict__ scores,
    const uint16_t *__restrict__ h, int P, int k, uint16_t *__restrict__ out,
    float *__restrict__ out32) {
  using LY = DownLds<D, F, SG, RSTEPS>;
  constexpr int U = LY::U, CPL = (U + SG - 1) / SG, RPS = LY::RPS, ROWS_WG = LY::ROWS_WG;
  constexpr int NG = LY::NG, NP = PBIAS ? 4 : 3, SB_U4 = LY::SB_U4, HU4 = F / 8;
  constexpr int HIT = (HU4 + 63) / 64, SIT = (2 * SB_U4 + 63) / 64;
  constexpr int NC = kSmallMaxPairs / 64;
  constexpr int MBD = HIT <= 2 ? 4 : HIT <= 4 ? 2 : 1;   // member activations loaded together
  extern __shared__ uint4 dyn_lds[];
  const int rb = blockIdx.x, row0 = rb * ROWS_WG;
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int rsub = lane / SG, j = lane % SG;
  char *wbase = reinterpret_cast<char *>(dyn_lds) + (size_t)wave * LY::WAVE_BYTES;
  uint4 *act_l = reinterpret_cast<uint4 *>(wbase);
  float *asum_l = reinterpret_cast<float *>(wbase + LY::ACT_BYTES);
  uint4 *sb_l = reinterpret_cast<uint4 *>(wbase + LY::ACT_BYTES + LY::SUM_BYTES);
  float *red = reinterpret_cast<float *>(reinterpret_cast<char *>(dyn_lds) +
                                         (size_t)NW * LY::WAVE_BYTES);
  // lane holds the refs of pairs lane + 64c; this wave's share of them
  int32_t r[NC];
  uint64_t rem[NC];
#pragma unroll
  for (int c = 0; c < NC; ++c) {
    const int i = lane + 64 * c;
    r[c] = refs[min(i, P - 1)];
    rem[c] = __ballot(i < P && (int)((uint32_t)r[c] % NW) == wave);
  }
  while (true) {
    // the lowest remaining pair of this wave names the next slot; its
    // members are the remaining pairs with the same reference
    int c0 = -1;
#pragma unroll
    for (int c = NC - 1; c >= 0; --c)
      if (rem[c]) c0 = c;
    if (c0 < 0) break;
    uint64_t lowc = 0;
    int32_t ref = 0;
#pragma unroll
    for (int c = 0; c < NC; ++c)
      if (c == c0) {
        lowc = rem[c];
        ref = __builtin_amdgcn_readlane(r[c], (int)__builtin_ctzll(lowc));
      }
    uint64_t mem[NC];
#pragma unroll
    for (int c = 0; c < NC; ++c) {
      mem[c] = __ballot(r[c] == ref) & rem[c];
      rem[c] &= ~mem[c];
    }
    bool ok;
    const char *dw = resolve_safe(pa, comp_index(PROJ_DOWN, PART_W, NP), ref, ok);
    const char *sp = resolve_safe(pa, comp_index(PROJ_DOWN, PART_S, NP), ref, ok);
    const char *bp = resolve_safe(pa, comp_index(PROJ_DOWN, PART_B, NP), ref, ok);
    if (!ok && lane == 0) flag_error();
    uint4 sr[SIT], cd[RSTEPS][CPL];
#pragma unroll
    for (int it = 0; it < SIT; ++it) {
      const int i = min(it * 64 + lane, 2 * SB_U4 - 1);
      const int p = i / SB_U4, o = i % SB_U4;
      sr[it] = load16(reinterpret_cast<const uint4 *>((p ? bp : sp) + (int64_t)row0 * NG * 2) + o);
    }
    float dbv[RSTEPS];
#pragma unroll
    for (int st = 0; st < RSTEPS; ++st) dbv[st] = 0.f;
    if (PBIAS) {
      bool okb;
      const uint16_t *dbias = reinterpret_cast<const uint16_t *>(
          resolve_safe(pa, comp_index(PROJ_DOWN, PART_BIAS, NP), ref, okb));
#pragma unroll
      for (int st = 0; st < RSTEPS; ++st) dbv[st] = bf16_to_f32(dbias[row0 + st * RPS + rsub]);
    }
    issue_order_fence();
#pragma unroll
    for (int st = 0; st < RSTEPS; ++st) {
      const uint4 *d4 = reinterpret_cast<const uint4 *>(dw + (int64_t)(row0 + st * RPS + rsub) * (F / 2));
#pragma unroll
      for (int i = 0; i < CPL; ++i) cd[st][i] = load_stream16(d4 + min(i * SG + j, U - 1));
    }
    issue_order_fence();
    __atomic_signal_fence(__ATOMIC_SEQ_CST);
    __builtin_amdgcn_wave_barrier();   // the previous slot's LDS reads are done
    __atomic_signal_fence(__ATOMIC_SEQ_CST);
#pragma unroll
    for (int it = 0; it < SIT; ++it) {
      const int i = it * 64 + lane;
      if (i < 2 * SB_U4) sb_l[i] = sr[it];
    }
    const uint16_t *sbh = reinterpret_cast<const uint16_t *>(sb_l);
    constexpr int SBN = SB_U4 * 8;
    // every member pair, in pair order, MBD at a time: their h loads (and
    // scores) issued together, then staged and applied one by one
    uint64_t mm[NC];
#pragma unroll
    for (int c = 0; c < NC; ++c) mm[c] = mem[c];
    while (true) {
      int qs[MBD];
#pragma unroll
      for (int b = 0; b < MBD; ++b) {
        qs[b] = -1;
#pragma unroll
        for (int c = 0; c < NC; ++c)
          if (qs[b] < 0 && mm[c]) {
            qs[b] = 64 * c + (int)__builtin_ctzll(mm[c]);
            mm[c] &= mm[c] - 1;
          }
      }
      if (qs[0] < 0) break;
      uint4 hr[MBD][HIT];
      float sc[MBD];
#pragma unroll
      for (int b = 0; b < MBD; ++b) {   // unconditional: absent members repeat the first
        const int q = qs[b] >= 0 ? qs[b] : qs[0];
        const uint4 *h4 = reinterpret_cast<const uint4 *>(h + (int64_t)q * F);
#pragma unroll
        for (int it = 0; it < HIT; ++it) hr[b][it] = load16(h4 + min(it * 64 + lane, HU4 - 1));
        sc[b] = scores[q];
      }
#pragma unroll
      for (int b = 0; b < MBD; ++b) {
        if (qs[b] < 0) break;
        const int q = qs[b];
        __atomic_signal_fence(__ATOMIC_SEQ_CST);
        __builtin_amdgcn_wave_barrier();   // the previous member's LDS reads are done
        __atomic_signal_fence(__ATOMIC_SEQ_CST);
#pragma unroll
        for (int it = 0; it < HIT; ++it) {
          const int i = it * 64 + lane;
          float sm = 0.f;
          if (i < HU4) sm = stage_piece<U>(act_l, i, hr[b][it]);
          sm += dpp_f<kDppQuadXor1>(sm);
          sm += dpp_f<kDppQuadXor2>(sm);
          if (i < HU4 && (i & 3) == 0) asum_l[i >> 2] = sm;
        }
        __atomic_signal_fence(__ATOMIC_SEQ_CST);
        __builtin_amdgcn_wave_barrier();
        __atomic_signal_fence(__ATOMIC_SEQ_CST);
#pragma unroll
        for (int st = 0; st < RSTEPS; ++st) {
          const int rl = st * RPS + rsub;
          float pv = 0.f;
#pragma unroll
          for (int i = 0; i < CPL; ++i) {
            const int cc = i * SG + j;
            if (CPL * SG == U || cc < U) {
              const int g = rl * NG + (cc >> 1);
              const float Sd = bf16_to_f32(sbh[g]), Bd = bf16_to_f32(sbh[SBN + g]);
              pv += Sd * chunk_dot_lds<U>(cd[st][i], act_l, cc) + (Bd - 128.f * Sd) * asum_l[cc];
            }
          }
          pv = group_sum<SG>(pv);
          if (j == 0) red[q * ROWS_WG + rl] = ok ? sc[b] * (pv + dbv[st]) : 0.f;
        }
      }
    }
  }
  __syncthreads();
  const int T = P / k;
  for (int i = threadIdx.x; i < T * ROWS_WG; i += NW * 64) {
    const int t = i / ROWS_WG, rr = i % ROWS_WG;
    float y = 0.f;
    for (int w = 0; w < k; ++w) y += red[(t * k + w) * ROWS_WG + rr];   // rank order
    const int64_t o = (int64_t)t * D + row0 + rr;
    if (out) out[o] = (uint16_t)f32_to_bf16(y);
    if (out32) out32[o] = y;
  }
}

// ---------------------------------------------------------------------------
// host-side dispatch over the compiled geometries
// ---------------------------------------------------------------------------
template <int D, int F, int SG, int WAVES, int RSTEPS, bool PBIAS>
static void launch_up(dim3 g, dim3 b, hipStream_t s, const PoolArgs &pa,
                      const RefList &refs, const uint16_t *x, int k,
                      uint16_t *h, int act, float alpha, float limit) {
  hipLaunchKernelGGL((ffn_gate_up_kernel<D, F, SG, WAVES, RSTEPS, PBIAS>), g, b,
                     0, s, pa, refs, x, k, h, act, alpha, limit);
}
template <int D, int F, int SG, int RSTEPS, bool PBIAS>
static void launch_down(dim3 g, dim3 b, hipStream_t s, const PoolArgs &pa,
                        const RefList &refs, const float *sc, const uint16_t *h,
                        int k, uint16_t *out, float *out32) {
  const size_t lds = DownLds<D, F, SG, RSTEPS>::bytes(k);
  hipLaunchKernelGGL((ffn_down_kernel<D, F, SG, RSTEPS, PBIAS>), g, b, lds, s,
                     pa, refs, sc, h, k, out, out32);
}

template <int D, int F, int SG, int RSTEPS>
static size_t down_lds_bytes(int k) {
  return DownLds<D, F, SG, RSTEPS>::bytes(k);
}

template <int D, int F, int SG, int WAVES, int RSTEPS, bool PBIAS>
static void launch_up_small(dim3 g, dim3 b, hipStream_t s, const PoolArgs &pa,
                            const int32_t *refs, int P, const uint16_t *x, int k, uint16_t *h,
                            int act, float alpha, float limit) {
  hipLaunchKernelGGL((ffn_gate_up_small_kernel<D, F, SG, WAVES, RSTEPS, PBIAS>), g, b, 0, s,
                     pa, refs, P, x, k, h, act, alpha, limit);
}
template <int D, int F, int SG, int RSTEPS, bool PBIAS, int NW>
static void launch_down_small(dim3 g, dim3 b, size_t lds, hipStream_t s, const PoolArgs &pa,
                              const int32_t *refs, const float *sc, const uint16_t *h, int P,
                              int k, uint16_t *out, float *out32) {
  hipLaunchKernelGGL((ffn_down_small_kernel<D, F, SG, RSTEPS, PBIAS, NW>), g, b, lds, s, pa,
                     refs, sc, h, P, k, out, out32);
}
template <int D, int F, int SG, int RSTEPS, int NW>
static size_t down_small_lds_bytes(int P) {
  return SmallDownLds<D, F, SG, RSTEPS, NW>::bytes(P);
}

#define MOE_FFN_GEOM(D, F, PB, SGU, WU, RU, SGD, RD, NWS)                    \
  {D, F, PB, (WU) * (RU) * (64 / (SGU)), (WU) * 64, (RD) * (64 / (SGD)), NWS, \
   &launch_up<D, F, SGU, WU, RU, PB>, &launch_down<D, F, SGD, RD, PB>,       \
   &down_lds_bytes<D, F, SGD, RD>,                                           \
   &launch_up_small<D, F, SGU, WU, RU, PB>,                                  \
   &launch_down_small<D, F, SGD, RD, PB, NWS>,                               \
   &down_small_lds_bytes<D, F, SGD, RD, NWS>}

// d_model, d_ff, proj bias | gate/up: SG, waves, row steps | down: SG, steps
// | grouped down: waves
static const FfnLaunch kFfnTable[] = {
    // Launch shapes from a sweep on MI355X (kernel time, rotating slots).
    // Qwen3-30B-A3B: 24 rows per workgroup -> 8 experts x 32 = 256 WGs.  Its
    // lane split (16 lanes per row, 4 chunks each) is the persistent
    // kernel's, so both paths sum every row in the same order and produce
    // identical bits (8 rows of 32 lanes measured 6.1 vs 7.0 us but would
    // break that).  gpt-oss: gate/up 8 rows 9.9 vs 10.3 us, down 8 rows of
    // 16 lanes 8.7 vs 9.1 us.
    MOE_FFN_GEOM(2048, 768, false, 16, 6, 1, 8, 1, 16),
    MOE_FFN_GEOM(2048, 768, true, 16, 6, 1, 8, 1, 16),
    MOE_FFN_GEOM(2880, 2880, true, 32, 4, 1, 16, 2, 6),  // gpt-oss-120b
    MOE_FFN_GEOM(2880, 2880, false, 32, 4, 1, 16, 2, 6),
    MOE_FFN_GEOM(256, 128, false, 8, 2, 1, 4, 1, 8),     // small test geometry
    MOE_FFN_GEOM(256, 128, true, 8, 2, 1, 4, 1, 8),
};

const FfnLaunch *find_ffn(int d_model, int d_ff, int has_bias) {
  for (const auto &e : kFfnTable)
    if (e.d_model == d_model && e.d_ff == d_ff && e.has_bias == (has_bias != 0))
      return &e;
  return nullptr;
}

// The grouped small-T kernels serve 2 <= T with T*k <= kSmallMaxPairs pairs
// whose refs are a device array; one token, or refs carried in the kernel
// arguments, take the per-pair kernels (identical results either way).
bool ffn_small_grouped(const FfnLaunch *L, const RefList &refs, int T, int k) {
  return T >= 2 && T * k <= kSmallMaxPairs && refs.ptr != nullptr &&
         L->down_small_lds(T * k) <= 65536;
}

void launch_ffn_up(const FfnLaunch *L, const PoolArgs &pa, const RefList &refs,
                   const uint16_t *x, int T, int k, uint16_t *h, int act,
                   float alpha, float limit, hipStream_t s) {
  dim3 g(T * k * (L->d_ff / L->up_rows_wg)), b(L->up_threads);
  if (ffn_small_grouped(L, refs, T, k))
    L->up_small(g, b, s, pa, refs.ptr, T * k, x, k, h, act, alpha, limit);
  else
    L->up(g, b, s, pa, refs, x, k, h, act, alpha, limit);
}

void launch_ffn_down(const FfnLaunch *L, const PoolArgs &pa,
                     const RefList &refs, const float *scores, int T, int k,
                     const uint16_t *h, uint16_t *out, float *out32,
                     hipStream_t s) {
  if (ffn_small_grouped(L, refs, T, k)) {
    dim3 g(L->d_model / L->down_rows_wg), b(64 * L->down_small_waves);
    L->down_small(g, b, L->down_small_lds(T * k), s, pa, refs.ptr, scores, h, T * k, k, out,
                  out32);
    return;
  }
  dim3 g(T * (L->d_model / L->down_rows_wg)), b(64 * k);
  L->down(g, b, s, pa, refs, scores, h, k, out, out32);
}

void launch_ffn_decode(const FfnLaunch *L, const PoolArgs &pa,
                       const RefList &refs, const float *scores,
                       const uint16_t *x, int T, int k, uint16_t *h,
                       uint16_t *out, float *out32, int act, float alpha,
                       float limit, hipStream_t s) {
  launch_ffn_up(L, pa, refs, x, T, k, h, act, alpha, limit, s);
  launch_ffn_down(L, pa, refs, scores, T, k, h, out, out32, s);
}

}  // namespace moe
