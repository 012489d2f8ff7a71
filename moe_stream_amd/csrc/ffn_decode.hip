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
// 64/SG rows with SG*16 contiguous bytes each.  A lane always sees the same
// input chunks, so the activations it needs sit in registers, already in
// the pair order of the decoded codes, for the whole kernel.  Row sums are an
// SG-lane butterfly.  All code loads of a lane are issued before any math.
#include "launchers.h"

namespace moe {

__device__ int g_device_error = 0;

template <int CPL, int SG, int U>
__device__ __forceinline__ void load_act_chunks(const uint16_t *__restrict__ v,
                                                int j, uint32_t (&xp)[CPL][16],
                                                float (&xs)[CPL]) {
  const uint4 *v4 = reinterpret_cast<const uint4 *>(v);
#pragma unroll
  for (int i = 0; i < CPL; ++i) {
    const int c = i * SG + j;
    xs[i] = 0.f;
    if (CPL * SG == U || c < U) {
#pragma unroll
      for (int q = 0; q < 4; ++q) {  // 8 activations per uint4
        uint4 a = v4[c * 4 + q];
        uint32_t in[4] = {a.x, a.y, a.z, a.w};
        uint32_t out[4];
        x_pairs(in, out);
#pragma unroll
        for (int m = 0; m < 4; ++m) xp[i][q * 4 + m] = out[m];
#pragma unroll
        for (int m = 0; m < 4; ++m)
          xs[i] += bf16_to_f32(in[m] & 0xffffu) + bf16_to_f32(in[m] >> 16);
      }
    } else {
#pragma unroll
      for (int m = 0; m < 16; ++m) xp[i][m] = 0u;
    }
  }
}

// sum((128+q)*x) over one 16-byte chunk of codes (32 inputs).
__device__ __forceinline__ float chunk_dot(const uint4 &c, const uint32_t *xp) {
  float acc = 0.f;
  const uint32_t w[4] = {c.x, c.y, c.z, c.w};
#pragma unroll
  for (int q = 0; q < 4; ++q) {
    uint32_t p[4];
    codes_to_bf16x2(w[q], p);
#pragma unroll
    for (int m = 0; m < 4; ++m) acc = dot2_bf16(p[m], xp[q * 4 + m], acc);
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
    PoolArgs pa, const int32_t *__restrict__ refs,
    const uint16_t *__restrict__ x, int k, uint16_t *__restrict__ h, int act,
    float alpha, float limit) {
  constexpr int U = D / 32;                 // 16-byte code chunks per row
  constexpr int CPL = (U + SG - 1) / SG;    // chunks per lane
  constexpr int RPS = 64 / SG;              // rows per wave step
  constexpr int ROWS_WG = WAVES * RSTEPS * RPS;
  constexpr int WG_PER_PAIR = F / ROWS_WG;
  constexpr int NG = D / 64;                // quant groups per row
  constexpr int NP = PBIAS ? 4 : 3;
  static_assert(F % ROWS_WG == 0, "rows per workgroup must divide d_ff");

  const int pair = blockIdx.x / WG_PER_PAIR;
  const int rb = blockIdx.x % WG_PER_PAIR;
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int rsub = lane / SG, j = lane % SG;
  const int t = pair / k;
  const int32_t ref = refs[pair];

  const char *gw = resolve(pa, comp_index(PROJ_GATE, PART_W, NP), ref);
  const char *uw = resolve(pa, comp_index(PROJ_UP, PART_W, NP), ref);
  const char *gsc = resolve(pa, comp_index(PROJ_GATE, PART_S, NP), ref);
  const char *usc = resolve(pa, comp_index(PROJ_UP, PART_S, NP), ref);
  const char *gbi = resolve(pa, comp_index(PROJ_GATE, PART_B, NP), ref);
  const char *ubi = resolve(pa, comp_index(PROJ_UP, PART_B, NP), ref);
  if (gw == nullptr) {  // uniform over the workgroup
    if (threadIdx.x == 0) flag_error();
#pragma unroll
    for (int s = 0; s < RSTEPS; ++s) {
      const int row = rb * ROWS_WG + (wave * RSTEPS + s) * RPS + rsub;
      if (j == 0) h[(int64_t)pair * F + row] = 0;
    }
    return;
  }

  // 1. issue every code load of this lane
  uint4 cg[RSTEPS][CPL], cu[RSTEPS][CPL];
#pragma unroll
  for (int s = 0; s < RSTEPS; ++s) {
    const int row = rb * ROWS_WG + (wave * RSTEPS + s) * RPS + rsub;
    const uint4 *g4 = reinterpret_cast<const uint4 *>(gw + (int64_t)row * (D / 2));
    const uint4 *u4 = reinterpret_cast<const uint4 *>(uw + (int64_t)row * (D / 2));
#pragma unroll
    for (int i = 0; i < CPL; ++i) {
      const int c = i * SG + j;
      if (CPL * SG == U || c < U) {
        cg[s][i] = load_stream16(g4 + c);
        cu[s][i] = load_stream16(u4 + c);
      } else {
        cg[s][i] = make_uint4(0, 0, 0, 0);
        cu[s][i] = make_uint4(0, 0, 0, 0);
      }
    }
  }
  // 2. scales and biases of the groups this lane touches
  uint16_t sg_[RSTEPS][CPL], bg_[RSTEPS][CPL], su_[RSTEPS][CPL], bu_[RSTEPS][CPL];
#pragma unroll
  for (int s = 0; s < RSTEPS; ++s) {
    const int row = rb * ROWS_WG + (wave * RSTEPS + s) * RPS + rsub;
    const uint16_t *gS = reinterpret_cast<const uint16_t *>(gsc) + row * NG;
    const uint16_t *uS = reinterpret_cast<const uint16_t *>(usc) + row * NG;
    const uint16_t *gB = reinterpret_cast<const uint16_t *>(gbi) + row * NG;
    const uint16_t *uB = reinterpret_cast<const uint16_t *>(ubi) + row * NG;
#pragma unroll
    for (int i = 0; i < CPL; ++i) {
      const int c = i * SG + j;
      const int g = (CPL * SG == U || c < U) ? c / 2 : 0;
      sg_[s][i] = gS[g];
      bg_[s][i] = gB[g];
      su_[s][i] = uS[g];
      bu_[s][i] = uB[g];
    }
  }
  // 3. activations of this token, in registers
  uint32_t xp[CPL][16];
  float xs[CPL];
  load_act_chunks<CPL, SG, U>(x + (int64_t)t * D, j, xp, xs);

  // 4. dot products, row sums, activation
#pragma unroll
  for (int s = 0; s < RSTEPS; ++s) {
    float pg = 0.f, pu = 0.f;
#pragma unroll
    for (int i = 0; i < CPL; ++i) {
      const int c = i * SG + j;
      if (CPL * SG == U || c < U) {
        const float Sg = bf16_to_f32(sg_[s][i]), Bg = bf16_to_f32(bg_[s][i]);
        const float Su = bf16_to_f32(su_[s][i]), Bu = bf16_to_f32(bu_[s][i]);
        pg += Sg * chunk_dot(cg[s][i], xp[i]) + (Bg - 128.f * Sg) * xs[i];
        pu += Su * chunk_dot(cu[s][i], xp[i]) + (Bu - 128.f * Su) * xs[i];
      }
    }
    pg = group_sum<SG>(pg);
    pu = group_sum<SG>(pu);
    if (j == 0) {
      const int row = rb * ROWS_WG + (wave * RSTEPS + s) * RPS + rsub;
      if (PBIAS) {
        const uint16_t *gbias = reinterpret_cast<const uint16_t *>(
            resolve(pa, comp_index(PROJ_GATE, PART_BIAS, NP), ref));
        const uint16_t *ubias = reinterpret_cast<const uint16_t *>(
            resolve(pa, comp_index(PROJ_UP, PART_BIAS, NP), ref));
        pg += bf16_to_f32(gbias[row]);
        pu += bf16_to_f32(ubias[row]);
      }
      h[(int64_t)pair * F + row] = (uint16_t)f32_to_bf16(apply_act(act, pg, pu, alpha, limit));
    }
  }
}

// ---------------------------------------------------------------------------
// down + weighted combine; one wave per routed expert, blockDim = 64*k
// ---------------------------------------------------------------------------
template <int D, int F, int SG, int RSTEPS, bool PBIAS>
__global__ __launch_bounds__(64 * MOE_MAX_TOPK) void ffn_down_kernel(
    PoolArgs pa, const int32_t *__restrict__ refs,
    const float *__restrict__ scores, const uint16_t *__restrict__ h, int k,
    uint16_t *__restrict__ out, float *__restrict__ out32) {
  constexpr int U = F / 32;
  constexpr int CPL = (U + SG - 1) / SG;
  constexpr int RPS = 64 / SG;
  constexpr int ROWS_WG = RSTEPS * RPS;
  constexpr int WG_PER_TOK = D / ROWS_WG;
  constexpr int NG = F / 64;
  constexpr int NP = PBIAS ? 4 : 3;
  static_assert(D % ROWS_WG == 0, "rows per workgroup must divide d_model");

  __shared__ float red[MOE_MAX_TOPK][ROWS_WG];

  const int t = blockIdx.x / WG_PER_TOK;
  const int rb = blockIdx.x % WG_PER_TOK;
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int rsub = lane / SG, j = lane % SG;
  const int pair = t * k + wave;
  const int32_t ref = refs[pair];
  const float score = scores[pair];

  const char *dw = resolve(pa, comp_index(PROJ_DOWN, PART_W, NP), ref);
  if (dw != nullptr) {
    const char *dsc = resolve(pa, comp_index(PROJ_DOWN, PART_S, NP), ref);
    const char *dbi = resolve(pa, comp_index(PROJ_DOWN, PART_B, NP), ref);
    uint4 cd[RSTEPS][CPL];
    uint16_t sd[RSTEPS][CPL], bd[RSTEPS][CPL];
#pragma unroll
    for (int s = 0; s < RSTEPS; ++s) {
      const int row = rb * ROWS_WG + s * RPS + rsub;
      const uint4 *d4 = reinterpret_cast<const uint4 *>(dw + (int64_t)row * (F / 2));
#pragma unroll
      for (int i = 0; i < CPL; ++i) {
        const int c = i * SG + j;
        cd[s][i] = (CPL * SG == U || c < U) ? load_stream16(d4 + c)
                                            : make_uint4(0, 0, 0, 0);
      }
    }
#pragma unroll
    for (int s = 0; s < RSTEPS; ++s) {
      const int row = rb * ROWS_WG + s * RPS + rsub;
      const uint16_t *S = reinterpret_cast<const uint16_t *>(dsc) + row * NG;
      const uint16_t *B = reinterpret_cast<const uint16_t *>(dbi) + row * NG;
#pragma unroll
      for (int i = 0; i < CPL; ++i) {
        const int c = i * SG + j;
        const int g = (CPL * SG == U || c < U) ? c / 2 : 0;
        sd[s][i] = S[g];
        bd[s][i] = B[g];
      }
    }
    uint32_t hp[CPL][16];
    float hs[CPL];
    load_act_chunks<CPL, SG, U>(h + (int64_t)pair * F, j, hp, hs);
#pragma unroll
    for (int s = 0; s < RSTEPS; ++s) {
      float p = 0.f;
#pragma unroll
      for (int i = 0; i < CPL; ++i) {
        const int c = i * SG + j;
        if (CPL * SG == U || c < U) {
          const float Sd = bf16_to_f32(sd[s][i]), Bd = bf16_to_f32(bd[s][i]);
          p += Sd * chunk_dot(cd[s][i], hp[i]) + (Bd - 128.f * Sd) * hs[i];
        }
      }
      p = group_sum<SG>(p);
      if (j == 0) {
        const int row = rb * ROWS_WG + s * RPS + rsub;
        if (PBIAS) {
          const uint16_t *dbias = reinterpret_cast<const uint16_t *>(
              resolve(pa, comp_index(PROJ_DOWN, PART_BIAS, NP), ref));
          p += bf16_to_f32(dbias[row]);
        }
        red[wave][s * RPS + rsub] = score * p;
      }
    }
  } else {
    if (lane == 0) flag_error();
    for (int i = lane; i < ROWS_WG; i += 64) red[wave][i] = 0.f;
  }
  __syncthreads();
  for (int r = threadIdx.x; r < ROWS_WG; r += blockDim.x) {
    float y = 0.f;
    for (int w = 0; w < k; ++w) y += red[w][r];  // expert order: deterministic
    const int64_t o = (int64_t)t * D + rb * ROWS_WG + r;
    if (out) out[o] = (uint16_t)f32_to_bf16(y);
    if (out32) out32[o] = y;
  }
}

// ---------------------------------------------------------------------------
// host-side dispatch over the compiled geometries
// ---------------------------------------------------------------------------

template <int D, int F, int SG, int WAVES, int RSTEPS, bool PBIAS>
static void launch_up(dim3 g, dim3 b, hipStream_t s, const PoolArgs &pa,
                      const int32_t *refs, const uint16_t *x, int k,
                      uint16_t *h, int act, float alpha, float limit) {
  hipLaunchKernelGGL((ffn_gate_up_kernel<D, F, SG, WAVES, RSTEPS, PBIAS>), g, b,
                     0, s, pa, refs, x, k, h, act, alpha, limit);
}
template <int D, int F, int SG, int RSTEPS, bool PBIAS>
static void launch_down(dim3 g, dim3 b, hipStream_t s, const PoolArgs &pa,
                        const int32_t *refs, const float *sc, const uint16_t *h,
                        int k, uint16_t *out, float *out32) {
  hipLaunchKernelGGL((ffn_down_kernel<D, F, SG, RSTEPS, PBIAS>), g, b, 0, s, pa,
                     refs, sc, h, k, out, out32);
}

#define MOE_FFN_GEOM(D, F, PB, SGU, WU, RU, SGD, RD)                         \
  {D, F, PB, (WU) * (RU) * (64 / (SGU)), (WU) * 64, (RD) * (64 / (SGD)),     \
   &launch_up<D, F, SGU, WU, RU, PB>, &launch_down<D, F, SGD, RD, PB>}

// d_model, d_ff, proj bias | gate/up: SG, waves, row steps | down: SG, steps
static const FfnLaunch kFfnTable[] = {
    MOE_FFN_GEOM(2048, 768, false, 16, 4, 1, 8, 1),   // Qwen3-30B-A3B
    MOE_FFN_GEOM(2048, 768, true, 16, 4, 1, 8, 1),
    MOE_FFN_GEOM(2880, 2880, true, 32, 4, 2, 32, 4),  // gpt-oss-120b
    MOE_FFN_GEOM(2880, 2880, false, 32, 4, 2, 32, 4),
    MOE_FFN_GEOM(256, 128, false, 8, 2, 1, 4, 1),     // small test geometry
    MOE_FFN_GEOM(256, 128, true, 8, 2, 1, 4, 1),
};

const FfnLaunch *find_ffn(int d_model, int d_ff, int has_bias) {
  for (const auto &e : kFfnTable)
    if (e.d_model == d_model && e.d_ff == d_ff && e.has_bias == (has_bias != 0))
      return &e;
  return nullptr;
}

void launch_ffn_up(const FfnLaunch *L, const PoolArgs &pa, const int32_t *refs,
                   const uint16_t *x, int T, int k, uint16_t *h, int act,
                   float alpha, float limit, hipStream_t s) {
  dim3 g(T * k * (L->d_ff / L->up_rows_wg)), b(L->up_threads);
  L->up(g, b, s, pa, refs, x, k, h, act, alpha, limit);
}

void launch_ffn_down(const FfnLaunch *L, const PoolArgs &pa,
                     const int32_t *refs, const float *scores, int T, int k,
                     const uint16_t *h, uint16_t *out, float *out32,
                     hipStream_t s) {
  dim3 g(T * (L->d_model / L->down_rows_wg)), b(64 * k);
  L->down(g, b, s, pa, refs, scores, h, k, out, out32);
}

void launch_ffn_decode(const FfnLaunch *L, const PoolArgs &pa,
                       const int32_t *refs, const float *scores,
                       const uint16_t *x, int T, int k, uint16_t *h,
                       uint16_t *out, float *out32, int act, float alpha,
                       float limit, hipStream_t s) {
  launch_ffn_up(L, pa, refs, x, T, k, h, act, alpha, limit, s);
  launch_ffn_down(L, pa, refs, scores, T, k, h, out, out32, s);
}

}  // namespace moe
