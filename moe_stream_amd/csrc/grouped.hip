// Multi-token (prefill / batched) expert block for gfx950: the T*k routed
// (token, slot) pairs are grouped by slot and every group runs as a dense
// bf16 MFMA contraction against that slot's 4-bit weights.
//
//   group_pairs_kernel : counting sort of the pairs by slot reference, one
//                        workgroup; emits perm (sorted row -> pair) and the
//                        list of 64-row tiles {ref, first row, rows}
//   grouped_gate_up    : per (tile, 64 features): H = act(X Wg^T, X Wu^T)
//   grouped_down       : per (tile, 64 outputs):  Yp[pair] = score * H Wd^T
//   combine_pairs      : y[t] = sum over ranks r of Yp[t*k + r] (rank order)
//
// Dequantisation rides on the MFMA.  A word of eight 4-bit codes becomes a
// B fragment of bf16 values 128+q (exact, one v_bfi_b32 per pair), each
// 64-input quant group accumulates into a fresh accumulator, and
//   out += S * acc + (B - 128*S) * rowsum(X over the group),
// the factorised group form of kernels.py:141-145, with exact products and
// fp32 accumulation.  The 8 inputs of one MFMA lane are permuted identically
// in A and B (x_pairs order), which leaves every dot product unchanged.
//
// Every output row is one dot product per feature, computed by exactly one
// tile with a fixed accumulation order, so results do not depend on how the
// pairs were grouped or on the order of pairs inside a group.
//
// Reference: the batched gather_qmm calls with rhs_indices = slot per
// (token, rank) (engine_v3.py:588-598, engine_120b.py:132-143) and the
// score-weighted sum over ranks (engine_v3.py:600, engine_120b.py:145).
#include <algorithm>

#include "launchers.h"

namespace moe {

typedef __bf16 bf16x8_t __attribute__((ext_vector_type(8)));
typedef float f32x4_t __attribute__((ext_vector_type(4)));

__device__ __forceinline__ f32x4_t mfma16x16x32(uint4 a, uint4 b, f32x4_t c) {
  return __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(bf16x8_t, a),
                                                 __builtin_bit_cast(bf16x8_t, b), c, 0, 0,
                                                 0);
}

constexpr int kTileM = 64;

// The bias term of one LDS pass, sum over its groups g of rowsum[row][g] *
// C[g][n], as fp32 MFMAs of K = 4 groups: A = the row sums (lane: row l%16,
// group l/16 of the 4-group chunk), B = this lane's feature's C of group
// l/16 of the chunk, accumulated straight into the output tile (the layout
// of the 16x16x32 products).  Replaces one FMA per output element and group.
template <int GPS>
__device__ __forceinline__ void bias_term(const float *rs_l, const float (&C)[GPS], int mb,
                                          int col, int kq, f32x4_t &o) {
#pragma unroll
  for (int c = 0; c < (GPS + 3) / 4; ++c) {
    float cb = 0.f;
#pragma unroll
    for (int g = 4 * c; g < (GPS < 4 * c + 4 ? GPS : 4 * c + 4); ++g)
      if (kq == g - 4 * c) cb = C[g];
    const int kk = 4 * c + kq;
    const float ra = rs_l[(kk < GPS ? kk : GPS - 1) * kTileM + mb * 16 + col];
    o = __builtin_amdgcn_mfma_f32_16x16x4f32(kk < GPS ? ra : 0.f, cb, o, 0, 0, 0);
  }
}

// ---------------------------------------------------------------------------
// grouping: one workgroup of 1024 threads; hist[] in dynamic LDS spans every
// valid slot reference, key = ref + n_records in [0, n_slots + n_records).
// ---------------------------------------------------------------------------
__device__ __forceinline__ int wave_incl_scan(int v, int lane) {
#pragma unroll
  for (int d = 1; d < 64; d <<= 1) {
    const int y = __shfl_up(v, d, 64);
    if (lane >= d) v += y;
  }
  return v;
}

__global__ __launch_bounds__(1024) void group_pairs_kernel(
    const int32_t *__restrict__ refs, int n_pairs, int n_slots, int n_records, int D,
    int32_t *__restrict__ perm, int4 *__restrict__ tiles, int32_t *__restrict__ n_tiles,
    float *__restrict__ yp) {
  extern __shared__ int hist[];
  __shared__ int wsum_p[16], wsum_t[16];
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int nkeys = n_slots + n_records;
  for (int i = tid; i < nkeys; i += 1024) hist[i] = 0;
  __syncthreads();
  for (int p = tid; p < n_pairs; p += 1024) {
    const int key = refs[p] + n_records;
    if (key >= 0 && key < nkeys) {
      atomicAdd(&hist[key], 1);
    } else {   // out-of-range reference: flagged, contributes zero
      flag_error();
      for (int n = 0; n < D; ++n) yp[(int64_t)p * D + n] = 0.f;
    }
  }
  __syncthreads();
  // per-thread contiguous key chunk: pair and tile totals, then a block scan
  const int chunk = (nkeys + 1023) / 1024;
  const int k0 = min(tid * chunk, nkeys), k1 = min(k0 + chunk, nkeys);
  int sp = 0, st = 0;
  for (int i = k0; i < k1; ++i) {
    const int c = hist[i];
    sp += c;
    st += (c + kTileM - 1) / kTileM;
  }
  const int ip = wave_incl_scan(sp, lane), it = wave_incl_scan(st, lane);
  if (lane == 63) {
    wsum_p[wave] = ip;
    wsum_t[wave] = it;
  }
  __syncthreads();
  int bp = ip - sp, bt = it - st;
  for (int w = 0; w < wave; ++w) {
    bp += wsum_p[w];
    bt += wsum_t[w];
  }
  if (tid == 1023) *n_tiles = bt + st;
  for (int i = k0; i < k1; ++i) {
    const int c = hist[i];
    hist[i] = bp;   // becomes the scatter cursor of key i
    for (int m = 0; m < c; m += kTileM)
      tiles[bt++] = make_int4(i - n_records, bp + m, min(kTileM, c - m), 0);
    bp += c;
  }
  __syncthreads();
  for (int p = tid; p < n_pairs; p += 1024) {
    const int key = refs[p] + n_records;
    if (key >= 0 && key < nkeys) perm[atomicAdd(&hist[key], 1)] = p;
  }
}

// Groups of 64 inputs staged per LDS pass: a divisor of the group count.
constexpr int pick_gps(int ng) {
  return ng % 4 == 0 ? 4 : ng % 5 == 0 ? 5 : ng % 3 == 0 ? 3 : ng % 2 == 0 ? 2 : 1;
}

// B fragment: 8 codes of one weight row as bf16 128+q, x_pairs order.
__device__ __forceinline__ uint4 b_frag(uint32_t w) {
  uint32_t p[4];
  codes_to_bf16x2(w, p);
  return make_uint4(p[0], p[1], p[2], p[3]);
}

// One LDS pass of the A operand: 64 rows x (GPS groups of 64 inputs).
// Thread work item j = (row, group): 128 contiguous bytes, consecutive
// threads on consecutive groups of a row; rows past the tile read as zero.
template <int GPS>
struct AStage {
  static constexpr int PAIRS = kTileM * GPS;
  static constexpr int PER = (PAIRS + 255) / 256;
  static constexpr int ROW = GPS * 8 + 1;   // uint4 per LDS row (+1 pad)
  uint4 v[PER][8];

  __device__ __forceinline__ void load(const uint16_t *const src[PER], int k0, int tid) {
#pragma unroll
    for (int j = 0; j < PER; ++j) {
      const int pr = tid + 256 * j;
      const bool ok = pr < PAIRS && src[j] != nullptr;
      const uint4 *p =
          ok ? reinterpret_cast<const uint4 *>(src[j] + k0 + (pr % GPS) * 64) : nullptr;
#pragma unroll
      for (int q = 0; q < 8; ++q) v[j][q] = ok ? p[q] : make_uint4(0, 0, 0, 0);
    }
  }
  __device__ __forceinline__ void store(uint4 *a_l, float *rs_l, int tid) const {
#pragma unroll
    for (int j = 0; j < PER; ++j) {
      const int pr = tid + 256 * j;
      if (pr >= PAIRS) continue;
      const int row = pr / GPS, grp = pr % GPS;
      float s = 0.f;
#pragma unroll
      for (int q = 0; q < 8; ++q) {
        const uint32_t in[4] = {v[j][q].x, v[j][q].y, v[j][q].z, v[j][q].w};
        uint32_t out[4];
        x_pairs(in, out);
        a_l[row * ROW + grp * 8 + q] = make_uint4(out[0], out[1], out[2], out[3]);
#pragma unroll
        for (int m = 0; m < 4; ++m)
          s += bf16_to_f32(in[m] & 0xffffu) + bf16_to_f32(in[m] >> 16);
      }
      rs_l[grp * kTileM + row] = s;
    }
  }
};

// ---------------------------------------------------------------------------
// grouped gate/up.  Work item = (tile, 64 features); 4 waves, wave w owns
// features 16w..16w+15 of the block for every 16-row block of the tile.
// Within a group, MFMA lane quarter kq takes code words 2kq and 2kq+1
// (A pieces 2kq and 2kq+1 of the same group).
// ---------------------------------------------------------------------------
template <int D, int F, bool PBIAS>
__global__ __launch_bounds__(256) void grouped_gate_up_kernel(
    PoolArgs pa, const uint16_t *__restrict__ x, int k, const int32_t *__restrict__ perm,
    const int4 *__restrict__ tiles, const int32_t *__restrict__ n_tiles,
    uint16_t *__restrict__ h, int act, float alpha, float limit) {
  constexpr int NG = D / 64, GPS = pick_gps(NG), NS = NG / GPS, NB = F / 64;
  constexpr int NP = PBIAS ? 4 : 3;
  using Stage = AStage<GPS>;
  __shared__ uint4 a_l[kTileM * Stage::ROW];
  __shared__ __align__(16) float rs_l[GPS * kTileM];
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int col = lane & 15, kq = lane >> 4;
  const int n_items = *n_tiles * NB;
  for (int item = blockIdx.x; item < n_items; item += gridDim.x) {
    const int4 tl = tiles[item / NB];
    const int ref = tl.x, r0 = tl.y, rows = tl.z;
    const int n = (item % NB) * 64 + wave * 16 + col;   // this lane's feature
    const char *gw = resolve(pa, comp_index(PROJ_GATE, PART_W, NP), ref);
    if (gw == nullptr) {   // uniform over the workgroup
      if (tid == 0) flag_error();
      continue;
    }
    const uint2 *gwr = reinterpret_cast<const uint2 *>(gw) + (int64_t)n * (D / 16);
    const uint2 *uwr =
        reinterpret_cast<const uint2 *>(resolve(pa, comp_index(PROJ_UP, PART_W, NP), ref)) +
        (int64_t)n * (D / 16);
    const uint16_t *gs = reinterpret_cast<const uint16_t *>(
                             resolve(pa, comp_index(PROJ_GATE, PART_S, NP), ref)) + (int64_t)n * NG;
    const uint16_t *gb = reinterpret_cast<const uint16_t *>(
                             resolve(pa, comp_index(PROJ_GATE, PART_B, NP), ref)) + (int64_t)n * NG;
    const uint16_t *us = reinterpret_cast<const uint16_t *>(
                             resolve(pa, comp_index(PROJ_UP, PART_S, NP), ref)) + (int64_t)n * NG;
    const uint16_t *ub = reinterpret_cast<const uint16_t *>(
                             resolve(pa, comp_index(PROJ_UP, PART_B, NP), ref)) + (int64_t)n * NG;

    const uint16_t *src[Stage::PER];
#pragma unroll
    for (int j = 0; j < Stage::PER; ++j) {
      const int row = (tid + 256 * j) / GPS;
      src[j] = row < rows ? x + (int64_t)(perm[r0 + row] / k) * D : nullptr;
    }
    const int nmb = (rows + 15) / 16;
    f32x4_t og[4], ou[4];
#pragma unroll
    for (int mb = 0; mb < 4; ++mb) {
      og[mb] = (f32x4_t){0.f, 0.f, 0.f, 0.f};
      ou[mb] = (f32x4_t){0.f, 0.f, 0.f, 0.f};
    }
    Stage st;
    st.load(src, 0, tid);
    for (int s = 0; s < NS; ++s) {
      uint2 wg[GPS], wu[GPS];
      float Sg[GPS], Cg[GPS], Su[GPS], Cu[GPS];
#pragma unroll
      for (int g = 0; g < GPS; ++g) {
        const int gg = s * GPS + g;
        wg[g] = gwr[gg * 4 + kq];
        wu[g] = uwr[gg * 4 + kq];
        Sg[g] = bf16_to_f32(gs[gg]);
        Cg[g] = bf16_to_f32(gb[gg]) - 128.f * Sg[g];
        Su[g] = bf16_to_f32(us[gg]);
        Cu[g] = bf16_to_f32(ub[gg]) - 128.f * Su[g];
      }
      __syncthreads();   // the previous pass's LDS reads are done
      st.store(a_l, rs_l, tid);
      __syncthreads();
      if (s + 1 < NS) st.load(src, (s + 1) * GPS * 64, tid);
#pragma unroll
      for (int g = 0; g < GPS; ++g) {
        const uint4 bg0 = b_frag(wg[g].x), bg1 = b_frag(wg[g].y);
        const uint4 bu0 = b_frag(wu[g].x), bu1 = b_frag(wu[g].y);
#pragma unroll
        for (int mb = 0; mb < 4; ++mb) {
          if (mb >= nmb) break;
          const uint4 *ar = a_l + (mb * 16 + col) * Stage::ROW + g * 8 + 2 * kq;
          const uint4 a0 = ar[0], a1 = ar[1];
          f32x4_t cg = {0.f, 0.f, 0.f, 0.f}, cu = {0.f, 0.f, 0.f, 0.f};
          cg = mfma16x16x32(a0, bg0, cg);
          cg = mfma16x16x32(a1, bg1, cg);
          cu = mfma16x16x32(a0, bu0, cu);
          cu = mfma16x16x32(a1, bu1, cu);
#pragma unroll
          for (int r = 0; r < 4; ++r) {
            og[mb][r] += Sg[g] * cg[r];
            ou[mb][r] += Su[g] * cu[r];
          }
        }
      }
#pragma unroll
      for (int mb = 0; mb < 4; ++mb) {
        if (mb >= nmb) break;
        bias_term<GPS>(rs_l, Cg, mb, col, kq, og[mb]);
        bias_term<GPS>(rs_l, Cu, mb, col, kq, ou[mb]);
      }
    }
    float pbg = 0.f, pbu = 0.f;
    if (PBIAS) {
      pbg = bf16_to_f32(reinterpret_cast<const uint16_t *>(
          resolve(pa, comp_index(PROJ_GATE, PART_BIAS, NP), ref))[n]);
      pbu = bf16_to_f32(reinterpret_cast<const uint16_t *>(
          resolve(pa, comp_index(PROJ_UP, PART_BIAS, NP), ref))[n]);
    }
#pragma unroll
    for (int mb = 0; mb < 4; ++mb) {
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        const int rr = mb * 16 + 4 * kq + r;
        if (rr < rows) {
          const float hv = apply_act(act, og[mb][r] + pbg, ou[mb][r] + pbu, alpha, limit);
          h[(int64_t)(r0 + rr) * F + n] = (uint16_t)f32_to_bf16(hv);
        }
      }
    }
  }
}

// ---------------------------------------------------------------------------
// grouped down.  Work item = (tile, 64 outputs of d_model); A = the tile's h
// rows (sorted order); Yp[pair, n] = score[pair] * (h . Wd[n] + bias[n]).
// ---------------------------------------------------------------------------
template <int D, int F, bool PBIAS>
__global__ __launch_bounds__(256) void grouped_down_kernel(
    PoolArgs pa, const uint16_t *__restrict__ h, const float *__restrict__ scores,
    const int32_t *__restrict__ perm, const int4 *__restrict__ tiles,
    const int32_t *__restrict__ n_tiles, float *__restrict__ yp) {
  constexpr int NG = F / 64, GPS = pick_gps(NG), NS = NG / GPS, NB = D / 64;
  constexpr int NP = PBIAS ? 4 : 3;
  using Stage = AStage<GPS>;
  __shared__ uint4 a_l[kTileM * Stage::ROW];
  __shared__ __align__(16) float rs_l[GPS * kTileM];
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int col = lane & 15, kq = lane >> 4;
  const int n_items = *n_tiles * NB;
  for (int item = blockIdx.x; item < n_items; item += gridDim.x) {
    const int4 tl = tiles[item / NB];
    const int ref = tl.x, r0 = tl.y, rows = tl.z;
    const int n = (item % NB) * 64 + wave * 16 + col;
    const char *dw = resolve(pa, comp_index(PROJ_DOWN, PART_W, NP), ref);
    if (dw == nullptr) {
      if (tid == 0) flag_error();
      continue;
    }
    const uint2 *dwr = reinterpret_cast<const uint2 *>(dw) + (int64_t)n * (F / 16);
    const uint16_t *ds = reinterpret_cast<const uint16_t *>(
                             resolve(pa, comp_index(PROJ_DOWN, PART_S, NP), ref)) + (int64_t)n * NG;
    const uint16_t *db = reinterpret_cast<const uint16_t *>(
                             resolve(pa, comp_index(PROJ_DOWN, PART_B, NP), ref)) + (int64_t)n * NG;

    const uint16_t *src[Stage::PER];
#pragma unroll
    for (int j = 0; j < Stage::PER; ++j) {
      const int row = (tid + 256 * j) / GPS;
      src[j] = row < rows ? h + (int64_t)(r0 + row) * F : nullptr;
    }
    const int nmb = (rows + 15) / 16;
    f32x4_t o[4];
#pragma unroll
    for (int mb = 0; mb < 4; ++mb) o[mb] = (f32x4_t){0.f, 0.f, 0.f, 0.f};
    Stage st;
    st.load(src, 0, tid);
    for (int s = 0; s < NS; ++s) {
      uint2 w[GPS];
      float S[GPS], C[GPS];
#pragma unroll
      for (int g = 0; g < GPS; ++g) {
        const int gg = s * GPS + g;
        w[g] = dwr[gg * 4 + kq];
        S[g] = bf16_to_f32(ds[gg]);
        C[g] = bf16_to_f32(db[gg]) - 128.f * S[g];
      }
      __syncthreads();
      st.store(a_l, rs_l, tid);
      __syncthreads();
      if (s + 1 < NS) st.load(src, (s + 1) * GPS * 64, tid);
#pragma unroll
      for (int g = 0; g < GPS; ++g) {
        const uint4 b0 = b_frag(w[g].x), b1 = b_frag(w[g].y);
#pragma unroll
        for (int mb = 0; mb < 4; ++mb) {
          if (mb >= nmb) break;
          const uint4 *ar = a_l + (mb * 16 + col) * Stage::ROW + g * 8 + 2 * kq;
          f32x4_t c = {0.f, 0.f, 0.f, 0.f};
          c = mfma16x16x32(ar[0], b0, c);
          c = mfma16x16x32(ar[1], b1, c);
#pragma unroll
          for (int r = 0; r < 4; ++r) o[mb][r] += S[g] * c[r];
        }
      }
#pragma unroll
      for (int mb = 0; mb < 4; ++mb) {
        if (mb >= nmb) break;
        bias_term<GPS>(rs_l, C, mb, col, kq, o[mb]);
      }
    }
    float pb = 0.f;
    if (PBIAS)
      pb = bf16_to_f32(reinterpret_cast<const uint16_t *>(
          resolve(pa, comp_index(PROJ_DOWN, PART_BIAS, NP), ref))[n]);
#pragma unroll
    for (int mb = 0; mb < 4; ++mb) {
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        const int rr = mb * 16 + 4 * kq + r;
        if (rr < rows) {
          const int p = perm[r0 + rr];
          yp[(int64_t)p * D + n] = scores[p] * (o[mb][r] + pb);
        }
      }
    }
  }
}

// y[t, :] = sum over ranks r (ascending) of Yp[t*k + r, :]; 4 outputs/thread
__global__ __launch_bounds__(256) void combine_pairs_kernel(
    const float *__restrict__ yp, int T, int k, int D, uint16_t *__restrict__ out,
    float *__restrict__ out32) {
  const int64_t i = ((int64_t)blockIdx.x * blockDim.x + threadIdx.x) * 4;
  if (i >= (int64_t)T * D) return;
  const int64_t t = i / D, n = i % D;
  float4 s = make_float4(0.f, 0.f, 0.f, 0.f);
  for (int r = 0; r < k; ++r) {
    const float4 v = *reinterpret_cast<const float4 *>(yp + (t * k + r) * D + n);
    s.x += v.x;
    s.y += v.y;
    s.z += v.z;
    s.w += v.w;
  }
  if (out) {
    const uint32_t lo = f32_to_bf16(s.x) | (f32_to_bf16(s.y) << 16);
    const uint32_t hi = f32_to_bf16(s.z) | (f32_to_bf16(s.w) << 16);
    *reinterpret_cast<uint2 *>(out + i) = make_uint2(lo, hi);
  }
  if (out32) *reinterpret_cast<float4 *>(out32 + i) = s;
}

// ---------------------------------------------------------------------------
template <int D, int F, bool PB>
static void launch_gg(dim3 g, hipStream_t s, const PoolArgs &pa, const uint16_t *x, int k,
                      const int32_t *perm, const int4 *tiles, const int32_t *nt, uint16_t *h,
                      int act, float alpha, float limit) {
  hipLaunchKernelGGL((grouped_gate_up_kernel<D, F, PB>), g, dim3(256), 0, s, pa, x, k, perm,
                     tiles, nt, h, act, alpha, limit);
}
template <int D, int F, bool PB>
static void launch_gd(dim3 g, hipStream_t s, const PoolArgs &pa, const uint16_t *h,
                      const float *sc, const int32_t *perm, const int4 *tiles,
                      const int32_t *nt, float *yp) {
  hipLaunchKernelGGL((grouped_down_kernel<D, F, PB>), g, dim3(256), 0, s, pa, h, sc, perm,
                     tiles, nt, yp);
}

#define MOE_GROUPED_GEOM(D, F, PB) {D, F, PB, &launch_gg<D, F, PB>, &launch_gd<D, F, PB>}
static const GroupedLaunch kGroupedTable[] = {
    MOE_GROUPED_GEOM(2048, 768, false),   // Qwen3-30B-A3B
    MOE_GROUPED_GEOM(2048, 768, true),
    MOE_GROUPED_GEOM(2880, 2880, true),   // gpt-oss-120b
    MOE_GROUPED_GEOM(2880, 2880, false),
    MOE_GROUPED_GEOM(256, 128, false),    // small test geometry
    MOE_GROUPED_GEOM(256, 128, true),
};

const GroupedLaunch *find_grouped(int d_model, int d_ff, int has_bias) {
  for (const auto &e : kGroupedTable)
    if (e.d_model == d_model && e.d_ff == d_ff && e.has_bias == (has_bias != 0)) return &e;
  return nullptr;
}

GroupedWs grouped_ws(int64_t T, int k, int D, int F) {
  auto al = [](size_t v) { return (v + 255) & ~(size_t)255; };
  const int64_t P = T * k;
  GroupedWs w;
  w.max_tiles = P + P / kTileM + 1;
  size_t o = 0;
  w.off_perm = o; o += al((size_t)P * 4);
  w.off_tiles = o; o += al((size_t)w.max_tiles * 16);
  w.off_ntiles = o; o += al(4);
  w.off_h = o; o += al((size_t)P * F * 2);
  w.off_yp = o; o += al((size_t)P * D * 4);
  w.total = o;
  return w;
}

void launch_grouped(const GroupedLaunch *G, const PoolArgs &pa, const int32_t *refs,
                    const float *scores, const uint16_t *x, int T, int k, uint16_t *out,
                    float *out32, char *ws, int act, float alpha, float limit,
                    hipStream_t s) {
  const int D = G->d_model, F = G->d_ff, P = T * k;
  const GroupedWs w = grouped_ws(T, k, D, F);
  int32_t *perm = reinterpret_cast<int32_t *>(ws + w.off_perm);
  int4 *tiles = reinterpret_cast<int4 *>(ws + w.off_tiles);
  int32_t *ntiles = reinterpret_cast<int32_t *>(ws + w.off_ntiles);
  uint16_t *h = reinterpret_cast<uint16_t *>(ws + w.off_h);
  float *yp = reinterpret_cast<float *>(ws + w.off_yp);
  const int nkeys = pa.n_slots + pa.n_records;
  hipLaunchKernelGGL(group_pairs_kernel, dim3(1), dim3(1024), (size_t)nkeys * 4, s, refs, P,
                     pa.n_slots, pa.n_records, D, perm, tiles, ntiles, yp);
  const int64_t items_up = w.max_tiles * (F / 64), items_down = w.max_tiles * (D / 64);
  G->gate_up(dim3((unsigned)std::min<int64_t>(items_up, kGroupedMaxWGs)), s, pa, x, k, perm,
             tiles, ntiles, h, act, alpha, limit);
  G->down(dim3((unsigned)std::min<int64_t>(items_down, kGroupedMaxWGs)), s, pa, h, scores,
          perm, tiles, ntiles, yp);
  const int64_t n4 = (int64_t)T * D / 4;
  hipLaunchKernelGGL(combine_pairs_kernel, dim3((unsigned)((n4 + 255) / 256)), dim3(256), 0,
                     s, yp, T, k, D, out, out32);
}

}  // namespace moe
