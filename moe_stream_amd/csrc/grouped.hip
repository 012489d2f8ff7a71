// Multi-token (prefill / batched) expert block for gfx950: the T*k routed
// (token, slot) pairs are grouped by slot and every group runs as a dense
// bf16 MFMA contraction against that slot's 4-bit weights.
//
//   group_pairs_kernel : counting sort of the pairs by slot reference, one
//                        workgroup; emits perm (sorted row -> pair) and the
//                        list of 64-row tiles {ref, first row, rows}
//   grouped_mm (gate/up): per (tile, NB features): H = act(X Wg^T, X Wu^T)
//   grouped_mm (down)   : per (tile, NB outputs):  Yp[pair] = score * H Wd^T
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
#include <type_traits>

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
constexpr int kRsPitch = 80;   // row-sum LDS pitch (floats): 4 groups' rows on distinct banks

// ---------------------------------------------------------------------------
// grouping: one workgroup of 1024 threads; hist[] in dynamic LDS spans every
// valid slot reference, key = ref + n_records in [0, n_slots + n_records).
// ---------------------------------------------------------------------------
// Inclusive scans on DPP (no LDS round trips): within each 16-lane row
// (row_shr 1, 2, 4, 8; lanes without a source add 0), and across the wave
// (then row 0's total into row 1 and row 2's into row 3 by row_bcast:15, rows
// 0-1's total into rows 2-3 by row_bcast:31).
__device__ __forceinline__ int row16_incl_scan(int v) {
  v += __builtin_amdgcn_update_dpp(0, v, 0x111, 0xf, 0xf, true);
  v += __builtin_amdgcn_update_dpp(0, v, 0x112, 0xf, 0xf, true);
  v += __builtin_amdgcn_update_dpp(0, v, 0x114, 0xf, 0xf, true);
  v += __builtin_amdgcn_update_dpp(0, v, 0x118, 0xf, 0xf, true);
  return v;
}
__device__ __forceinline__ int wave_incl_scan(int v) {
  v = row16_incl_scan(v);
  v += __builtin_amdgcn_update_dpp(0, v, 0x142, 0xa, 0xf, false);
  v += __builtin_amdgcn_update_dpp(0, v, 0x143, 0xc, 0xf, false);
  return v;
}

__device__ __forceinline__ void group_pairs_body(
    const int32_t *__restrict__ refs, int n_pairs, int n_slots, int n_records, int D,
    int32_t *__restrict__ perm, int4 *__restrict__ tiles, int32_t *__restrict__ n_tiles,
    float *__restrict__ yp) {
  extern __shared__ int hist[];
  // tiles are listed by size class, largest first (classes 4..1: a tile of
  // r rows is class ceil(r / 16)), so the longest work items start first
  __shared__ int wsum[5][16];   // per wave: pairs, class-1..4 tiles
  __shared__ int wpre[5][16];   // exclusive prefixes over the waves
  __shared__ int cbase[4];      // first tile of each class (class 4 first)
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
  // per-thread contiguous key chunk: pair and per-class tile totals, then
  // block scans
  const int chunk = (nkeys + 1023) / 1024;
  const int k0 = min(tid * chunk, nkeys), k1 = min(k0 + chunk, nkeys);
  auto tile_class = [](int rows) { return (rows + 15) >> 4; };   // 1..4
  int st[5] = {0, 0, 0, 0, 0};   // pairs, then tiles of classes 1..4
  for (int i = k0; i < k1; ++i) {
    const int c = hist[i];
    const int cl = c % kTileM ? tile_class(c % kTileM) : 0;
    st[0] += c;
    st[1] += cl == 1;
    st[2] += cl == 2;
    st[3] += cl == 3;
    st[4] += c / kTileM + (cl == 4);
  }
  int it[5];
#pragma unroll
  for (int q = 0; q < 5; ++q) {
    it[q] = wave_incl_scan(st[q]);
    if (lane == 63) wsum[q][wave] = it[q];
  }
  __syncthreads();
  if (wave == 0) {   // the 16 waves' prefixes: one quantity per 16-lane row
    const int row = lane >> 4, w = lane & 15;
    __shared__ int ctot[8];
#pragma unroll
    for (int h = 0; h < 2; ++h) {
      const int q = h * 4 + row;   // quantities 0-3, then 4
      const int v = q < 5 ? wsum[q][w] : 0;
      const int sc = row16_incl_scan(v);
      if (q < 5) wpre[q][w] = sc - v;
      if (w == 15) ctot[q] = sc;   // the quantity's total
    }
    if (lane == 0) {   // class bases, class 4 first
      const int c1 = ctot[1], c2 = ctot[2], c3 = ctot[3], c4 = ctot[4];
      cbase[3] = 0;
      cbase[2] = c4;
      cbase[1] = c4 + c3;
      cbase[0] = c4 + c3 + c2;
      *n_tiles = c4 + c3 + c2 + c1;
    }
  }
  __syncthreads();
  int bp = wpre[0][wave] + it[0] - st[0], bt[4];
#pragma unroll
  for (int q = 0; q < 4; ++q) bt[q] = cbase[q] + wpre[q + 1][wave] + it[q + 1] - st[q + 1];
  for (int i = k0; i < k1; ++i) {
    const int c = hist[i];
    hist[i] = bp;   // becomes the scatter cursor of key i
    for (int m = 0; m < c; m += kTileM) {
      const int rows = min(kTileM, c - m), q = tile_class(rows) - 1;   // bt index
      int t = 0;
#pragma unroll
      for (int qq = 0; qq < 4; ++qq)   // (registers, not a dynamic index)
        if (qq == q) t = bt[qq]++;
      tiles[t] = make_int4(i - n_records, bp + m, rows, 0);
    }
    bp += c;
  }
  __syncthreads();
  for (int p = tid; p < n_pairs; p += 1024) {
    const int key = refs[p] + n_records;
    if (key >= 0 && key < nkeys) perm[atomicAdd(&hist[key], 1)] = p;
  }
}

__global__ __launch_bounds__(1024) void group_pairs_kernel(
    const int32_t *__restrict__ refs, int n_pairs, int n_slots, int n_records, int D,
    int32_t *__restrict__ perm, int4 *__restrict__ tiles, int32_t *__restrict__ n_tiles,
    float *__restrict__ yp) {
  group_pairs_body(refs, n_pairs, n_slots, n_records, D, perm, tiles, n_tiles, yp);
}

// B fragment: 8 codes of one weight row as bf16 128+q, x_pairs order.
__device__ __forceinline__ uint4 b_frag(uint32_t w) {
  uint32_t p[4];
  codes_to_bf16x2(w, p);
  return make_uint4(p[0], p[1], p[2], p[3]);
}

// ---------------------------------------------------------------------------
// The A operand's rows in x_pairs order (each 8-input piece p holds inputs
// (0,4), (1,5), (2,6), (3,7) pairwise, the order of the B fragments) and their
// 64-input row sums, once per call: one thread per piece, the 8 pieces of a
// group in 8 consecutive lanes (rs: [rows][K / 64] fp32).
// ---------------------------------------------------------------------------
// piece i of `rows` rows of K inputs (32-bit index arithmetic: the host
// passes at most 2^30 pieces at a time)
__device__ __forceinline__ void prep_piece(int i, const uint16_t *__restrict__ src, int64_t rows,
                                           int K, uint16_t *__restrict__ dst,
                                           float *__restrict__ rs) {
  const int ppr = K / 8;
  const bool ok = i < (int)(rows * ppr);
  const int r = ok ? i / ppr : 0;
  const int pc = ok ? i - r * ppr : 0;
  const uint4 v = ok ? load16(reinterpret_cast<const uint4 *>(src + (int64_t)r * K + pc * 8))
                     : make_uint4(0, 0, 0, 0);
  const uint32_t in[4] = {v.x, v.y, v.z, v.w};
  uint32_t out[4];
  x_pairs(in, out);
  float sm = 0.f;
#pragma unroll
  for (int m = 0; m < 4; ++m) sm += bf16_to_f32(in[m] & 0xffffu) + bf16_to_f32(in[m] >> 16);
  sm = group_sum<8>(sm);
  if (ok) {
    *reinterpret_cast<uint4 *>(dst + (int64_t)r * K + pc * 8) = make_uint4(out[0], out[1], out[2], out[3]);
    if ((pc & 7) == 0) rs[(int64_t)r * (K / 64) + pc / 8] = sm;
  }
}

__global__ __launch_bounds__(256) void grouped_prep_kernel(const uint16_t *__restrict__ src,
                                                           int64_t rows, int K,
                                                           uint16_t *__restrict__ dst,
                                                           float *__restrict__ rs) {
  prep_piece(blockIdx.x * 256 + threadIdx.x, src, rows, K, dst, rs);
}

// The grouping (workgroup 0) and the token rows' prep (the other workgroups)
// in one launch: they are independent, so the prep runs beside the grouping.
__global__ __launch_bounds__(1024) void group_prep_kernel(
    const int32_t *__restrict__ refs, int n_pairs, int n_slots, int n_records, int D,
    int32_t *__restrict__ perm, int4 *__restrict__ tiles, int32_t *__restrict__ n_tiles,
    float *__restrict__ yp, const uint16_t *__restrict__ x, int64_t T, uint16_t *__restrict__ xq,
    float *__restrict__ rsx) {
  if (blockIdx.x == 0)
    group_pairs_body(refs, n_pairs, n_slots, n_records, D, perm, tiles, n_tiles, yp);
  else
    prep_piece((blockIdx.x - 1) * 1024 + threadIdx.x, x, T, D, xq, rsx);
}

// ---------------------------------------------------------------------------
// One work item of the grouped contraction: the rows of one tile (A, up to
// 64 rows of KIN bf16 inputs, already in x_pairs order) against NPROJ
// projections' 4-bit weights for NB consecutive output features.  WAVES
// waves; wave w owns CPW 16-feature column blocks of every projection for
// the NMB 16-row blocks the tile fills (a template parameter: no branches
// around the MFMAs).
//
// The inputs are processed a quad (4 quant groups of 64 inputs) at a time.
// A quad's operands sit in LDS while the workgroup computes its 4 groups
// with no barrier in between; the next quad's operands wait in registers
// (their loads issued a quad earlier) and go to LDS between two barriers at
// the quad's end, when the loads of the quad after it are issued.
//  * A: the token rows' 8-input pieces, row-major per group, piece p of row r
//    at r * 8 + (p ^ (r & 7)): each 8-lane run of the copy writes one whole
//    row (no bank conflict) and the MFMA reads of a piece across 16 rows fall
//    on distinct banks.
//  * B: 128 bytes of every weight row per quad (whole cache lines, 8 lanes
//    per row); in LDS 8 chunks of 16 bytes, chunk c at c ^ ((row >> 1) & 7),
//    so the 32 lanes of one 8-byte fragment read (16 rows x 2 halves) fall on
//    distinct banks.  Each lane reads its two code words (8 bytes) per group.
// Every thread issues the same loads on every path (rows past the tile and
// chunks past the row are clamped to a valid address and never used; the
// last quads are unrolled), so the compiler's counter waits ask for exactly
// the data in hand.  The item's scales, biases and row sums are staged in
// LDS once: scales quad-major (each lane reads its row's 4 scales of a quad
// as 8 contiguous bytes, the 16 rows of a fragment side by side), row sums at
// a pitch of 80 floats (the 4 groups of one bias MFMA on distinct banks).
// Each group accumulates into a fresh 16x16 block (2 MFMAs over the bf16
// 128+q codes), folded into the output by S; the bias term
// sum_g rowsum[g] * (B - 128 S) runs on fp32 MFMAs (K = 4 groups) per quad.
// Rows past the tile compute garbage from a copy of a real row, which no
// output row depends on (MFMA rows are independent) and nothing stores.
// ---------------------------------------------------------------------------
template <int KIN, int NB, int WAVES, int NPROJ>
struct GItem {
  static constexpr int NT = 64 * WAVES;
  static constexpr int NG = KIN / 64;                  // quant groups along the inputs
  static constexpr int NQ = (NG + 3) / 4;              // quads (B staging units)
  static constexpr int NG4 = NQ;                       // bias MFMAs, 4 groups each
  static constexpr int CPW = NB / 16 / WAVES;          // column blocks per wave
  static constexpr int SPT = (kTileM * 8 + NT - 1) / NT;   // A pieces per thread and group
  static constexpr int BROWS = NPROJ * NB;             // weight rows of the item
  static constexpr int BPT = BROWS * 8 / NT;           // B 16-byte pieces per thread and quad
  static constexpr int SCB = NB * NG * 2;              // bytes of one scale array's block
  static constexpr int NARR = 2 * NPROJ;               // (S, B) per projection
  static constexpr int SCP = NARR * SCB / 16;          // 16-byte pieces of all of them
  static constexpr int SCW = (SCP + NT - 1) / NT;      // ... per thread
  // with NG a multiple of 4 the scales are staged quad-major: [array][quad][feature]
  // x 4 halfwords (8-byte pieces), else copied as they are ([array][feature][group])
  static constexpr bool QS = NG % 4 == 0;
  static constexpr int SQP = NARR * NQ * NB;           // 8-byte pieces, quad-major
  static constexpr int SQW = (SQP + NT - 1) / NT;      // ... per thread
  static constexpr int RSW = (NG4 * 4 + WAVES - 1) / WAVES;   // row-sum groups per thread
  static_assert(KIN % 64 == 0 && NB % (16 * WAVES) == 0 && CPW >= 1, "feature split");
  static_assert(SCB % 16 == 0 && NT % 8 == 0 && (BROWS * 8) % NT == 0, "staging");
  // quads [0, QMAIN) refill the registers with quad q + 2 (a loop); the last
  // two quads are unrolled
  static constexpr int QMAIN = NQ >= 2 ? NQ - 2 : 0;
};

struct GLds {   // (one layout for every instantiation; sized by the caller)
  float *part;             // gate/up with the fused input prep: [NB / 16][64] row partial sums
  int *rperm;              // down: the tile rows' pair ids [64] ...
  float *rsc;              // ... and their scores [64]
  uint4 (*a)[kTileM * 8];  // [4 groups][row * 8 + (piece ^ (row & 7))]
  uint4 *b;                // [BROWS][8]: one quad of codes
  float *rs;               // [NG4 * 4][kRsPitch]: 64-input row sums (row < 64), zero past NG
  uint4 *sc;
};

template <int NMB, int D, int F, bool PBIAS, int NB, int WAVES, bool GU>
__device__ __forceinline__ void grouped_item(
    const PoolArgs &pa, const uint16_t *__restrict__ aq, const float *__restrict__ ars, int k,
    const int32_t *__restrict__ perm, int ref, int r0, int rows, int nb0,
    uint16_t *__restrict__ h_out, float *__restrict__ rs_out, const float *__restrict__ scores,
    float *__restrict__ yp, int act, float alpha, float limit, const GLds &L) {
  constexpr int KIN = GU ? D : F, NPROJ = GU ? 2 : 1;
  using I = GItem<KIN, NB, WAVES, NPROJ>;
  constexpr int NG = I::NG, NQ = I::NQ, CPW = I::CPW, NT = I::NT, SPT = I::SPT;
  constexpr int BPT = I::BPT;
  constexpr int NP = PBIAS ? 4 : 3, SCH = I::SCB / 2;   // halfwords per scale array block
  constexpr int ROWS = NMB * 16;                        // staged rows
  constexpr int RB = KIN / 2;                           // bytes per weight row
  const uint16_t *sch = reinterpret_cast<const uint16_t *>(L.sc);
  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int col = lane & 15, kq = lane >> 4;
  const char *w[NPROJ];
  const char *sa[I::NARR];
#pragma unroll
  for (int j = 0; j < NPROJ; ++j) {
    const int proj = GU ? (j == 0 ? PROJ_GATE : PROJ_UP) : PROJ_DOWN;
    w[j] = resolve(pa, comp_index(proj, PART_W, NP), ref);
    sa[2 * j] = resolve(pa, comp_index(proj, PART_S, NP), ref);
    sa[2 * j + 1] = resolve(pa, comp_index(proj, PART_B, NP), ref);
  }
  // the A source row of tile row r (clamped into the tile)
  auto src_row = [&](int r) -> int64_t {
    r = min(r, rows - 1);
    return GU ? gload4i(perm + r0 + r) / k : r0 + r;
  };
  // this thread's A pieces (slot s = 8 * row + piece)
  const uint16_t *asrc[SPT];
#pragma unroll
  for (int j = 0; j < SPT; ++j) {
    const int s = tid + NT * j;
    asrc[j] = aq + src_row(s >> 3) * KIN + (s & 7) * 8;
  }
  auto load_a = [&](int g, uint4 (&v)[SPT]) {
#pragma unroll
    for (int j = 0; j < SPT; ++j) v[j] = gload16(asrc[j] + g * 64);
  };
  // this thread's B pieces: piece p = tid + NT * i is chunk p % 8 of item
  // weight row p / 8 (rows [0, NB) the first projection, then the second)
  const char *bsrc[BPT];
  uint32_t bdst[BPT];   // LDS byte offset of the piece in the quad buffer
#pragma unroll
  for (int i = 0; i < BPT; ++i) {
    const int p = tid + NT * i, row = p >> 3, c = p & 7;
    const int j = row / NB, fl = row % NB;
    bsrc[i] = w[NPROJ > 1 ? j : 0] + (int64_t)(nb0 + fl) * RB + c * 16;
    bdst[i] = (uint32_t)(row * 128 + ((c ^ ((row >> 1) & 7)) << 4));
  }
  auto load_b = [&](int q, uint4 (&v)[BPT]) {
#pragma unroll
    for (int i = 0; i < BPT; ++i) {
      // (a chunk past the row end, in a last partial quad: any valid chunk)
      const int off = (RB % 128 == 0 || q * 128 + 128 <= RB)
                          ? q * 128
                          : min(q * 128, RB - 16 - (int)((tid + NT * i) & 7) * 16);
      v[i] = gload16(bsrc[i] + off);
    }
  };
  auto store_b = [&](int buf, const uint4 (&v)[BPT]) {
    char *base = reinterpret_cast<char *>(L.b + buf * I::BROWS * 8);
#pragma unroll
    for (int i = 0; i < BPT; ++i) *reinterpret_cast<uint4 *>(base + bdst[i]) = v[i];
  };
  // this lane's B fragment rows: feature col of column block cb, projection j
  uint32_t bfr[NPROJ][CPW];   // LDS byte offset of the row in a quad buffer
  uint32_t bx[NPROJ][CPW];    // its chunk swizzle ((row >> 1) & 7), as a byte offset
#pragma unroll
  for (int j = 0; j < NPROJ; ++j)
#pragma unroll
    for (int cb = 0; cb < CPW; ++cb) {
      const int row = j * NB + (wave * CPW + cb) * 16 + col;
      bfr[j][cb] = row * 128;
      bx[j][cb] = ((row >> 1) & 7) << 4;
    }
  // the item's scales and biases (each array's NB rows are one contiguous
  // block) and row sums, loaded ahead of the first quad and written to LDS after
  constexpr bool QS = I::QS;
  constexpr int SCN = QS ? I::SQW : I::SCW;
  uint4 scv[QS ? 1 : I::SCW];
  uint2 sqv[QS ? I::SQW : 1];
#pragma unroll
  for (int j = 0; j < SCN; ++j) {
    if (QS) {   // piece i: feature i % NB, quad (i / NB) % NQ, array i / (NB * NQ)
      const int i = min(tid + NT * j, I::SQP - 1);
      const int nl = i % NB, q = (i / NB) % NQ, arr = i / (NB * NQ);
      sqv[j] = gload8(sa[arr] + ((int64_t)(nb0 + nl) * NG + 4 * q) * 2);
    } else {
      const int i = min(tid + NT * j, I::SCP - 1);
      const int arr = i / (I::SCB / 16), o = i % (I::SCB / 16);
      scv[j] = gload16(sa[arr] + (int64_t)nb0 * NG * 2 + (int64_t)o * 16);
    }
  }
  float rsv[I::RSW];
  {
    const float *rrow = ars + src_row(lane) * NG;
#pragma unroll
    for (int j = 0; j < I::RSW; ++j) rsv[j] = gload4f(rrow + min(wave + WAVES * j, NG - 1));
  }
  // one quad of token-row pieces and codes in registers at a time
  uint4 breg[BPT];
  uint4 areg[4][SPT];
  auto load_quad = [&](int q, int ng) {   // ng: the quad's groups (a constant)
#pragma unroll
    for (int gi = 0; gi < 4; ++gi)
      if (gi < ng) load_a(4 * q + gi, areg[gi]);
    load_b(q, breg);
  };
  auto store_quad = [&](int ng) {
#pragma unroll
    for (int gi = 0; gi < 4; ++gi) {
      if (gi >= ng) continue;
#pragma unroll
      for (int j = 0; j < SPT; ++j) {
        const int sl = tid + NT * j;
        if (sl < ROWS * 8) {   // uniform per wave
          const int r = sl >> 3, p = sl & 7;
          L.a[gi][r * 8 + (p ^ (r & 7))] = areg[gi][j];
        }
      }
    }
    store_b(0, breg);
  };
  constexpr int NGL = NG - 4 * (NQ - 1);   // groups of the last quad
  load_quad(0, NQ > 1 ? 4 : NGL);
  // down: the pair id and score of tile row `lane` for the epilogue (every
  // wave loads them, wave 0 keeps them: no branch around the loads)
  int my_pr = 0;
  float my_sc = 0.f;
  if (!GU) {
    my_pr = gload4i(perm + r0 + min(lane, rows - 1));
    my_sc = gload4f(scores + my_pr);
  }
#pragma unroll
  for (int j = 0; j < SCN; ++j) {
    if (QS) {
      if (I::SQP % NT == 0 || tid + NT * j < I::SQP)
        reinterpret_cast<uint2 *>(L.sc)[tid + NT * j] = sqv[j];
    } else {
      if (I::SCP % NT == 0 || tid + NT * j < I::SCP) L.sc[tid + NT * j] = scv[j];
    }
  }
#pragma unroll
  for (int j = 0; j < I::RSW; ++j) {
    const int g = wave + WAVES * j;
    if (g < I::NG4 * 4) L.rs[g * kRsPitch + lane] = g < NG ? rsv[j] : 0.f;
  }
  f32x4_t acc[NMB][CPW][NPROJ];
#pragma unroll
  for (int rb = 0; rb < NMB; ++rb)
#pragma unroll
    for (int cb = 0; cb < CPW; ++cb)
#pragma unroll
      for (int j = 0; j < NPROJ; ++j) acc[rb][cb][j] = (f32x4_t){0.f, 0.f, 0.f, 0.f};
  store_quad(NQ > 1 ? 4 : NGL);
  if (!GU && wave == 0) {
    L.rperm[lane] = my_pr;
    L.rsc[lane] = my_sc;
  }
  if (NQ > 1) load_quad(1, NQ > 2 ? 4 : NGL);
  __syncthreads();
  // with quad-major scales each lane reads its row's scales 4 groups at a
  // time (8 bytes at the quad's first group)
  const uint2 *scq = reinterpret_cast<const uint2 *>(L.sc);
  uint2 s4[NPROJ][CPW];
  // the bias term of quad q: fp32 MFMAs of K = 4 groups, A = row sums (lane:
  // row col, group 4q + kq), B = B - 128 S of this lane's feature (zero past
  // NG).  Each starts from a zero accumulator and is added on the VALU (no
  // MFMA reads registers as its accumulator input: see below).
  auto bias_step = [&](int q, const uint2 (&s4)[NPROJ][CPW]) {
    const int gb = 4 * q + kq, gc = min(gb, NG - 1);
    float C[NPROJ][CPW];
#pragma unroll
    for (int j = 0; j < NPROJ; ++j)
#pragma unroll
      for (int cb = 0; cb < CPW; ++cb) {
        const int nl = (wave * CPW + cb) * 16 + col;
        float sv, bv;
        if (QS) {   // this lane's group of the quad from the quad's 4 halfwords
          const uint2 b4 = scq[((2 * j + 1) * NQ + q) * NB + nl];
          const uint32_t hs = kq < 2 ? s4[j][cb].x : s4[j][cb].y;
          const uint32_t hb = kq < 2 ? b4.x : b4.y;
          sv = __uint_as_float((kq & 1) ? (hs & 0xffff0000u) : (hs << 16));
          bv = __uint_as_float((kq & 1) ? (hb & 0xffff0000u) : (hb << 16));
        } else {
          sv = bf16_to_f32(sch[(2 * j) * SCH + nl * NG + gc]);
          bv = bf16_to_f32(sch[(2 * j + 1) * SCH + nl * NG + gc]);
        }
        C[j][cb] = gb < NG ? bv - 128.f * sv : 0.f;
      }
#pragma unroll
    for (int rb = 0; rb < NMB; ++rb) {
      const float ra = L.rs[gb * kRsPitch + rb * 16 + col];
#pragma unroll
      for (int cb = 0; cb < CPW; ++cb)
#pragma unroll
        for (int j = 0; j < NPROJ; ++j) {
          const f32x4_t bz = __builtin_amdgcn_mfma_f32_16x16x4f32(
              ra, C[j][cb], (f32x4_t){0.f, 0.f, 0.f, 0.f}, 0, 0, 0);
#pragma unroll
          for (int e = 0; e < 4; ++e) acc[rb][cb][j][e] += bz[e];
        }
    }
  };
  // One group of the quad in LDS (gi: its index in the quad, a constant), in
  // source order: decode, MFMAs, fold (down, held to 128 VGPRs)
  auto group = [&](int g, int gi) {
    if (QS && gi == 0) {   // the quad's scales, 4 halfwords per lane and row
#pragma unroll
      for (int j = 0; j < NPROJ; ++j)
#pragma unroll
        for (int cb = 0; cb < CPW; ++cb) {
          const int nl = (wave * CPW + cb) * 16 + col;
          s4[j][cb] = scq[((2 * j) * NQ + (g >> 2)) * NB + nl];
        }
    }
    const uint4 *al = L.a[gi];
    const char *bq = reinterpret_cast<const char *>(L.b);
    const uint32_t cpos = (uint32_t)(gi * 32 + kq * 8);   // logical chunk and half
    uint4 b0[NPROJ][CPW], b1[NPROJ][CPW];
    float S[NPROJ][CPW];
#pragma unroll
    for (int j = 0; j < NPROJ; ++j)
#pragma unroll
      for (int cb = 0; cb < CPW; ++cb) {
        const uint2 cw = *reinterpret_cast<const uint2 *>(bq + bfr[j][cb] + (cpos ^ bx[j][cb]));
        b0[j][cb] = b_frag(cw.x);
        b1[j][cb] = b_frag(cw.y);
        if (QS) {
          const uint32_t h = gi < 2 ? s4[j][cb].x : s4[j][cb].y;
          S[j][cb] = __uint_as_float((gi & 1) ? (h & 0xffff0000u) : (h << 16));
        } else {
          const int nl = (wave * CPW + cb) * 16 + col;
          S[j][cb] = bf16_to_f32(sch[(2 * j) * SCH + nl * NG + g]);
        }
      }
#pragma unroll
    for (int rb = 0; rb < NMB; ++rb) {
      const int r = rb * 16 + col;
      const uint4 a0 = al[r * 8 + ((2 * kq) ^ (r & 7))], a1 = al[r * 8 + ((2 * kq + 1) ^ (r & 7))];
#pragma unroll
      for (int cb = 0; cb < CPW; ++cb)
#pragma unroll
        for (int j = 0; j < NPROJ; ++j) {
          const f32x4_t c0 = mfma16x16x32(a0, b0[j][cb], (f32x4_t){0.f, 0.f, 0.f, 0.f});
          const f32x4_t c = mfma16x16x32(a1, b1[j][cb], c0);
#pragma unroll
          for (int e = 0; e < 4; ++e) acc[rb][cb][j][e] += S[j][cb] * c[e];
          // c0 (the second MFMA's accumulator input) stays allocated until the
          // fold has read c: this compiler otherwise reuses its registers a
          // few instructions after the MFMA issues, before the MFMA has read
          // them.  The empty asm passes acc through (a data dependency, not a
          // side effect), so it orders no memory access and LDS reads of
          // later row blocks can still be issued ahead of this fold
          asm("" : "+v"(acc[rb][cb][j]) : "v"(c0));
        }
    }
  };
  // One group of the quad in LDS (gi: its index in the quad, a constant), in
  // three steps so the quad can run them as a software pipeline: its B
  // fragments decoded (and its scales), its MFMAs into fresh 16x16 blocks, and
  // the fold of those blocks into the output by S.  The quad issues group
  // gi's MFMAs, then decodes group gi + 1 and folds group gi, so that VALU
  // work independent of the MFMAs in flight follows them.
  struct GFrag {
    uint4 b0[NPROJ][CPW], b1[NPROJ][CPW];
    float S[NPROJ][CPW];
  };
  struct GOut {
    f32x4_t c0[NMB][CPW][NPROJ], c[NMB][CPW][NPROJ];
  };
  auto decode = [&](int g, int gi, GFrag &f) {
    if (QS && gi == 0) {   // the quad's scales, 4 halfwords per lane and row
#pragma unroll
      for (int j = 0; j < NPROJ; ++j)
#pragma unroll
        for (int cb = 0; cb < CPW; ++cb) {
          const int nl = (wave * CPW + cb) * 16 + col;
          s4[j][cb] = scq[((2 * j) * NQ + (g >> 2)) * NB + nl];
        }
    }
    const char *bq = reinterpret_cast<const char *>(L.b);
    const uint32_t cpos = (uint32_t)(gi * 32 + kq * 8);   // logical chunk and half
#pragma unroll
    for (int j = 0; j < NPROJ; ++j)
#pragma unroll
      for (int cb = 0; cb < CPW; ++cb) {
        const uint2 cw = *reinterpret_cast<const uint2 *>(bq + bfr[j][cb] + (cpos ^ bx[j][cb]));
        f.b0[j][cb] = b_frag(cw.x);
        f.b1[j][cb] = b_frag(cw.y);
        if (QS) {
          const uint32_t h = gi < 2 ? s4[j][cb].x : s4[j][cb].y;
          f.S[j][cb] = __uint_as_float((gi & 1) ? (h & 0xffff0000u) : (h << 16));
        } else {
          const int nl = (wave * CPW + cb) * 16 + col;
          f.S[j][cb] = bf16_to_f32(sch[(2 * j) * SCH + nl * NG + g]);
        }
      }
  };
  auto mma = [&](int gi, const GFrag &f, GOut &o) {
    const uint4 *al = L.a[gi];
#pragma unroll
    for (int rb = 0; rb < NMB; ++rb) {
      const int r = rb * 16 + col;
      const uint4 a0 = al[r * 8 + ((2 * kq) ^ (r & 7))], a1 = al[r * 8 + ((2 * kq + 1) ^ (r & 7))];
#pragma unroll
      for (int cb = 0; cb < CPW; ++cb)
#pragma unroll
        for (int j = 0; j < NPROJ; ++j) {
          o.c0[rb][cb][j] = mfma16x16x32(a0, f.b0[j][cb], (f32x4_t){0.f, 0.f, 0.f, 0.f});
          o.c[rb][cb][j] = mfma16x16x32(a1, f.b1[j][cb], o.c0[rb][cb][j]);
        }
    }
  };
  auto fold = [&](const GFrag &f, const GOut &o) {
#pragma unroll
    for (int rb = 0; rb < NMB; ++rb)
#pragma unroll
      for (int cb = 0; cb < CPW; ++cb)
#pragma unroll
        for (int j = 0; j < NPROJ; ++j) {
#pragma unroll
          for (int e = 0; e < 4; ++e) acc[rb][cb][j][e] += f.S[j][cb] * o.c[rb][cb][j][e];
          // c0 (the second MFMA's accumulator input) stays allocated until the
          // fold has read c: this compiler otherwise reuses its registers a
          // few instructions after the MFMA issues, before the MFMA has read
          // them.  The empty asm passes acc through (a data dependency, not a
          // side effect), so it orders no memory access
          asm("" : "+v"(acc[rb][cb][j]) : "v"(o.c0[rb][cb][j]));
        }
  };
  // one quad: its groups from LDS, its bias term; then (all waves done with
  // the quad) the next quad's operands from registers to LDS and the loads of
  // the one after
  auto quad = [&](int q, int ng, bool next, int ng_next, bool refill, int ng_refill) {
    if (GU && QS) {   // gate/up: the pipelined order (down keeps 4 waves per
                      // SIMD; with NG % 4 != 0 it would not fit 256 VGPRs)
      GFrag fr[2];
      GOut o;
      decode(4 * q, 0, fr[0]);
#pragma unroll
      for (int gi = 0; gi < 4; ++gi) {
        if (gi >= ng) continue;
        mma(gi, fr[gi & 1], o);
        if (gi + 1 < ng) decode(4 * q + gi + 1, gi + 1, fr[(gi + 1) & 1]);
        fold(fr[gi & 1], o);
      }
    } else {
#pragma unroll
      for (int gi = 0; gi < 4; ++gi)
        if (gi < ng) group(4 * q + gi, gi);
    }
    bias_step(q, s4);
    if (next) {
      __syncthreads();
      store_quad(ng_next);
      if (refill) load_quad(q + 2, ng_refill);
      __syncthreads();
    }
  };
  for (int q = 0; q < I::QMAIN; ++q) quad(q, 4, true, 4, true, q + 2 < NQ - 1 ? 4 : NGL);
  if (NQ >= 2) quad(NQ - 2, 4, true, NGL, false, 0);
  quad(NQ - 1, NGL, false, 0, false, 0);
  // epilogue.  The item's output tile goes through LDS (the quad buffers,
  // free once every wave is past the last quad) and out as whole rows, 16
  // bytes per lane.  Gate/up with NB a multiple of 64 also does the down
  // kernel's input prep: h goes out in x_pairs order (feature f of an
  // 8-feature piece at 2 * (f % 4) + f / 4) with the sums of its bf16 values
  // over each 64-feature group (16 features per 16-lane row, then 4 column
  // blocks in order through LDS).  Down scales each row by its score.
  constexpr bool FUSE = GU && NB % 64 == 0;
  constexpr int OB = GU ? 2 : 4;                          // output bytes per element
  constexpr bool STAGE = ROWS * NB * OB <= (int)(4 * kTileM * 8 * sizeof(uint4));
  // the staged tile's element swizzle: XOR with 16 x ((row >> 2) & mask), the
  // mask kept so that an element never leaves its row (NB features)
  constexpr int SWM = NB % 64 == 0 ? 3 : NB % 32 == 0 ? 1 : 0;
  auto swz = [](int r) { return ((r >> 2) & SWM) << 4; };
  __syncthreads();
  char *tile = reinterpret_cast<char *>(L.a[0]);
#pragma unroll
  for (int cb = 0; cb < CPW; ++cb) {
    const int nl = (wave * CPW + cb) * 16 + col, n = nb0 + nl;
    const int npl = FUSE ? (nl & ~7) + ((nl & 3) << 1) + ((nl >> 2) & 1) : nl;
    float pb[NPROJ];
#pragma unroll
    for (int j = 0; j < NPROJ; ++j) {
      pb[j] = 0.f;
      if (PBIAS) {
        const int proj = GU ? (j == 0 ? PROJ_GATE : PROJ_UP) : PROJ_DOWN;
        pb[j] = bf16_to_f32(reinterpret_cast<const uint16_t *>(
            resolve(pa, comp_index(proj, PART_BIAS, NP), ref))[n]);
      }
    }
#pragma unroll
    for (int rb = 0; rb < NMB; ++rb) {
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        const int rr = rb * 16 + 4 * kq + e;   // (uniform over each 16-lane row)
        // staged tile: row rr, element npl ^ swz(rr) (the 4 rows of one
        // store fall on distinct banks)
        const int ec = npl ^ swz(rr);
        if (GU) {
          const float hv = apply_act(act, acc[rb][cb][0][e] + pb[0],
                                     acc[rb][cb][NPROJ - 1][e] + pb[NPROJ - 1], alpha, limit);
          const uint32_t hb = f32_to_bf16(hv);
          if (STAGE)
            reinterpret_cast<uint16_t *>(tile)[rr * NB + ec] = (uint16_t)hb;
          else if (rr < rows)
            h_out[(int64_t)(r0 + rr) * F + nb0 + npl] = (uint16_t)hb;
          if (FUSE) {
            const float ps = group_sum<16>(bf16_to_f32(hb));
            if (col == 0) L.part[(wave * CPW + cb) * kTileM + rr] = ps;
          }
        } else {
          const float v = acc[rb][cb][0][e] + pb[0];
          if (STAGE) {
            reinterpret_cast<float *>(tile)[rr * NB + ec] = L.rsc[rr] * v;
          } else if (rr < rows) {
            const int pr = L.rperm[rr];
            yp[(int64_t)pr * D + n] = L.rsc[rr] * v;
          }
        }
      }
    }
  }
  __syncthreads();
  if (STAGE) {   // whole rows out, 16 bytes per lane
    constexpr int CPR = NB * OB / 16;                     // 16-byte chunks per row
    constexpr int EPC = 16 / OB;                          // elements per chunk
    // (the thread index made opaque: the LDS addresses below are computed
    // here, not held in registers across the work items)
    int tid_e = tid;
    asm volatile("" : "+v"(tid_e));
#pragma unroll 1
    for (int it = 0; it < (ROWS * CPR + NT - 1) / NT; ++it) {
      const int i = tid_e + NT * it, r = i / CPR, c = i % CPR;
      if (i < ROWS * CPR && r < rows) {
        const int ec = (c * EPC) ^ swz(r);
        const uint4 v = *reinterpret_cast<const uint4 *>(tile + (r * NB + ec) * OB);
        if (GU)
          *reinterpret_cast<uint4 *>(h_out + (int64_t)(r0 + r) * F + nb0 + c * EPC) = v;
        else
          *reinterpret_cast<uint4 *>(yp + (int64_t)L.rperm[r] * D + nb0 + c * EPC) = v;
      }
    }
  }
  if (FUSE) {
#pragma unroll
    for (int i = tid; i < ROWS * (NB / 64); i += NT) {
      const int r = i % ROWS, gq = i / ROWS;
      if (r < rows) {
        float sm = 0.f;
#pragma unroll
        for (int c = 0; c < 4; ++c) sm += L.part[(gq * 4 + c) * kTileM + r];
        rs_out[(int64_t)(r0 + r) * (F / 64) + nb0 / 64 + gq] = sm;
      }
    }
  }
}

template <int D, int F, bool PBIAS, int NB, int WAVES, bool GU>
__global__ __launch_bounds__(64 * WAVES) __attribute__((amdgpu_waves_per_eu(WAVES == 8 && !GU ? 4 : 2))) void grouped_mm_kernel(
    PoolArgs pa, const uint16_t *__restrict__ aq, const float *__restrict__ ars, int k,
    const int32_t *__restrict__ perm, const int4 *__restrict__ tiles,
    const int32_t *__restrict__ n_tiles, uint16_t *__restrict__ h_out,
    float *__restrict__ rs_out, const float *__restrict__ scores, float *__restrict__ yp,
    int act, float alpha,
    float limit) {
  constexpr int KIN = GU ? D : F, NOUT = GU ? F : D, NPROJ = GU ? 2 : 1;
  constexpr int NBK = NOUT / NB, NP = PBIAS ? 4 : 3;
  using I = GItem<KIN, NB, WAVES, NPROJ>;
  static_assert(NOUT % NB == 0, "whole feature blocks");
  __shared__ uint4 a_l[4][kTileM * 8];
  __shared__ uint4 b_l[I::BROWS * 8];
  __shared__ float rs_l[I::NG4 * 4 * kRsPitch];
  __shared__ uint4 sc_l[I::QS ? (I::SQP + 1) / 2 : I::SCP];
  __shared__ float pt_l[GU && NB % 64 == 0 ? NB / 16 * kTileM : 1];
  __shared__ int rp_l[GU ? 1 : kTileM];
  __shared__ float rc_l[GU ? 1 : kTileM];
  const GLds L{pt_l, rp_l, rc_l, a_l, b_l, rs_l, sc_l};
  const int n_items = *n_tiles * NBK;
  for (int item = blockIdx.x; item < n_items; item += gridDim.x) {
    const int4 tl = tiles[item / NBK];
    const int ref = tl.x, r0 = tl.y, rows = tl.z;
    const int nb0 = (item % NBK) * NB;
    bool bad = false;
#pragma unroll
    for (int j = 0; j < NPROJ; ++j) {
      const int proj = GU ? (j == 0 ? PROJ_GATE : PROJ_UP) : PROJ_DOWN;
      bad = bad || resolve(pa, comp_index(proj, PART_W, NP), ref) == nullptr;
    }
    if (bad) {   // uniform over the workgroup
      if (threadIdx.x == 0) flag_error();
      continue;
    }
    const int nmb = (rows + 15) >> 4;
#define MOE_GITEM(M)                                                                      \
  grouped_item<M, D, F, PBIAS, NB, WAVES, GU>(pa, aq, ars, k, perm, ref, r0, rows, nb0, h_out, \
                                              rs_out, scores, yp, act, alpha, limit, L)
    if (nmb == 1) MOE_GITEM(1);
    else if (nmb == 2) MOE_GITEM(2);
    else if (nmb == 3) MOE_GITEM(3);
    else MOE_GITEM(4);
#undef MOE_GITEM
    __syncthreads();   // the LDS of this item is read before the next item stages
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
template <int D, int F, bool PB, int NBU, int WU>
static void launch_gg(dim3 g, hipStream_t s, const PoolArgs &pa, const uint16_t *xq,
                      const float *rsx, int k, const int32_t *perm, const int4 *tiles,
                      const int32_t *nt, uint16_t *h, float *rsh, int act, float alpha,
                      float limit) {
  hipLaunchKernelGGL((grouped_mm_kernel<D, F, PB, NBU, WU, true>), g, dim3(64 * WU), 0, s, pa,
                     xq, rsx, k, perm, tiles, nt, h, rsh, nullptr, nullptr, act, alpha, limit);
}
template <int D, int F, bool PB, int NBD, int WD>
static void launch_gd(dim3 g, hipStream_t s, const PoolArgs &pa, const uint16_t *hq,
                      const float *rsh, const float *sc, const int32_t *perm,
                      const int4 *tiles, const int32_t *nt, float *yp) {
  hipLaunchKernelGGL((grouped_mm_kernel<D, F, PB, NBD, WD, false>), g, dim3(64 * WD), 0, s,
                     pa, hq, rsh, 1, perm, tiles, nt, nullptr, nullptr, sc, yp, 0, 0.f, 0.f);
}

// (features per work item, waves) of gate/up and of down per geometry.  Only
// these shapes are validated (the grouped parity tests with tiles of 1 to 64
// rows); another shape that compiles is not known to be correct (down at
// (64, 4) was measured wrong at 64-row tiles).
#define MOE_GROUPED_GEOM(D, F, PB, NBU, WU, NBD, WD)                                     \
  {D, F, PB, NBU, NBD, &launch_gg<D, F, PB, NBU, WU>, &launch_gd<D, F, PB, NBD, WD>}
static const GroupedLaunch kGroupedTable[] = {
    MOE_GROUPED_GEOM(2048, 768, false, 64, 4, 128, 8),   // Qwen3-30B-A3B
    MOE_GROUPED_GEOM(2048, 768, true, 64, 4, 128, 8),
    MOE_GROUPED_GEOM(2880, 2880, true, 96, 6, 192, 6),   // gpt-oss-120b
    MOE_GROUPED_GEOM(2880, 2880, false, 96, 6, 192, 6),
    MOE_GROUPED_GEOM(256, 128, false, 128, 8, 128, 8),   // small test geometry
    MOE_GROUPED_GEOM(256, 128, true, 128, 8, 128, 8),
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
  w.off_xq = o; o += al((size_t)T * D * 2);
  w.off_rsx = o; o += al((size_t)T * (D / 64) * 4);
  w.off_hq = o; o += al((size_t)P * F * 2);
  w.off_rsh = o; o += al((size_t)P * (F / 64) * 4);
  w.total = o;
  return w;
}

// (in launches of at most 2^30 pieces, so the kernel's indices fit 32 bits)
static void launch_prep(const uint16_t *src, int64_t rows, int K, uint16_t *dst, float *rs,
                        hipStream_t s) {
  const int64_t chunk = ((int64_t)1 << 30) / (K / 8);
  for (int64_t r0 = 0; r0 < rows; r0 += chunk) {
    const int64_t nr = std::min(chunk, rows - r0);
    const int64_t n = nr * (K / 8);
    hipLaunchKernelGGL(grouped_prep_kernel, dim3((unsigned)((n + 255) / 256)), dim3(256), 0, s,
                       src + r0 * K, nr, K, dst + r0 * K, rs + r0 * (K / 64));
  }
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
  uint16_t *xq = reinterpret_cast<uint16_t *>(ws + w.off_xq);
  float *rsx = reinterpret_cast<float *>(ws + w.off_rsx);
  uint16_t *hq = reinterpret_cast<uint16_t *>(ws + w.off_hq);
  float *rsh = reinterpret_cast<float *>(ws + w.off_rsh);
  const int nkeys = pa.n_slots + pa.n_records;
  const int64_t xpieces = (int64_t)T * (D / 8);
  if (xpieces < ((int64_t)1 << 30)) {   // grouping and x prep in one launch
    hipLaunchKernelGGL(group_prep_kernel, dim3((unsigned)(1 + (xpieces + 1023) / 1024)), dim3(1024),
                       (size_t)nkeys * 4, s, refs, P, pa.n_slots, pa.n_records, D, perm, tiles,
                       ntiles, yp, x, (int64_t)T, xq, rsx);
  } else {
    hipLaunchKernelGGL(group_pairs_kernel, dim3(1), dim3(1024), (size_t)nkeys * 4, s, refs, P,
                       pa.n_slots, pa.n_records, D, perm, tiles, ntiles, yp);
    launch_prep(x, T, D, xq, rsx, s);
  }
  const int64_t items_up = w.max_tiles * (F / G->nb_up), items_down = w.max_tiles * (D / G->nb_down);
  const bool fused = G->nb_up % 64 == 0;   // gate/up writes hq and rsh itself
  G->gate_up(dim3((unsigned)std::min<int64_t>(items_up, kGroupedMaxWGs)), s, pa, xq, rsx, k, perm,
             tiles, ntiles, fused ? hq : h, fused ? rsh : nullptr, act, alpha, limit);
  if (!fused) launch_prep(h, P, F, hq, rsh, s);
  G->down(dim3((unsigned)std::min<int64_t>(items_down, kGroupedMaxWGs)), s, pa, hq, rsh, scores,
          perm, tiles, ntiles, yp);
  const int64_t n4 = (int64_t)T * D / 4;
  hipLaunchKernelGGL(combine_pairs_kernel, dim3((unsigned)((n4 + 255) / 256)), dim3(256), 0,
                     s, yp, T, k, D, out, out32);
}

}  // namespace moe
