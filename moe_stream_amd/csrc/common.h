// Device-side helpers shared by the gfx950 kernels of the expert hot path.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include "../../include/moe_stream.h"

namespace moe {

// Set by kernels when a slot reference is out of range for the pool view it
// is resolved against; read and cleared by moe_check_device_error().
extern __device__ int g_device_error;

typedef __bf16 bf16x2_t __attribute__((ext_vector_type(2)));
typedef uint32_t u32x4_t __attribute__((ext_vector_type(4)));

// 16-byte streaming load (weights are read once per launch).
// 16 bytes as one vector load into registers.  (Assigning the uint4 struct
// from memory is lowered to a memcpy that can keep a small array of them in
// scratch, whose later reload waits for every load issued before it.)
__device__ __forceinline__ uint4 load16(const uint4 *p) {
  u32x4_t v = *reinterpret_cast<const u32x4_t *>(p);
  return make_uint4(v.x, v.y, v.z, v.w);
}

// Loads through a pointer the compiler cannot place (one built from pool or
// store bases): as global loads.  A generic (flat) load also counts on the
// LDS counter, so every LDS wait (each workgroup barrier among them) would
// wait for it too.
typedef uint32_t u32x2_t __attribute__((ext_vector_type(2)));
__device__ __forceinline__ uint4 gload16(const void *p) {
  const u32x4_t v = *(const __attribute__((address_space(1))) u32x4_t *)(p);
  return make_uint4(v.x, v.y, v.z, v.w);
}
__device__ __forceinline__ uint2 gload8(const void *p) {
  const u32x2_t v = *(const __attribute__((address_space(1))) u32x2_t *)(p);
  return make_uint2(v.x, v.y);
}
__device__ __forceinline__ float gload4f(const void *p) {
  return *(const __attribute__((address_space(1))) float *)(p);
}
__device__ __forceinline__ int gload4i(const void *p) {
  return *(const __attribute__((address_space(1))) int *)(p);
}

__device__ __forceinline__ uint4 load_stream16(const uint4 *p) {
  u32x4_t v = __builtin_nontemporal_load(reinterpret_cast<const u32x4_t *>(p));
  return make_uint4(v.x, v.y, v.z, v.w);
}

// Keep memory instructions in program order across this point, both in the
// compiler's IR passes (the empty asm with a memory clobber) and in the
// machine scheduler (the scheduling barrier).  Emits no instruction and no
// wait: the loads issued before it stay in flight.
__device__ __forceinline__ void issue_order_fence() {
  asm volatile("" ::: "memory");
  __builtin_amdgcn_sched_barrier(0);
}

// --- bf16 <-> f32 -----------------------------------------------------------
__device__ __forceinline__ float bf16_to_f32(uint32_t bits16) {
  return __uint_as_float(bits16 << 16);
}
// round to nearest even (inputs are finite here; NaN stays NaN)
__device__ __forceinline__ uint32_t f32_to_bf16(float f) {
  uint32_t u = __float_as_uint(f);
  if ((u & 0x7fffffffu) > 0x7f800000u) return (u >> 16) | 0x40u;
  return (u + 0x7fffu + ((u >> 16) & 1u)) >> 16;
}
__device__ __forceinline__ float round_bf16(float f) {
  return bf16_to_f32(f32_to_bf16(f));
}

// v_dot2c_f32_bf16: acc + a.lo*b.lo + a.hi*b.hi, fp32 accumulation.
__device__ __forceinline__ float dot2_bf16(uint32_t a, uint32_t b, float acc) {
  return __builtin_amdgcn_fdot2_f32_bf16(__builtin_bit_cast(bf16x2_t, a),
                                         __builtin_bit_cast(bf16x2_t, b), acc,
                                         false);
}

// (w & M) | E in one v_bfi_b32 (E has no bits inside M).
__device__ __forceinline__ uint32_t bfi_mask(uint32_t w, uint32_t M, uint32_t E) {
  uint32_t r;
  asm("v_bfi_b32 %0, %1, %2, %3" : "=v"(r) : "v"(M), "v"(w), "v"(E));
  return r;
}

// Four packed bf16 pairs (128+q) from one word of eight 4-bit codes.  Pair m
// holds codes m (low half) and m+4 (high half): 0x4300 is bf16 128.0 and its
// 7-bit mantissa takes the code exactly, so no conversion instruction runs.
__device__ __forceinline__ void codes_to_bf16x2(uint32_t w, uint32_t p[4]) {
  const uint32_t M = 0x000f000fu, E = 0x43004300u;
  p[0] = bfi_mask(w, M, E);
  p[1] = bfi_mask(w >> 4, M, E);
  p[2] = bfi_mask(w >> 8, M, E);
  p[3] = bfi_mask(w >> 12, M, E);
}

// --- cross-lane reductions on DPP (no LDS round trip) -----------------------
template <int CTRL>
__device__ __forceinline__ float dpp_f(float v) {
  return __int_as_float(
      __builtin_amdgcn_update_dpp(0, __float_as_int(v), CTRL, 0xf, 0xf, false));
}
template <int CTRL>
__device__ __forceinline__ int dpp_i(int v) {
  return __builtin_amdgcn_update_dpp(0, v, CTRL, 0xf, 0xf, false);
}
constexpr int kDppQuadXor1 = 0xb1;      // quad_perm [1,0,3,2]
constexpr int kDppQuadXor2 = 0x4e;      // quad_perm [2,3,0,1]
constexpr int kDppHalfMirror = 0x141;   // row_half_mirror
constexpr int kDppMirror = 0x140;       // row_mirror
constexpr int kSwizzleXor16 = 0x401f;   // ds_swizzle bitmask mode, xor 16

__device__ __forceinline__ float swz_xor16_f(float v) {
  return __int_as_float(__builtin_amdgcn_ds_swizzle(__float_as_int(v), kSwizzleXor16));
}

// Eight consecutive bf16 activations (4 words) rearranged into the pair order
// of codes_to_bf16x2: out[m] = (x[m], x[m+4]).
__device__ __forceinline__ void x_pairs(const uint32_t in[4], uint32_t out[4]) {
  out[0] = (in[0] & 0xffffu) | (in[2] << 16);
  out[1] = (in[0] >> 16) | (in[2] & 0xffff0000u);
  out[2] = (in[1] & 0xffffu) | (in[3] << 16);
  out[3] = (in[1] >> 16) | (in[3] & 0xffff0000u);
}

// Sum over SG consecutive lanes (SG a power of two <= 64); every lane of the
// group ends with the total (each pairwise sum is commutative, so all lanes
// hold the identical value).  Quad and mirror DPP steps inside a 16-lane row,
// a swizzle across rows of 32, readlanes across halves of 64.
template <int SG>
__device__ __forceinline__ float group_sum(float v) {
  if (SG >= 2) v += dpp_f<kDppQuadXor1>(v);
  if (SG >= 4) v += dpp_f<kDppQuadXor2>(v);
  if (SG >= 8) v += dpp_f<kDppHalfMirror>(v);
  if (SG >= 16) v += dpp_f<kDppMirror>(v);
  if (SG == 32) v += swz_xor16_f(v);
  if (SG >= 64) {  // the four 16-lane rows through readlanes: a uniform value
    const float a = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), 0));
    const float b = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), 16));
    const float c = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), 32));
    const float d = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), 48));
    v = (a + b) + (c + d);
  }
  return v;
}

__device__ __forceinline__ float wave_max(float v) {
  v = fmaxf(v, dpp_f<kDppQuadXor1>(v));
  v = fmaxf(v, dpp_f<kDppQuadXor2>(v));
  v = fmaxf(v, dpp_f<kDppHalfMirror>(v));
  v = fmaxf(v, dpp_f<kDppMirror>(v));
  const float a = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), 0));
  const float b = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), 16));
  const float c = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), 32));
  const float d = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), 48));
  return fmaxf(fmaxf(a, b), fmaxf(c, d));
}

__device__ __forceinline__ int wave_max_i(int v) {
  v = max(v, dpp_i<kDppQuadXor1>(v));
  v = max(v, dpp_i<kDppQuadXor2>(v));
  v = max(v, dpp_i<kDppHalfMirror>(v));
  v = max(v, dpp_i<kDppMirror>(v));
  const int a = __builtin_amdgcn_readlane(v, 0), b = __builtin_amdgcn_readlane(v, 16);
  const int c = __builtin_amdgcn_readlane(v, 32), d = __builtin_amdgcn_readlane(v, 48);
  return max(max(a, b), max(c, d));
}

// Pool view passed to kernels by value.
struct PoolArgs {
  const char *base[MOE_MAX_COMPONENTS];
  int64_t slot_bytes[MOE_MAX_COMPONENTS];
  const char *store;
  int64_t record_bytes;
  int64_t comp_offset[MOE_MAX_COMPONENTS];
  int32_t n_slots;
  int32_t n_records;
};

// Slot references of one decode launch: a device array of T*k entries, or,
// with ptr == nullptr, at most MOE_MAX_TOPK entries carried in the kernel
// arguments (a host that holds the refs then launches without copying them
// to the device first).  The index is wave-uniform, so either form is one
// scalar load.
struct RefList {
  const int32_t *ptr;
  int32_t inl[MOE_MAX_TOPK];
  __device__ __forceinline__ int32_t operator[](int i) const {
    if (ptr != nullptr) return __builtin_amdgcn_readfirstlane(ptr[i]);
    return __builtin_amdgcn_readfirstlane(inl[i]);
  }
};

// Base address of component c for a slot reference; nullptr when the
// reference is out of range (the caller then contributes nothing and the
// device error word is set).
__device__ __forceinline__ const char *resolve(const PoolArgs &pa, int c,
                                               int32_t ref) {
  if (ref >= 0) {
    if (ref >= pa.n_slots) return nullptr;
    return pa.base[c] + (int64_t)ref * pa.slot_bytes[c];
  }
  int64_t r = -(int64_t)ref - 1;
  if (pa.store == nullptr || r >= pa.n_records) return nullptr;
  return pa.store + r * pa.record_bytes + pa.comp_offset[c];
}

// As resolve(), but an out-of-range reference yields slot 0 (or store record
// 0 when the pool has no slots; the host rejects a pool with neither) and
// clears `ok`: the kernel reads valid memory with no branch around its
// loads, then flags the error and contributes nothing.
__device__ __forceinline__ const char *resolve_safe(const PoolArgs &pa, int c, int32_t ref,
                                                    bool &ok) {
  const char *p = resolve(pa, c, ref);
  ok = p != nullptr;
  return ok ? p : (pa.n_slots > 0 ? pa.base[c] : pa.store + pa.comp_offset[c]);
}

// The packed pool layout of one geometry: per-component slot arrays
// [n_slots, *shape] with no padding and repacked store records (components
// back to back in (gate, up, down) x (weight, scales, biases[, bias]) order,
// the record padded to 16 KiB pages).  Strides and offsets are constants, so
// a kernel that requires this layout holds only the base addresses.
template <int D, int F, bool PB>
struct PackedLayout {
  static constexpr int NP = PB ? 4 : 3;
  static constexpr int64_t bytes(int c) {
    const int proj = c / NP, part = c % NP;
    const int64_t out = proj == 2 ? D : F, in = proj == 2 ? F : D;
    return part == 0 ? out * in / 2 : part == 3 ? out * 2 : out * (in / 64) * 2;
  }
  static constexpr int64_t slot_bytes(int c) { return bytes(c); }
  static constexpr int64_t comp_offset(int c) {
    int64_t o = 0;
    for (int i = 0; i < c; ++i) o += bytes(i);
    return o;
  }
  static constexpr int64_t kRecordBytes = (comp_offset(3 * NP) + 16383) / 16384 * 16384;
};

// resolve() / resolve_safe() for a pool in the packed layout L.
template <class L>
__device__ __forceinline__ const char *resolve_packed(const PoolArgs &pa, int c, int32_t ref) {
  if (ref >= 0) {
    if (ref >= pa.n_slots) return nullptr;
    return pa.base[c] + (int64_t)ref * L::slot_bytes(c);
  }
  int64_t r = -(int64_t)ref - 1;
  if (pa.store == nullptr || r >= pa.n_records) return nullptr;
  return pa.store + r * L::kRecordBytes + L::comp_offset(c);
}
template <class L>
__device__ __forceinline__ const char *resolve_packed_safe(const PoolArgs &pa, int c,
                                                           int32_t ref, bool &ok) {
  const char *p = resolve_packed<L>(pa, c, ref);
  ok = p != nullptr;
  return ok ? p : (pa.n_slots > 0 ? pa.base[c] : pa.store + L::comp_offset(c));
}

// Bits of the device error word.
constexpr int kErrBadRef = 1;    // a slot reference outside the pool view
constexpr int kErrTimeout = 2;   // a bounded cross-workgroup wait gave up

__device__ __forceinline__ void flag_error_bits(int bits) {
  __hip_atomic_fetch_or(&g_device_error, bits, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
// an out-of-range slot reference (the kernel contributes zeros for it)
__device__ __forceinline__ void flag_error() { flag_error_bits(kErrBadRef); }
// a bounded wait for another workgroup ran past its spin limit
__device__ __forceinline__ void flag_timeout() { flag_error_bits(kErrTimeout); }

// Component indices inside a pool view.
__host__ __device__ constexpr int comp_index(int proj, int part, int nparts) {
  return proj * nparts + part;
}
enum { PROJ_GATE = 0, PROJ_UP = 1, PROJ_DOWN = 2 };
enum { PART_W = 0, PART_S = 1, PART_B = 2, PART_BIAS = 3 };

}  // namespace moe
