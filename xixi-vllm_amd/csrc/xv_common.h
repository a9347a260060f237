// Shared device helpers for the gfx950 kernels: bf16 <-> fp32, 16-byte vector
// access, wave64 cross-lane reductions built on DPP row operations.
#pragma once
#include <hip/hip_runtime.h>
#include <stdint.h>

#define XV_INLINE __device__ __forceinline__

// Host-side layout checks of the 16-byte vector paths: a 16-byte aligned base
// (null allowed: unused operand) and strides in whole 8-element (16-byte) units.
static inline bool xv_al16(const void* p) { return ((uintptr_t)p & 15u) == 0; }
static inline bool xv_st8(int64_t s) { return (s & 7) == 0; }

typedef uint16_t bf16_t;  // raw bf16 bits as stored in HBM
typedef __bf16 bf16x8_t __attribute__((ext_vector_type(8)));
typedef float floatx4_t __attribute__((ext_vector_type(4)));

XV_INLINE float bf16_to_f32(uint32_t bits16) { return __uint_as_float(bits16 << 16); }
XV_INLINE float bf16lo(uint32_t w) { return __uint_as_float(w << 16); }
XV_INLINE float bf16hi(uint32_t w) { return __uint_as_float(w & 0xffff0000u); }

// fp32 -> bf16 with round-to-nearest-even (torch's rounding); NaN stays NaN.
// gfx950 converts in hardware (v_cvt_pk_bf16_f32, two values per instruction).
typedef __bf16 xv_bf16x2 __attribute__((ext_vector_type(2)));
typedef float xv_f32x2 __attribute__((ext_vector_type(2)));
XV_INLINE uint32_t pack_bf16x2(float lo, float hi) {
  const xv_bf16x2 h = __builtin_convertvector((xv_f32x2){lo, hi}, xv_bf16x2);
  uint32_t r;
  __builtin_memcpy(&r, &h, 4);
  return r;
}
XV_INLINE uint32_t f32_to_bf16(float f) { return pack_bf16x2(f, 0.f) & 0xffffu; }

// Eight bf16 values held as a 16-byte vector.
struct alignas(16) Vec8 {
  uint32_t w[4];
};
XV_INLINE Vec8 load_vec8(const bf16_t* p) {
  uint4 v = *reinterpret_cast<const uint4*>(p);
  Vec8 r; r.w[0] = v.x; r.w[1] = v.y; r.w[2] = v.z; r.w[3] = v.w; return r;
}
XV_INLINE void store_vec8(bf16_t* p, const Vec8& r) {
  *reinterpret_cast<uint4*>(p) = make_uint4(r.w[0], r.w[1], r.w[2], r.w[3]);
}
// Non-temporal streaming load for data read exactly once.
XV_INLINE Vec8 load_vec8_nt(const bf16_t* p) {
  typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
  u32x4 v = __builtin_nontemporal_load(reinterpret_cast<const u32x4*>(p));
  Vec8 r; r.w[0] = v[0]; r.w[1] = v[1]; r.w[2] = v[2]; r.w[3] = v[3]; return r;
}
// Non-temporal streaming store for data written once and not re-read soon.
// On this part nt loads and stores raise a plain stream copy from ~6.1 to
// ~6.6 TB/s.
XV_INLINE void store_vec8_nt(bf16_t* p, const Vec8& r) {
  typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
  u32x4 v = {r.w[0], r.w[1], r.w[2], r.w[3]};
  __builtin_nontemporal_store(v, reinterpret_cast<u32x4*>(p));
}
// An empty asm that reads and writes v's registers: v's load is complete and
// issued at this point in program order (the compiler may not sink it into a
// later branch).
XV_INLINE void pin_vec8(Vec8& v) {
  __asm__ __volatile__("" : "+v"(v.w[0]), "+v"(v.w[1]), "+v"(v.w[2]), "+v"(v.w[3]));
}
XV_INLINE void unpack8(const Vec8& v, float* f) {
#pragma unroll
  for (int i = 0; i < 4; ++i) { f[2 * i] = bf16lo(v.w[i]); f[2 * i + 1] = bf16hi(v.w[i]); }
}
XV_INLINE Vec8 pack8(const float* f) {
  Vec8 r;
#pragma unroll
  for (int i = 0; i < 4; ++i) r.w[i] = pack_bf16x2(f[2 * i], f[2 * i + 1]);
  return r;
}

// ---- DPP cross-lane moves (wave64, rows of 16 lanes) ----
// dpp_ctrl encodings (GCN/CDNA): quad_perm = 0x00-0xFF, row_ror:n = 0x120+n,
// row_bcast:15 = 0x142, row_bcast:31 = 0x143.
template <int CTRL>
XV_INLINE float dpp_f(float x) {
  return __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(x), CTRL, 0xf, 0xf, false));
}
// Sum / max over the 16 lanes of a DPP row; every lane of the row gets the result.
XV_INLINE float row16_sum(float x) {
  x += dpp_f<0x128>(x);   // row_ror:8
  x += dpp_f<0x124>(x);   // row_ror:4
  x += dpp_f<0x4E>(x);    // quad_perm [2,3,0,1]
  x += dpp_f<0xB1>(x);    // quad_perm [1,0,3,2]
  return x;
}
XV_INLINE float row16_max(float x) {
  x = fmaxf(x, dpp_f<0x128>(x));
  x = fmaxf(x, dpp_f<0x124>(x));
  x = fmaxf(x, dpp_f<0x4E>(x));
  x = fmaxf(x, dpp_f<0xB1>(x));
  return x;
}
// max(x[l], x[l ^ 16]) and max(x[l], x[l ^ 32]) with the gfx950 row-swap
// permutes (VALU, no LDS round trip).  permlane16_swap exchanges the odd
// 16-lane rows of its first operand with the even rows of its second, so with
// both operands = x each lane ends up holding x[l] in one result and
// x[l ^ 16] in the other; permlane32_swap does the same across halves.
XV_INLINE float xor16_max(float x) {
  const auto r = __builtin_amdgcn_permlane16_swap(__float_as_uint(x), __float_as_uint(x), false, false);
  return fmaxf(__uint_as_float(r[0]), __uint_as_float(r[1]));
}
XV_INLINE float xor32_max(float x) {
  const auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(x), __float_as_uint(x), false, false);
  return fmaxf(__uint_as_float(r[0]), __uint_as_float(r[1]));
}
XV_INLINE float xor16_sum(float x) {
  const auto r = __builtin_amdgcn_permlane16_swap(__float_as_uint(x), __float_as_uint(x), false, false);
  return __uint_as_float(r[0]) + __uint_as_float(r[1]);
}
XV_INLINE float xor32_sum(float x) {
  const auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(x), __float_as_uint(x), false, false);
  return __uint_as_float(r[0]) + __uint_as_float(r[1]);
}
// Lane n of each 16-lane row, broadcast to the row (DPP row_newbcast).
template <int N>
XV_INLINE float row_bcast(float x) {
  return __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(x), 0x150 + N, 0xf, 0xf, false));
}
// Full wave64 reductions (result valid in every lane), all in registers.
XV_INLINE float wave_sum(float x) { return xor32_sum(xor16_sum(row16_sum(x))); }
XV_INLINE float wave_max(float x) { return xor32_max(xor16_max(row16_max(x))); }

#define XV_CHECK_LAUNCH() do { hipError_t e_ = hipGetLastError(); if (e_ != hipSuccess) return (int)e_; } while (0)
