// Device-side building blocks shared by the gfx950 attention kernels.
//
// Wave64 MFMA layouts used throughout (checked on gfx950 hardware):
//   v_mfma_f32_32x32x16_{bf16,f16}:  A lane l holds A[m = l%32][k = 8*(l/32) + 0..7],
//     B lane l holds B[k = 8*(l/32) + 0..7][n = l%32],
//     C lane l holds C[m = 8*(i/4) + 4*(l/32) + i%4][n = l%32] for i = 0..15.
//   ds_read_b64_tr_b16: in each 16-lane group, lane j gives the address of
//     row j/4, columns 4*(j%4)..+3 of a 4 x 16 block of 16-bit values and
//     receives column j, rows 0..3.
//   v_permlane32_swap(x, x) returns {x[l%32], x[l%32 + 32]} in every lane.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

namespace fa {

typedef __bf16 bf16;
typedef _Float16 f16;
typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef float f32x16 __attribute__((ext_vector_type(16)));
typedef short s16x4 __attribute__((ext_vector_type(4)));
typedef short s16x8 __attribute__((ext_vector_type(8)));
typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef _Float16 f16x8 __attribute__((ext_vector_type(8)));
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
typedef uint32_t u32x2 __attribute__((ext_vector_type(2)));

// 64-bit minimum: the HIP headers' min overloads differ between the host and
// device passes (the host pass picks min(int, int) for two int64_t).
__host__ __device__ __forceinline__ int64_t min_i64(int64_t x, int64_t y) { return x < y ? x : y; }

template <typename T> struct Vec8;
template <> struct Vec8<bf16> { typedef bf16x8 type; };
template <> struct Vec8<f16> { typedef f16x8 type; };

#define FA_LDS __attribute__((address_space(3)))

constexpr float kNegInf = -__builtin_huge_valf();
constexpr float kPosInf = __builtin_huge_valf();
constexpr float kLog2e = 1.4426950408889634f;

__device__ __forceinline__ f32x16 mfma32(bf16x8 a, bf16x8 b, f32x16 c) {
  return __builtin_amdgcn_mfma_f32_32x32x16_bf16(a, b, c, 0, 0, 0);
}
__device__ __forceinline__ f32x16 mfma32(f16x8 a, f16x8 b, f32x16 c) {
  return __builtin_amdgcn_mfma_f32_32x32x16_f16(a, b, c, 0, 0, 0);
}

// 16-byte vector <-> 8 elements.
template <typename T>
__device__ __forceinline__ typename Vec8<T>::type as_vec8(u32x4 x) {
  return __builtin_bit_cast(typename Vec8<T>::type, x);
}
template <typename T>
__device__ __forceinline__ u32x4 as_u32x4(typename Vec8<T>::type x) {
  return __builtin_bit_cast(u32x4, x);
}

// Pack 8 fp32 values into 8 x T (round to nearest even).
template <typename T>
__device__ __forceinline__ typename Vec8<T>::type pack8(float x0, float x1, float x2, float x3, float x4,
                                                          float x5, float x6, float x7) {
  typename Vec8<T>::type r;
  r[0] = (T)x0; r[1] = (T)x1; r[2] = (T)x2; r[3] = (T)x3;
  r[4] = (T)x4; r[5] = (T)x5; r[6] = (T)x6; r[7] = (T)x7;
  return r;
}

// Two fp32 values as a pair of 16-bit T (round to nearest even) in *hi and
// the rounding residuals (exact in fp32), rounded, in *lo: hi + lo carries
// each value to about 16 significant bits.
template <typename T>
__device__ __forceinline__ void split2(float x0, float x1, uint32_t* hi, uint32_t* lo) {
  typedef T T2 __attribute__((ext_vector_type(2)));
  T2 h;
  h[0] = (T)x0;
  h[1] = (T)x1;
  const uint32_t w = __builtin_bit_cast(uint32_t, h);
  float f0, f1;
  if constexpr (sizeof(T) == 2 && __is_same(T, __bf16)) {
    f0 = __uint_as_float(w << 16);
    f1 = __uint_as_float(w & 0xffff0000u);
  } else {
    f0 = (float)(T)x0;
    f1 = (float)(T)x1;
  }
  T2 l;
  l[0] = (T)(x0 - f0);
  l[1] = (T)(x1 - f1);
  *hi = w;
  *lo = __builtin_bit_cast(uint32_t, l);
}

// The same with a second residual: hi + lo + lo2 carries each value to about
// 24 significant bits (all of an fp32 value's).
template <typename T>
__device__ __forceinline__ void split3(float x0, float x1, uint32_t* hi, uint32_t* lo, uint32_t* lo2) {
  typedef T T2 __attribute__((ext_vector_type(2)));
  auto pack = [](float a, float b) {
    T2 v;
    v[0] = (T)a;
    v[1] = (T)b;
    return __builtin_bit_cast(uint32_t, v);
  };
  auto lo_f = [](uint32_t w, float a) {   // the low element of a pair as fp32
    if constexpr (__is_same(T, __bf16)) return __uint_as_float(w << 16);
    else return (float)(T)a;
  };
  auto hi_f = [](uint32_t w, float b) {   // the high element
    if constexpr (__is_same(T, __bf16)) return __uint_as_float(w & 0xffff0000u);
    else return (float)(T)b;
  };
  const uint32_t w = pack(x0, x1);
  const float r0 = x0 - lo_f(w, x0), r1 = x1 - hi_f(w, x1);
  const uint32_t l = pack(r0, r1);
  *hi = w;
  *lo = l;
  *lo2 = pack(r0 - lo_f(l, r0), r1 - hi_f(l, r1));
}

// Transposed LDS read of 4 x 16-bit values (see the header comment).
__device__ __forceinline__ s16x4 lds_read_tr(const void* p) {
  return __builtin_amdgcn_ds_read_tr16_b64_v4i16((FA_LDS s16x4*)(uintptr_t)p);
}
template <typename T>
__device__ __forceinline__ typename Vec8<T>::type cat_tr(s16x4 lo, s16x4 hi) {
  s16x8 r = __builtin_shufflevector(lo, hi, 0, 1, 2, 3, 4, 5, 6, 7);
  return __builtin_bit_cast(typename Vec8<T>::type, r);
}

__device__ __forceinline__ u32x4 lds_read16(const void* p) {
  return *(const FA_LDS u32x4*)(uintptr_t)p;
}
__device__ __forceinline__ void lds_write16(void* p, u32x4 v) {
  *(FA_LDS u32x4*)(uintptr_t)p = v;
}
__device__ __forceinline__ void lds_write8(void* p, u32x2 v) {
  *(FA_LDS u32x2*)(uintptr_t)p = v;
}

__device__ __forceinline__ u32x4 gload16(const void* p) {
  return *(const u32x4*)p;
}
__device__ __forceinline__ void gstore16(void* p, u32x4 v) {
  *(u32x4*)p = v;
}

// Partner value from the other 32-lane half (lane l^32), as a pair that holds
// both halves' values in every lane.
__device__ __forceinline__ float half_max(float x) {
  auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(x), __float_as_uint(x), false, false);
  return fmaxf(__uint_as_float(r[0]), __uint_as_float(r[1]));
}
__device__ __forceinline__ float half_sum(float x) {
  auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(x), __float_as_uint(x), false, false);
  return __uint_as_float(r[0]) + __uint_as_float(r[1]);
}

__device__ __forceinline__ float exp2_fast(float x) { return __builtin_amdgcn_exp2f(x); }
__device__ __forceinline__ float log2_fast(float x) { return __builtin_amdgcn_logf(x); }

__device__ __forceinline__ bool wave_any(bool p) {
  return __builtin_amdgcn_ballot_w64(p) != 0;
}

// XOR swizzle of 16-byte chunks within a row of a [rows][D] 16-bit LDS tile.
// Chosen so that (a) 16 lanes reading one chunk of 16 consecutive rows with
// ds_read_b128 and (b) 32 lanes doing the ds_read_b64_tr_b16 pattern over 4
// consecutive rows (row % 4 == 0) and 4 consecutive chunks (chunk % 4 == 0) hit
// distinct banks.
template <int W>
__device__ __forceinline__ int chunk_swz(int r) {
  static_assert(W == 64 || W == 128, "tile width");
  if constexpr (W == 128) return ((r & 3) << 2) | ((r >> 2) & 3);
  else return (((r >> 1) & 1) << 2) | ((r >> 2) & 3);
}
// Element offset of (row r, column c) in a swizzled [rows][W] tile.
template <int W>
__device__ __forceinline__ int tile_off(int r, int c) {
  return r * W + ((((c >> 3) ^ chunk_swz<W>(r))) << 3) + (c & 7);
}

// Maps a 1-D block index onto a logical work index so that consecutive
// logical indices land on the same XCD (hardware dispatches block L to XCD
// L % 8): XCD x receives the contiguous logical range starting at
// x*(n/8) + min(x, n%8).
__device__ __forceinline__ int xcd_remap(int L, int n) {
  const int q = n >> 3, r = n & 7;
  const int x = L & 7, s = L >> 3;
  return x * q + (x < r ? x : r) + s;
}

}  // namespace fa
