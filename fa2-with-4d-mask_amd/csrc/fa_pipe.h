// Helpers of the software-pipelined backward kernels (one wave per SIMD,
// MFMA work of neighbouring steps interleaved with the VALU work of the
// current one): LDS access by raw byte address, the shared tile swizzle, and
// the MFMA form that keeps its accumulator in AGPRs.
#pragma once

#include "fa_common.h"

namespace fa {
namespace pipe {

template <int N> struct IC { static constexpr int value = N; };

// Chunk swizzle of a [32][D] 16-bit tile (16-byte chunks).  ds_read_b128 of
// one chunk over 16 consecutive rows and ds_read_b64_tr_b16 over rows
// 4 r0 .. 4 r0 + 3 x chunks 4 m .. 4 m + 3 both hit 64 distinct banks.
template <int D> __device__ __forceinline__ int swz_q(int r) {
  return D == 128 ? (((r & 3) << 2) | ((r >> 2) & 3)) : ((((r >> 1) & 1) << 2) | ((r >> 2) & 3));
}

__device__ __forceinline__ uint32_t opaque(uint32_t x) {
  asm volatile("" : "+v"(x));
  return x;
}
__device__ __forceinline__ u32x4 lds_rd16(uint32_t addr) { return *(const FA_LDS u32x4*)(uintptr_t)addr; }
__device__ __forceinline__ f32x4 lds_rdf4(uint32_t addr) { return *(const FA_LDS f32x4*)(uintptr_t)addr; }
__device__ __forceinline__ s16x4 lds_rdtr(uint32_t addr) {
  return __builtin_amdgcn_ds_read_tr16_b64_v4i16((FA_LDS s16x4*)(uintptr_t)addr);
}
__device__ __forceinline__ void lds_wr16(uint32_t addr, u32x4 v) { *(FA_LDS u32x4*)(uintptr_t)addr = v; }
__device__ __forceinline__ void lds_wrf(uint32_t addr, float v) { *(FA_LDS float*)(uintptr_t)addr = v; }
__device__ __forceinline__ void lds_wr8(uint32_t addr, u32x2 v) { *(FA_LDS u32x2*)(uintptr_t)addr = v; }

__device__ __forceinline__ void lds_barrier() {
  __builtin_amdgcn_sched_barrier(0);
  asm volatile("s_waitcnt lgkmcnt(0)\n\ts_barrier" ::: "memory");
  __builtin_amdgcn_sched_barrier(0);
}

// Output-gradient accumulation: MFMA with the accumulator pinned to AGPRs.
// The other MFMAs (compiler builtins, built in VGPR form for the files that
// use this) then leave their results in VGPRs, where the VALU work reads them
// without copies.  Callers pass A from an LDS read (the compiler places the
// wait for it before the asm) and B produced at least one pipeline iteration
// earlier, touch each accumulator only through this function, several MFMAs
// apart, and wait MFMA-to-VALU states (mfma_acc_drain) before reading it.
__device__ __forceinline__ void mfma_acc(f32x16& acc, bf16x8 a, bf16x8 b) {
  asm volatile("v_mfma_f32_32x32x16_bf16 %0, %1, %2, %0" : "+a"(acc) : "v"(a), "v"(b));
}
__device__ __forceinline__ void mfma_acc(f32x16& acc, f16x8 a, f16x8 b) {
  asm volatile("v_mfma_f32_32x32x16_f16 %0, %1, %2, %0" : "+a"(acc) : "v"(a), "v"(b));
}

template <typename T>
__device__ __forceinline__ u32x2 pack4(float x0, float x1, float x2, float x3) {
  typedef T T4 __attribute__((ext_vector_type(4)));
  T4 v;
  v[0] = (T)x0; v[1] = (T)x1; v[2] = (T)x2; v[3] = (T)x3;
  return __builtin_bit_cast(u32x2, v);
}

// Wait states after the last mfma_acc before its accumulator is read by
// other instructions (the compiler does not see the asm as an MFMA).
__device__ __forceinline__ void mfma_acc_drain() { asm volatile("s_nop 7\n\ts_nop 7\n\ts_nop 7" ::: "memory"); }

}  // namespace pipe
}  // namespace fa
