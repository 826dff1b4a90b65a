// Kernel argument blocks and launcher declarations (internal to the library).
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

namespace fa {

struct FwdArgs {
  const void* q; const void* k; const void* v; void* o; float* lse;
  const uint8_t* mask; const float* score;
  int64_t qsb, qst, qsh, ksb, kst, ksh, vsb, vst, vsh, osb, ost, osh;
  int64_t msb, msh, msq, ssb, ssh, ssq;
  int B, Tq, Tk, Hq, Hk, G;
  int nqt;              // query tiles per (b, h)
  float scale_log2;     // |scale| * log2(e)  (1 when zero_scale)
  float qsign;          // -1 folds a negative scale into Q and Score
  int zero_scale;       // scale == 0: every kept logit is 0
  int mask_vec;         // mask rows 4-byte aligned: 32-bit loads allowed
  int score_vec;        // score rows 16-byte aligned: 128-bit loads allowed
};

struct PreArgs {
  const void* o; const void* dout; const float* lse;
  float* delta; int32_t* dead; float* dq_accum;
  int64_t osb, ost, osh, dsb, dst, dsh;
  int B, Tq, Hq, Hk, G;
};

struct BwdArgs {
  const void* q; const void* k; const void* v; const void* dout;
  const float* lse; const float* delta; const int32_t* dead;
  const uint8_t* mask; const float* score;
  float* dq_accum; float* dk_accum; float* dv_accum;
  void* dk; void* dv; void* dq;
  int64_t qsb, qst, qsh, ksb, kst, ksh, vsb, vst, vsh, dsb, dst, dsh;
  int64_t dqsb, dqst, dqsh, dksb, dkst, dksh, dvsb, dvst, dvsh;
  int64_t msb, msh, msq, ssb, ssh, ssq;
  int B, Tq, Tk, Hq, Hk, G;
  int nkt;              // key tiles per (b, kv-head)
  int nqt;              // query tiles per (b, h) (dQ kernel)
  int split;            // query-head-group split of the dK/dV kernel
  int do_dq;            // dK/dV kernel also accumulates dQ with fp32 atomics
  float scale;          // softmax scale (dS multiplier)
  float scale_log2;     // |scale| * log2(e)  (1 when zero_scale)
  float qsign;
  int zero_scale;
  int mask_vec, score_vec;
  // dS tiles of the deterministic path (written by the dK/dV kernel, read by
  // the dQ kernel); null when dQ is recomputed instead.  Tile (b, h, s, kb)
  // holds dS / scale of query rows 32 s.. and keys 32 kb.. as [key][32] 16-bit
  // values, element offset ((b Hq + h) ds_plane + ds_row(s) + kb) * 1024.
  void* ds;
  int64_t ds_plane;     // tiles per (b, h)
  int nq32, nk32;       // 32-row / 32-key steps
};

// First tile of query step s in a (b, h) plane of dS tiles: causal planes
// keep tiles kb <= s only (and kb < nk32), full planes keep every kb < nk32.
__host__ __device__ inline int64_t ds_row(int64_t s, int64_t nk32, bool causal) {
  if (!causal) return s * nk32;
  return s <= nk32 ? s * (s + 1) / 2 : nk32 * (nk32 + 1) / 2 + (s - nk32) * nk32;
}

struct CvtArgs {
  const float* src;      // nsplit fp32 slabs, element (b, t, h, d) at b*src_sb + t*src_st + h*src_sh + d
  void* dst;             // dtype, strided
  int64_t sb, st, sh;
  int B, T, H, D;
  int nsplit;            // number of slabs summed (1 = plain conversion)
  int64_t split_stride;  // elements between slabs
  int64_t src_sb, src_st, src_sh;
};

hipError_t launch_fwd(const FwdArgs& a, int D, int dtype, bool causal, hipStream_t s);
hipError_t launch_preprocess(const PreArgs& a, int D, int dtype, hipStream_t s);
hipError_t launch_bwd_dkdv(const BwdArgs& a, int D, int dtype, bool causal, hipStream_t s);
hipError_t launch_bwd_dq(const BwdArgs& a, int D, int dtype, bool causal, hipStream_t s);
// dK/dV of the deterministic path (no dQ), 4 waves x 32 keys per workgroup.
hipError_t launch_bwd_dkdv2(const BwdArgs& a, int D, int dtype, bool causal, hipStream_t s);
int dkdv2_block_keys();
// dQ = scale * dS K from the dS tiles, 256 query rows per workgroup.
hipError_t launch_bwd_dq_ds(const BwdArgs& a, int D, int dtype, bool causal, hipStream_t s);
int dq_ds_block_rows();
hipError_t launch_convert(const CvtArgs& a, int dtype, hipStream_t s);

}  // namespace fa
