// Kernel argument blocks and launcher declarations (internal to the library).
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

namespace fa {

// Work shapes the prepared-mask lists are built for (each kernel asserts its own).
constexpr int kFwdRows = 256;    // forward: query rows per workgroup
constexpr int kFwdKeys = 64;     //          keys per tile
constexpr int kKv2Keys = 128;    // dK/dV (deterministic): keys per workgroup, 32-row steps
constexpr int kDqDsRows = 256;   // dQ from dS: query rows per workgroup, 32-key steps
constexpr int kDqDsRowsWide = 512;   // the same with 8 waves (deterministic, D 128, no mask)

// Prepared mask (workspace written by fa_mask_prepare from the bool mask).
// One plane per (mask batch, mask head): Bm = 1 when the mask's batch stride
// is 0 (broadcast), else B; Hm likewise over the query heads.  Per plane:
//   bits   uint32 [Tq][wk]      bit j%32 of word j/32 = keep(i, j); zero past Tk
//   bitsT  uint32 [nk32][wq][32] word (j/32, i/32, j%32): bit i%32 = keep(i, j);
//                               zero past Tq (32 keys of one row word: one 128-byte line)
//   blk    uint8  [nq32][nk32]  32x32 block: 0 no kept entry, 1 some, 2 all (in bounds)
//   lfwd   int32  [nfq][1+nft]  per 256-row block: count, then the live 64-key
//                               tiles ascending, bit 31 set when every block is 2
//   lkv    int32  [nkb][1+nq32] per 128-key block: count, live 32-row steps
//   ldq    int32  [ndq][1+nk32] per 256-row block: count, live 32-key steps
//   ord    int32  [nfq + nkb + ndq] the units of lfwd, lkv, ldq (in that order)
//                               by count, largest first, ties by unit: the
//                               kernels run their longest workgroups first
//   hist   int32  [nft+1 + nq32+1 + nk32+1]  scratch of the ordering: per list
//                               kind a histogram of the counts (0 .. its
//                               largest possible count), then bin offsets
// "Live" folds in causality when the workspace was prepared with is_causal.
struct MaskLayout {
  int Bm, Hm;
  int nq32, nk32, wk, wq;
  int nfq, nft, nkb, ndq;
  int64_t bits, bitsT, blk, lfwd, lkv, ldq, ord, hist, total;   // byte offsets of the plane arrays, workspace size
  int64_t pbits, pbitsT, pblk, plfwd, plkv, pldq, pord, phist;  // per-plane sizes (bytes)
};

__host__ __device__ inline int64_t align256(int64_t x) { return (x + 255) & ~(int64_t)255; }

__host__ __device__ inline MaskLayout mask_layout(int B, int Hq, int Tq, int Tk, bool bcast_b, bool bcast_h) {
  MaskLayout m{};
  m.Bm = bcast_b ? 1 : B;
  m.Hm = bcast_h ? 1 : Hq;
  m.nq32 = (Tq + 31) / 32;
  m.nk32 = (Tk + 31) / 32;
  m.wk = (m.nk32 + 3) & ~3;
  m.wq = (m.nq32 + 3) & ~3;
  m.nfq = (Tq + kFwdRows - 1) / kFwdRows;
  m.nft = (Tk + kFwdKeys - 1) / kFwdKeys;
  m.nkb = (Tk + kKv2Keys - 1) / kKv2Keys;
  m.ndq = (Tq + kDqDsRows - 1) / kDqDsRows;
  m.pbits = (int64_t)Tq * m.wk * 4;
  m.pbitsT = (int64_t)m.nk32 * m.wq * 32 * 4;
  m.pblk = (int64_t)m.nq32 * m.nk32;
  m.plfwd = (int64_t)m.nfq * (1 + m.nft) * 4;
  m.plkv = (int64_t)m.nkb * (1 + m.nq32) * 4;
  m.pldq = (int64_t)m.ndq * (1 + m.nk32) * 4;
  m.pord = (int64_t)(m.nfq + m.nkb + m.ndq) * 4;
  m.phist = (int64_t)(m.nft + 1 + m.nq32 + 1 + m.nk32 + 1) * 4;
  const int64_t np = (int64_t)m.Bm * m.Hm;
  m.bits = 0;
  m.bitsT = align256(m.bits + np * m.pbits);
  m.blk = align256(m.bitsT + np * m.pbitsT);
  m.lfwd = align256(m.blk + np * m.pblk);
  m.lkv = align256(m.lfwd + np * m.plfwd);
  m.ldq = align256(m.lkv + np * m.plkv);
  m.ord = align256(m.ldq + np * m.pldq);
  m.hist = align256(m.ord + np * m.pord);
  m.total = align256(m.hist + np * m.phist);
  return m;
}

// Count order of list kind `kind` (0 lfwd, 1 lkv, 2 ldq) of plane pm: entry
// r is the unit with the r-th largest count.
__host__ __device__ inline const int32_t* mask_order(const MaskLayout& m, const char* ws, int pm, int kind) {
  return (const int32_t*)(ws + m.ord + pm * m.pord) + (kind == 0 ? 0 : (kind == 1 ? m.nfq : m.nfq + m.nkb));
}

// Plane of (batch b, query head h).
__host__ __device__ inline int mask_plane(const MaskLayout& m, int b, int h) {
  return (m.Bm == 1 ? 0 : b) * m.Hm + (m.Hm == 1 ? 0 : h);
}

struct MaskArgs {
  const uint8_t* mask;
  int64_t msb, msh, msq;
  int Tq, Tk;
  int is_causal;
  int vec16;            // rows 16-byte aligned: 128-bit loads allowed
  char* ws;
  MaskLayout ml;
};

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
  const char* mws;      // prepared mask (with a mask)
  MaskLayout ml;
  void* olo;            // optional (mask or score): O's rounding residual, dtype, strided like O
  int64_t olsb, olst, olsh;
};

struct PreArgs {
  const void* o; const void* dout; const float* lse;
  float* delta;         // Delta [B, Hq, Tq]
  float* lse_b;         // LSE the backward kernels use [B, Hq, Tq]: the forward's, except
                        // -inf for a row whose kept keys all have -inf logits
  int32_t* dead; float* dq_accum;
  int64_t osb, ost, osh, dsb, dst, dsh;
  const void* olo;      // optional: O's rounding residual (Delta = sum dO (O + olo))
  int64_t olsb, olst, olsh;
  int B, Tq, Hq, Hk, G;
  int is_causal;
  const char* mws;      // prepared mask (with a mask): tells rows without a kept key
  MaskLayout ml;
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
  // (batch, kv-head) units bk = b Hk + kv-head of this launch: bk0 ..
  // bk0 + nbk - 1 of the B Hk.  The dS-tile kernels run in slices of units
  // when the tiles of all units exceed the workspace; the workspace then
  // holds the planes of the slice, from unit bk0 on.  Others: 0, B Hk.
  int bk0, nbk;
  // Query steps (32 rows) of this launch: [q32_lo, q32_hi).  The dS-tile
  // kernels run in ranges of rows when not even one unit's tiles fit the
  // workspace; its planes then hold the tiles of those steps only, step s at
  // ds_row(s) - ds_row(q32_lo).  Others: 0, nq32.
  int q32_lo, q32_hi;
  // dK/dV kernel over row ranges: 0 writes dK/dV, or with a head-group split
  // its part's fp32 slab (the whole row range in one launch); 1 writes the
  // fp32 sums dk_accum/dv_accum [B, Tk, Hk, D] (a slab per part with a split)
  // (first range), 2 adds to them, 3 adds them and writes dK/dV (last range,
  // split 1).
  int acc_mode;
  // Slices within a head group: the dK/dV kernel runs parts sp0 .. sp0 +
  // nsp - 1 of its head-group split, the dQ kernel heads g0 .. g0 + ng - 1
  // of each group; the workspace's first dS plane is (b Hq + h) = ds_p0.
  // Others: 0, split, 0, G, bk0 G.
  int sp0, nsp, g0, ng;
  int64_t ds_p0;
  int nqt;              // query tiles per (b, h) (dQ kernel)
  int dq_rows;          // query rows per dQ-from-dS workgroup: kDqDsRows or kDqDsRowsWide
  int split;            // query-head-group split of the dK/dV kernel
  int do_dq;            // dQ accumulated with fp32 atomics into dq_accum (by the dQ-from-dS
                        // kernel over dq_split key ranges)
  int dq_split;         // key ranges of the atomic dQ-from-dS kernel
  float scale;          // softmax scale (dS multiplier)
  float scale_log2;     // |scale| * log2(e)  (1 when zero_scale)
  float qsign;
  int zero_scale;
  // dS tiles (written by the dK/dV kernel, read by the dQ kernel); null when
  // dQ is recomputed instead.  Tile (b, h, s, kb) holds dS / scale of query
  // rows 32 s.. and keys 32 kb.. as 32 key rows of 32 16-bit values stored
  // chunk-major (16-byte chunk c of key row k at byte c 512 + k 16), element
  // offset of the tile ((b Hq + h) ds_plane + ds_row(s) + kb) * 1024.
  void* ds;
  int64_t ds_plane;     // tiles per (b, h)
  int nq32, nk32;       // 32-row / 32-key steps
  const char* mws;      // prepared mask (with a mask; the deterministic kernels read it)
  MaskLayout ml;
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
hipError_t launch_bwd_dq(const BwdArgs& a, int D, int dtype, bool causal, hipStream_t s);
// dK/dV of the deterministic path (no dQ), 4 waves x 32 keys per workgroup.
hipError_t launch_bwd_dkdv2(const BwdArgs& a, int D, int dtype, bool causal, hipStream_t s);
int dkdv2_block_keys();
// dQ = scale * dS K from the dS tiles, 256 query rows per workgroup.
hipError_t launch_bwd_dq_ds(const BwdArgs& a, int D, int dtype, bool causal, hipStream_t s);
hipError_t launch_convert(const CvtArgs& a, int dtype, hipStream_t s);
// Head dim 256 (fa_wide.hip): forward, 128 query rows per workgroup; dK and
// dV in two launches over 128-key workgroups (grid nbk x nkt x split, dK/dV
// written like the dK/dV kernel's: dtype, or fp32 slabs with a split).
hipError_t launch_fwd_wide(const FwdArgs& a, int dtype, bool causal, hipStream_t s);
hipError_t launch_bwd_kv_wide(const BwdArgs& a, int dtype, bool causal, hipStream_t s);
// dQ recomputed at head dim 256, 128 query rows per workgroup (grid B Hq nqt).
hipError_t launch_bwd_dq_wide(const BwdArgs& a, int dtype, bool causal, hipStream_t s);
int fwd_wide_block_rows();
int dq_wide_block_rows();
int kv_wide_block_keys();
// Bool mask -> prepared mask workspace (bits, transposed bits, block states, lists).
hipError_t launch_mask_prepare(const MaskArgs& a, hipStream_t s);

}  // namespace fa
