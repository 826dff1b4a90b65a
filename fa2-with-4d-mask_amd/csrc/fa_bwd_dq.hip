// dQ of the deterministic FlashAttention-2 backward for gfx950 (MI355X), from
// the dS tiles the dK/dV kernel writes:
//   dQ = scale * dS K,   dS = P (dP - Delta) per (query row, key)
// which is the dQ part of the reference's TileLang backward
// (python/fa2.py:181-302, 305-426: dq = dS K accumulated over key blocks).
// Storing dS (16-bit, the precision the dQ MFMA consumes anyway) replaces the
// second evaluation of S, P and dP that a separate dQ kernel would need: this
// kernel is one streaming pass over the dS tiles with a small GEMM on top.
//
// dS tile (b, h, s, kb): 32 keys x 32 query rows, row "key" of 64 bytes whose
// 16-bit entries hold, at position p, query row
//   perm(p) = 16 (p / 16) + 4 ((p / 8) % 2) + 8 ((p / 4) % 2) + p % 4
// (the order in which the dK/dV kernel's lanes hold them).  In memory the
// tile is chunk-major: 16-byte chunk c of key row k at byte c 512 + k 16 (the
// dK/dV kernel then writes whole lines).  In LDS it stays chunk-major, with
// the key index of chunk c XOR-ed with 4 c: chunk c of key k at byte
// c 512 + (k ^ 4 c) 16.  A staging write (16 lanes: 16 keys of one chunk)
// then covers one 256-byte span, and a transpose read (32 lanes: 4 keys x 4
// chunks) 16 distinct 16-byte slots of one -- both free of bank conflicts
// (with [key][64 bytes] rows the 64-byte stride of the writes cost 8 conflict
// cycles per instruction).  ds_read_b64_tr_b16 over that tile yields the B
// operand of dQ^T = K^T dS^T with lane l = position p directly, so perm only
// matters when dQ rows are stored.
//
// Work decomposition: one workgroup of NW (4 or 8) waves per (32 NW ST query
// rows, head, batch[, key split]); wave w owns the ST (1 or 2) query steps
// NW ST qb + ST w, ... (32 ST rows) and walks the key steps of 32.  Written dQ (deterministic mode,
// and atomic mode when the row blocks give every CU a workgroup): one
// workgroup covers every key step and stores dQ.  Atomic (use_atomic_backward
// on smaller grids): the key steps are cut into dq_split contiguous ranges
// and each workgroup adds its fp32 partial dQ into the zeroed accumulator
// with fp32 atomics, one coalesced row segment per instruction (the reference
// adds a partial per 64-key block, python/fa2.py:295-297, which on this part
// is bound by atomic throughput).  Per step the workgroup stages one K tile
// (shared, XOR-swizzled for the transpose reads) and each wave its two dS
// tile(s) (private) through registers into LDS, kSets steps ahead of use; the
// kernel is bound by the HBM reads of the dS tiles, so it keeps as many bytes
// in flight as registers allow at two waves per SIMD.
#include "fa_common.h"
#include "fa_kernels.h"
#include "fa_pipe.h"

namespace fa {
namespace {

using namespace pipe;

constexpr int kSets = 3;                              // register staging sets: tiles in flight
constexpr unsigned kCuCount = 256;                    // compute units of the part

// NW waves per workgroup, ST query steps (32 ST rows) each.  NW = 8, ST = 2
// (deterministic, head dim 128, no mask, enough rows to give every CU a
// workgroup) shares each step's K tile among 512 query rows, which halves its
// L2 reads (15 % faster at T 8192).  With a mask the row blocks are the
// prepared lists' 256 rows: NW = 8, ST = 1 (deterministic, head dim 128: twice
// the waves, and dS bytes in flight, of NW = 4, ST = 2).  Else NW = 4, ST = 2
// (with atomics 8 waves were 3-5 % slower).
// PREC (a mask or a score): each stored block is a pair of tiles, dS rounded
// and its rounding residual, and dQ adds both products (dS to about 16
// significant bits); two register staging sets then hold as many bytes as
// three of single tiles.
template <typename T, int D, bool CAUSAL, bool MASK, bool ATOMIC, int NW, int ST, bool PREC>
__global__ __launch_bounds__(NW * 64, 2) void dq_ds_kernel(const BwdArgs a) {
  constexpr int kDqWaves = NW;
  constexpr int kDqSteps = ST;                       // 32-row query steps per wave
  constexpr int kDqRows = kDqWaves * kDqSteps * 32;   // query rows per workgroup
  using V8 = typename Vec8<T>::type;
  constexpr int NPART = PREC ? 2 : 1;                // 2 KB tiles per stored block
  constexpr int kS = PREC && ST == 2 ? 2 : kSets;    // register staging sets
  constexpr int NB = D / 32, CH = D / 8, ROWB = 2 * D;
  constexpr int KTILE = 32 * ROWB;                   // bytes of one K step tile
  constexpr int DSW = kDqSteps * NPART * 2048;       // dS bytes of one wave and step
  constexpr int BUFB = KTILE + kDqWaves * DSW;       // one LDS buffer
  constexpr int UK = 32 * CH / (kDqWaves * 64);      // K chunks per thread
  constexpr int UD = DSW / (64 * 16);                // dS chunks per lane
  constexpr int OS = D + 8;                          // epilogue staging stride (elements)
  static_assert(UK >= 1 && UD >= 1, "tile split");
  static_assert(kDqRows == (NW == 8 && ST == 2 ? kDqDsRowsWide : kDqDsRows) && (!MASK || kDqRows == kDqDsRows),
                "row blocks as the host and the prepared-mask lists assume");
  constexpr int OSF = D + 4;                         // atomic epilogue: fp32 staging stride
  constexpr int SMEM0 = kDqWaves * 32 * OS * 2 > 2 * BUFB ? kDqWaves * 32 * OS * 2 : 2 * BUFB;   // + epilogue staging
  constexpr int SMEM = ATOMIC && kDqWaves * 32 * OSF * 4 > SMEM0 ? kDqWaves * 32 * OSF * 4 : SMEM0;
  __shared__ __attribute__((aligned(1024))) char smem[SMEM];

  // ---- which (batch, head, 256-row block) ----------------------------------------
  // Logical order: kv-head major (the heads of a group share K in L2), longest
  // blocks first: causal blocks from the last one, with a mask by the count of
  // live key steps.
  const int nqb = a.nqt;
  const int nsp = ATOMIC ? a.dq_split : 1;
  const int ng = a.ng;                   // heads of each group in this launch, from g0
  const int nblk = a.nbk * ng * nqb * nsp;
  const int W0 = xcd_remap(blockIdx.x, nblk);
  const int W = ATOMIC ? W0 / nsp : W0;
  const int ksp = ATOMIC ? W0 - W * nsp : 0;        // key split of this workgroup
  const int per_kv = ng * nqb;
  const int bkl = W / per_kv;             // unit within this launch's slice
  const int bk = a.bk0 + bkl;
  const int rem = W - bkl * per_kv;
  const int qb_rank = rem / ng;
  const int g = a.g0 + rem - qb_rank * ng;
  const int b = bk / a.Hk, kvh = bk - b * a.Hk;
  const int h = kvh * a.G + g;
  // (over a range of rows, block 0 of the launch is the range's first)
  const int qb0 = a.q32_lo / (kDqRows / 32);
  const int qb = MASK ? mask_order(a.ml, a.mws, mask_plane(a.ml, b, h), 2)[qb_rank] : qb0 + nqb - 1 - qb_rank;

  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int l32 = lane & 31, hf = lane >> 5;
  const int wv = __builtin_amdgcn_readfirstlane(wave);
  const int Tq = a.Tq, Tk = a.Tk, nk32 = a.nk32, nq32 = a.nq32;
  const int s0 = qb * (kDqRows / 32) + wv * kDqSteps;          // this wave's first query step
  const int s_last = min(qb * (kDqRows / 32) + kDqRows / 32, nq32) - 1;
  // Key steps of the workgroup: 0 .. nstep-1, or with a mask the live steps of
  // the prepared list (causality folded in).  A dS tile is read only where the
  // dK/dV kernel stored it: its 32x32 block holds a kept entry.
  const int32_t* dql = nullptr;
  const uint8_t* blk = nullptr;
  if constexpr (MASK) {
    const int pm = mask_plane(a.ml, b, h);
    dql = (const int32_t*)(a.mws + a.ml.ldq + pm * a.ml.pldq) + (int64_t)qb * (1 + nk32);
    blk = (const uint8_t*)(a.mws + a.ml.blk + pm * a.ml.pblk);
  }
  const int nstep = MASK ? dql[0] : (CAUSAL ? min(s_last + 1, nk32) : nk32);
  // positions [jb, jb + nloc) of that sequence are this workgroup's
  const int chunk = (nstep + nsp - 1) / nsp;
  const int jb = min(nstep, ksp * chunk);
  const int nloc = min(nstep, jb + chunk) - jb;
  // With a mask, 128 positions jl of this workgroup's range at a time sit in
  // two registers (lane i of ents[w]: position ebase + 64 w + i), read with
  // readlane: the key step, and in bits 30 and 31 whether the dK/dV kernel
  // stored the tile of this wave's query step 0 and 1 (step below Tq, on or
  // below the causal diagonal, block holding a kept entry).  The window moves
  // every 128 steps.  (Per-step scalar loads of the list and block states
  // cost a quarter of the kernel's time at the packed-document config, and
  // made each step wait for all of the wave's loads.)
  int32_t ents[MASK ? 2 : 1] = {};
  int ebase = -128;
  auto fill_ents = [&](int base) __attribute__((always_inline)) {
#pragma unroll
    for (int w = 0; w < 2; ++w) {
      const int jl = base + 64 * w + lane;
      int32_t e = 0;
      if (jl < nloc) {
        const int kb = dql[1 + jb + jl];
        e = kb;
#pragma unroll
        for (int i = 0; i < kDqSteps; ++i) {
          const int s = s0 + i;
          const bool ok = s < nq32 && (!CAUSAL || kb <= s) && blk[(int64_t)s * nk32 + kb] != 0;
          e |= ok ? (int32_t)(1u << (30 + i)) : 0;
        }
      }
      ents[w] = e;
    }
    // consumed here, inside the branch that moves the window: loads still
    // pending where it rejoins would make every step wait for all loads
    asm volatile("" : "+v"(ents[0]), "+v"(ents[1]));
    ebase = base;
  };
  if constexpr (MASK) fill_ents(0);

  // ---- LDS addresses ---------------------------------------------------------------
  const uint32_t lds0 = (uint32_t)(uintptr_t)(FA_LDS char*)smem;
  const int rr = (lane >> 2) & 3;
  const int tr_col = ((lane >> 4) & 1) * 16 + (lane & 3) * 4;
  // A = K^T (transpose reads of the swizzled K tile), rows 4 hf + rr (+8), key chunk c adds 16 rows
  uint32_t at[2][NB];
#pragma unroll
  for (int hi = 0; hi < 2; ++hi)
#pragma unroll
    for (int nb = 0; nb < NB; ++nb) {
      const int row = 4 * hf + rr + 8 * hi, col = nb * 32 + tr_col;
      at[hi][nb] = opaque(lds0 + row * ROWB + (((col >> 3) ^ swz_q<D>(row)) * 16) + (col & 7) * 2);
    }
  // B = dS^T (transpose reads of the wave's chunk-major tiles): key rows
  // 4 hf + rr + 8 hi (+16 for the second half, +256 bytes), positions tr_col..+3
  // in chunk tr_col / 8
  uint32_t bd[2];
#pragma unroll
  for (int hi = 0; hi < 2; ++hi) {
    const int key = 4 * hf + rr + 8 * hi, ch = tr_col >> 3;
    bd[hi] = opaque(lds0 + KTILE + wv * DSW + ch * 512 + ((key ^ (4 * ch)) & 31) * 16 + (tr_col & 7) * 2);
  }

  // ---- staging -----------------------------------------------------------------------
  const T* __restrict__ kbase = (const T*)a.k + b * a.ksb + kvh * a.ksh;
  uint32_t gk[UK], swk[UK];
#pragma unroll
  for (int u = 0; u < UK; ++u) {
    const int idx = tid + u * kDqWaves * 64, r = idx / CH, c = idx % CH;
    gk[u] = (uint32_t)(r * a.kst * 2 + c * 16);
    swk[u] = opaque(lds0 + r * ROWB + ((c ^ swz_q<D>(r)) * 16));
  }
  // staging chunk u' (bytes lane 16 + u' 1024 of a tile) = chunk lane/32 + 2 u' of key lane%32
  const int skey = lane & 31;
  uint32_t sd[2];
#pragma unroll
  for (int u = 0; u < 2; ++u) {
    const int ch = (lane >> 5) + 2 * u;
    sd[u] = opaque(lds0 + KTILE + wv * DSW + ch * 512 + ((skey ^ (4 * ch)) & 31) * 16);
  }
  const uint16_t* __restrict__ dsp = (const uint16_t*)a.ds;
  const int64_t plane = ((int64_t)b * a.Hq + h - a.ds_p0) * a.ds_plane - ds_row(a.q32_lo, nk32, CAUSAL);
  int64_t row0[kDqSteps];
#pragma unroll
  for (int i = 0; i < kDqSteps; ++i) row0[i] = plane + ds_row(s0 + i, nk32, CAUSAL);

  u32x4 stk[kS][UK], std_[kS][UD];
  // Key step at local position jl (position jb + jl) into staging set S (keys
  // past Tk and dS tiles outside the stored set load as zeros; jl >= nloc
  // loads nothing).
  auto load = [&](int S, int jl) __attribute__((always_inline)) {
    const bool inr = jl < nloc;
    const int j = jb + jl;
    int kb = j;
    uint32_t okb = 0;   // with a mask, bit i: the tile of query step s0 + i is stored
    if constexpr (MASK) {
      kb = 0;
      if (inr) {
        if ((jl & ~127) != ebase) fill_ents(jl & ~127);
        const int r = jl - ebase;
        const int32_t lo = __builtin_amdgcn_readlane(ents[0], r & 63);
        const int32_t hi = __builtin_amdgcn_readlane(ents[1], r & 63);
        const int32_t e = r < 64 ? lo : hi;
        kb = e & 0x3fffffff;
        okb = (uint32_t)e >> 30;
      }
    }
    const int rows = inr ? min(32, Tk - kb * 32) : 0;
    const int nrec = rows > 0 ? (int)((int64_t)(rows - 1) * a.kst * 2 + ROWB) : 0;
    const auto rk = __builtin_amdgcn_make_buffer_rsrc((void*)(kbase + (int64_t)kb * 32 * a.kst), (short)0, nrec, 0x00020000);
#pragma unroll
    for (int u = 0; u < UK; ++u) stk[S][u] = __builtin_amdgcn_raw_buffer_load_b128(rk, gk[u], 0, 0);
#pragma unroll
    for (int i = 0; i < kDqSteps; ++i) {
      const int s = s0 + i;
      const bool ok = MASK ? ((okb >> i) & 1u) != 0 : inr && s < nq32 && (!CAUSAL || kb <= s);
      const auto rd = __builtin_amdgcn_make_buffer_rsrc((void*)(dsp + (row0[i] + kb) * 1024 * NPART), (short)0,
                                                        ok ? 2048 * NPART : 0, 0x00020000);
#pragma unroll
      for (int u = 0; u < UD / kDqSteps; ++u)   // non-temporal: each dS tile is read once
        std_[S][i * (UD / kDqSteps) + u] = __builtin_amdgcn_raw_buffer_load_b128(rd, (uint32_t)(lane * 16 + u * 1024), 0, 2);
    }
  };
  auto store = [&](int S, int BUF) __attribute__((always_inline)) {
#pragma unroll
    for (int u = 0; u < UK; ++u) lds_wr16(swk[u] + BUF * BUFB, stk[S][u]);
#pragma unroll
    for (int u = 0; u < UD; ++u) lds_wr16(sd[u & 1] + BUF * BUFB + (u >> 1) * 2048, std_[S][u]);
  };

  // ---- accumulators: dQ^T [32 nb + 8 (e/4) + 4 hf + e%4][position l32] per query step ----
  f32x16 acc[kDqSteps][NB];
#pragma unroll
  for (int i = 0; i < kDqSteps; ++i)
#pragma unroll
    for (int nb = 0; nb < NB; ++nb) acc[i][nb] = f32x16{};

  auto compute = [&](int BUF) __attribute__((always_inline)) {
#pragma unroll
    for (int c = 0; c < 2; ++c) {
      V8 bf[kDqSteps * NPART];   // tile (step i, part) at (i NPART + part) 2048
#pragma unroll
      for (int i = 0; i < kDqSteps * NPART; ++i) {
        const uint32_t off = (uint32_t)(BUF * BUFB + i * 2048 + c * 256);   // keys 16 c ..
        bf[i] = cat_tr<T>(lds_rdtr(bd[0] + off), lds_rdtr(bd[1] + off));
      }
#pragma unroll
      for (int nb = 0; nb < NB; ++nb) {
        const uint32_t off = (uint32_t)(BUF * BUFB + c * 16 * ROWB);
        const V8 af = cat_tr<T>(lds_rdtr(at[0][nb] + off), lds_rdtr(at[1][nb] + off));
#pragma unroll
        for (int i = 0; i < kDqSteps; ++i) {
          acc[i][nb] = mfma32(af, bf[i * NPART], acc[i][nb]);
          if constexpr (PREC) acc[i][nb] = mfma32(af, bf[i * NPART + 1], acc[i][nb]);
        }
      }
    }
  };

  // ---- prologue: tiles 0 .. kSets-1 loading (tile t in set t % kSets), tile 0 in buffer 0 --
#pragma unroll
  for (int t = 0; t < kS; ++t) load(t, t);
  store(0, 0);
  load(0, kS);
  lds_barrier();

  // ---- main loop: iteration j writes tile j+1 to LDS buffer (j+1)%2, loads tile
  // j+1+kS into the set it freed, computes tile j from buffer j%2 ---------------------
  constexpr int U = kS == 2 ? 2 : 6;   // lcm(kS, 2): sets and buffers static per copy
  int nu = (nloc + U - 1) / U * U;
  asm volatile("" : "+s"(nu));
  for (int j = 0; j < nu; j += U) {
#pragma unroll
    for (int u = 0; u < U; ++u) {
      store((u + 1) % kS, (u + 1) & 1);
      load((u + 1) % kS, j + u + 1 + kS);
      compute(u & 1);
      lds_barrier();
    }
  }

  // ---- epilogue: dQ rows of each query step through LDS, coalesced stores --------------
  const float scale = a.scale;
  const int qrow_l = 16 * (l32 >> 4) + 4 * ((l32 >> 3) & 1) + 8 * ((l32 >> 2) & 1) + (l32 & 3);
  if constexpr (ATOMIC) {
    if (nloc == 0) return;   // no key step: nothing to add
    // fp32 partial rows [32][D] per step, then 64 consecutive floats per atomic instruction
    float* stf = (float*)smem + wv * 32 * OSF;
    float* dqa = a.dq_accum + ((int64_t)b * a.Hq + h) * Tq * D;
#pragma unroll
    for (int i = 0; i < kDqSteps; ++i) {
#pragma unroll
      for (int nb = 0; nb < NB; ++nb)
#pragma unroll
        for (int gi = 0; gi < 4; ++gi) {
          f32x4 v;
#pragma unroll
          for (int t = 0; t < 4; ++t) v[t] = acc[i][nb][gi * 4 + t] * scale;
          *(FA_LDS f32x4*)(uintptr_t)(stf + qrow_l * OSF + nb * 32 + gi * 8 + hf * 4) = v;
        }
      asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
      const int q0 = (s0 + i) * 32;
#pragma unroll 4
      for (int u = 0; u < 32 * D / 64; ++u) {
        const int idx = lane + u * 64, r = idx / D, c = idx % D;
        const float v = *(const FA_LDS float*)(uintptr_t)(stf + r * OSF + c);
        if (q0 + r < Tq) unsafeAtomicAdd(dqa + (int64_t)(q0 + r) * D + c, v);
      }
      asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
    }
    return;
  }
  T* stg = (T*)smem + wv * 32 * OS;
  T* dqp = (T*)a.dq + b * a.dqsb + h * a.dqsh;
  const int qrow = qrow_l;
#pragma unroll
  for (int i = 0; i < kDqSteps; ++i) {
#pragma unroll
    for (int nb = 0; nb < NB; ++nb)
#pragma unroll
      for (int gi = 0; gi < 4; ++gi) {
        const int d = nb * 32 + gi * 8 + hf * 4;
        lds_write8(stg + qrow * OS + d, pack4<T>(acc[i][nb][gi * 4 + 0] * scale, acc[i][nb][gi * 4 + 1] * scale,
                                                 acc[i][nb][gi * 4 + 2] * scale, acc[i][nb][gi * 4 + 3] * scale));
      }
    asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
    const int q0 = (s0 + i) * 32;
    // all staging reads first (one wait), then the row-guarded stores
    constexpr int NU = 32 * CH / 64;
    u32x4 ov[NU];
#pragma unroll
    for (int u = 0; u < NU; ++u) {
      const int idx = lane + u * 64;
      ov[u] = lds_read16(stg + (idx / CH) * OS + (idx % CH) * 8);
    }
#pragma unroll
    for (int u = 0; u < NU; ++u) {
      const int idx = lane + u * 64, r = idx / CH, c = idx % CH;
      if (q0 + r < Tq) gstore16(dqp + (int64_t)(q0 + r) * a.dqst + c * 8, ov[u]);
    }
    asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
  }
}

template <typename T, int D, bool CAUSAL, bool ATOMIC, bool PREC>
hipError_t launch_p(const BwdArgs& a, hipStream_t s) {
  const dim3 grid((unsigned)(a.nbk * a.ng * a.nqt * (ATOMIC ? a.dq_split : 1)));
  if (PREC && a.mask) {
    // With a mask the row blocks stay at 256 rows (the prepared lists are per
    // 256-row block).  At head dim 128: 8 waves of one 32-row step each (with
    // the tile pairs, the 4-wave shape of two steps per wave needs more
    // registers than two waves per SIMD hold); at 64: 4 waves of two steps.
    if constexpr (PREC) {
      if constexpr (D == 128) hipLaunchKernelGGL((dq_ds_kernel<T, D, CAUSAL, true, ATOMIC, 8, 1, PREC>), grid, dim3(512), 0, s, a);
      else hipLaunchKernelGGL((dq_ds_kernel<T, D, CAUSAL, true, ATOMIC, 4, 2, PREC>), grid, dim3(256), 0, s, a);
    }
  } else if constexpr (D == 128 && !ATOMIC && !PREC) {
    if (a.dq_rows == kDqDsRowsWide) hipLaunchKernelGGL((dq_ds_kernel<T, D, CAUSAL, false, ATOMIC, 8, 2, PREC>), grid, dim3(512), 0, s, a);
    else hipLaunchKernelGGL((dq_ds_kernel<T, D, CAUSAL, false, ATOMIC, 4, 2, PREC>), grid, dim3(256), 0, s, a);
  } else {
    hipLaunchKernelGGL((dq_ds_kernel<T, D, CAUSAL, false, ATOMIC, 4, 2, PREC>), grid, dim3(256), 0, s, a);
  }
  return hipGetLastError();
}

// A mask (PREC with the prepared lists) always has PREC; a score without a
// mask runs the unmasked kernel with PREC.
template <typename T, int D, bool CAUSAL, bool ATOMIC>
hipError_t launch_a(const BwdArgs& a, hipStream_t s) {
  if (a.mask || a.score) return launch_p<T, D, CAUSAL, ATOMIC, true>(a, s);
  return launch_p<T, D, CAUSAL, ATOMIC, false>(a, s);
}

template <typename T, int D, bool CAUSAL>
hipError_t launch_t(const BwdArgs& a, hipStream_t s) {
  return a.do_dq ? launch_a<T, D, CAUSAL, true>(a, s) : launch_a<T, D, CAUSAL, false>(a, s);
}

}  // namespace


hipError_t launch_bwd_dq_ds(const BwdArgs& a, int D, int dtype, bool causal, hipStream_t s) {
  if (dtype == 0) {
    if (D == 128) return causal ? launch_t<bf16, 128, true>(a, s) : launch_t<bf16, 128, false>(a, s);
    if (D == 64) return causal ? launch_t<bf16, 64, true>(a, s) : launch_t<bf16, 64, false>(a, s);
  } else {
    if (D == 128) return causal ? launch_t<f16, 128, true>(a, s) : launch_t<f16, 128, false>(a, s);
    if (D == 64) return causal ? launch_t<f16, 64, true>(a, s) : launch_t<f16, 64, false>(a, s);
  }
  return hipErrorInvalidValue;
}

}  // namespace fa
