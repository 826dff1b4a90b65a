// dK/dV of the FlashAttention-2 backward for gfx950 (MI355X), deterministic
// path (dQ comes from the separate dQ kernel).  Restates the dK/dV part of the
// reference's TileLang backward (python/fa2.py:181-302, 305-426): per key
// block, over every query row of every query head of the GQA group,
//   S  = Q K^T, dP = dO V^T            P  = exp2(S scale log2e - LSE2)
//   dS = P (dP - Delta) scale          dV += P^T dO,  dK += dS^T Q
// (dP - Delta comes out of the MFMA chain started from -Delta, and the factor
// scale is applied once to dK at the end.)
// with dK/dV of the whole group accumulated in registers.
//
// Work decomposition: one workgroup of 4 waves (one per SIMD, 512 registers
// each) per (128 keys, kv-head, batch[, head-group split]); wave w owns keys
// 32 w .. 32 w + 31 and walks the query rows in steps of 32.  Per step:
//   S, dP     32x32x16 MFMA, A = Q / dO rows (ds_read_b128 from LDS),
//             B = K / V fragments resident in registers
//   P, dS     fp32 VALU on the accumulators, packed to 16 bits in place
//   dV^T, dK^T += dO^T P, Q^T dS   A = dO^T / Q^T (ds_read_b64_tr_b16),
//             B = P / dS straight from the accumulator registers
// The step loop is software-pipelined inside each wave: iteration j issues
// the MFMAs of S/dP(j+1) and of dV/dK(j-1) interleaved with the VALU work of
// P/dS(j), which depends on neither, so one wave keeps its SIMD's MFMA and
// VALU pipes busy at the same time.
//
// Q/dO step tiles (32 rows) live in 4 LDS buffers (tiles j-1 and j+1 are read
// in iteration j while j+2 is written; 6 buffers and tile j+3 in the plain
// head-dim-128 instance), rows unpadded with one XOR swizzle of
// their 16-byte chunks that keeps both the ds_read_b128 pattern (16 rows) and
// the transpose-read pattern (4 rows x 4 chunks) conflict-free.  Tiles are
// staged through registers: loaded with buffer loads (loop-invariant lane
// offsets, tile base in scalar registers, rows past Tq zero-filled) and
// written into LDS one iteration later, both at the start of an iteration.  LSE and -Delta of the
// tile's rows travel with it (LSE = +inf past Tq, so P = 0 there).
#include "fa_common.h"
#include "fa_kernels.h"
#include "fa_pipe.h"

namespace fa {
namespace {

using namespace pipe;

constexpr int kKvWaves = 4;
constexpr int kKvKeys = kKvWaves * 32;   // keys per workgroup
constexpr int kStep = 32;                // query rows per step
constexpr int kNBuf = 4;                 // LDS buffers of step tiles

template <typename T, int D, bool CAUSAL, bool MASK, bool SCORE>
__global__ __launch_bounds__(kKvWaves * 64, 1) __attribute__((amdgpu_waves_per_eu(1, 1))) void dkdv2_kernel(const BwdArgs a) {
  using V8 = typename Vec8<T>::type;
  constexpr int DS = D / 16, NB = D / 32, CH = D / 8, ROWB = 2 * D;
  constexpr int QTILE = kStep * ROWB;            // bytes of one Q (or dO) step tile
  // Six buffers in the plain head-dim-128 instance (the registers for a second
  // set of LDS base addresses are there since the K/V fragments live in
  // AGPRs): tile j+3 is written in iteration j and first read in iteration
  // j+2, and each buffer's previous tile was last read in iteration j-2, so a
  // workgroup barrier after every second iteration suffices.  Otherwise four
  // buffers, tile j+2 written in iteration j, a barrier after every iteration.
  constexpr bool SIX = !MASK && !SCORE && D == 128;
  constexpr int NBUF = SIX ? 6 : kNBuf;
  constexpr int AHD = SIX ? 3 : 2;               // tiles written ahead of the step computed
  // Buffer b: Q tile at b QST, dO tile at b QST + DOFF.  Six buffers
  // interleave Q and dO; offsets of 64 KB and more go through a second set of
  // base registers (the DS immediate offset has 16 bits).
  constexpr int QST = SIX ? 2 * QTILE : QTILE;
  constexpr int DOFF = SIX ? QTILE : kNBuf * QTILE;
  constexpr int LOFF = 2 * NBUF * QTILE;         // [buf][LSE | -Delta][32] fp32
  constexpr int LBUF = 2 * kStep * 4;
  constexpr int UQ = kStep * CH / (kKvWaves * 64);  // chunks per thread per tile
  constexpr int OS = D + 8;                      // epilogue staging stride (elements)
  static_assert(UQ >= 1, "tile split");
  static_assert(SIX || DOFF + kNBuf * QTILE <= 65536, "buffer offsets fit the DS immediate");
  static_assert(!SIX || (NBUF - 1) * QST + DOFF + QTILE - 65536 <= 65536, "high buffers fit the second base");
  static_assert(kKvWaves * 32 * OS * 2 <= 2 * NBUF * QTILE, "epilogue staging fits");
  static_assert(kKvKeys == kKv2Keys && kStep == 32, "prepared-mask lists are built for this shape");
  // With a mask or a score, P and dS enter dV += P^T dO and dK += dS^T Q in
  // several 16-bit parts each (the rounded value and its rounding residuals:
  // more MFMAs on the same LDS operand): dS in two, P in three, which carries
  // P to fp32 precision -- dV sums the few large P of rows that see few keys
  // into entries whose 16-bit output step is coarse, and two parts left
  // about one in a thousand of those entries a step off.  Each dS tile is
  // followed by the tile of its residuals for the dQ kernel.
  constexpr bool PREC = MASK || SCORE;
  constexpr int NPART = PREC ? 2 : 1;   // 2 KB tiles per stored 32x32 block
  __shared__ __attribute__((aligned(1024))) char smem[LOFF + NBUF * LBUF];

  // ---- which (batch, kv-head, split, key block) ------------------------------
  const int nblk = a.nbk * a.nkt * a.nsp;
  const int W = xcd_remap(blockIdx.x, nblk);
  const int per_bk = a.nsp * a.nkt;
  const int bkl = W / per_bk;             // unit within this launch's slice
  const int bk = a.bk0 + bkl;
  const int rem = W - bkl * per_bk;
  const int spl = rem / a.nkt;            // part within this launch's parts
  const int sp = a.sp0 + spl;
  const int b = bk / a.Hk, kvh = bk - b * a.Hk;
  // longest workgroups first: key blocks ascending (causal work shrinks with
  // the block), with a mask by the count of live steps of the group's first head
  const int kt_rank = rem - spl * a.nkt;
  const int kt = MASK ? mask_order(a.ml, a.mws, mask_plane(a.ml, b, kvh * a.G + sp * (a.G / a.split)), 1)[kt_rank]
                      : kt_rank;

  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int l32 = lane & 31, hf = lane >> 5;
  const int Tq = a.Tq, Tk = a.Tk;
  const int wv = __builtin_amdgcn_readfirstlane(wave);   // wave-uniform copy for scalar branches
  const int kt0 = kt * kKvKeys, kw0 = kt0 + wv * 32;
  const int key = kw0 + l32;              // this lane's key (column of S)
  const int kc = min(key, Tk - 1);
  // scale == 0: every kept logit is 0, i.e. P = exp2(-LSE2): a zero multiplier
  const float c2 = a.zero_scale ? 0.f : a.scale_log2, scale = a.scale;

  const T* __restrict__ kp = (const T*)a.k + b * a.ksb + kvh * a.ksh;
  const T* __restrict__ vp = (const T*)a.v + b * a.vsb + kvh * a.vsh;

  // K, V fragments (B operands of S = Q K^T, dP = dO V^T): lane holds
  // K[key][16 ds + 8 hf .. +7].  Keys past Tk read row Tk-1: their dK/dV
  // rows are never stored and nothing else depends on them.
  V8 kf[DS], vf[DS];
#pragma unroll
  for (int ds = 0; ds < DS; ++ds) {
    kf[ds] = as_vec8<T>(gload16(kp + (int64_t)kc * a.kst + ds * 16 + hf * 8));
    vf[ds] = as_vec8<T>(gload16(vp + (int64_t)kc * a.vst + ds * 16 + hf * 8));
  }
  // The fragments stay in AGPRs for the whole loop (MFMA reads its A and B
  // operands from AGPRs as well): 64 VGPRs freed, which the masked and score
  // instances otherwise spill into AGPRs with a copy back per use (their
  // P / dS residual parts fill the VGPRs).
#pragma unroll
  for (int ds = 0; ds < DS; ++ds) asm volatile("" : "+a"(kf[ds]), "+a"(vf[ds]));

  // ---- iteration space: (head of the group split, 32-row step) ---------------
  // Without a mask: every step from qstart on, for each head.  With a mask: per
  // head, the live steps of the prepared list of this key block (causality
  // folded in), ascending.
  const int gsz = a.G / a.split;
  const int g0 = sp * gsz;
  const int h_first = kvh * a.G + g0, h_end = h_first + gsz;
  // rows of this launch: [rlo, rhi) (a range of steps when the backward runs
  // in row ranges; the lists of a mask are never ranged)
  const int rlo = a.q32_lo * kStep, rhi = min(Tq, a.q32_hi * kStep);
  const int qstart = max(CAUSAL && !MASK ? (kt0 / kStep) * kStep : 0, rlo);   // rows above the block are masked
  const int nst = qstart < rhi ? (rhi - qstart + kStep - 1) / kStep : 0;
  // Causal without a mask walks each head's steps downwards, from the last
  // one (first row qfirst) to the one at the diagonal (qstart): the workgroups
  // of a (batch, kv-head) that run together then read the same Q/dO rows at
  // the same time (from L2), where upwards each would start at its own
  // diagonal.  Otherwise steps go upwards from qfirst = qstart.
  constexpr bool DESC = CAUSAL && !MASK;
  const int qfirst = DESC && nst > 0 ? qstart + kStep * (nst - 1) : qstart;
  auto kv_list = [&](int h) __attribute__((always_inline)) -> const int32_t* {
    const int pm = mask_plane(a.ml, b, h);
    return (const int32_t*)(a.mws + a.ml.lkv + pm * a.ml.plkv) + (int64_t)kt * (1 + a.ml.nq32);
  };
  int n = gsz * nst;
  if constexpr (MASK) {
    n = 0;
    if (a.ml.Hm == 1) n = gsz * kv_list(h_first)[0];
    else for (int h = h_first; h < h_end; ++h) n += kv_list(h)[0];
  }
  // Step lists (MASK) are read through a window of 128 positions of one
  // head's list held in two registers (lane i of lreg_v[w]: position
  // win_base + 64 w + i), read with readlane.  The window moves (two vector
  // loads and one wait) when the load cursor leaves it: once per 128 steps
  // and per head, not at a head switch when the heads share one list (a mask
  // broadcast over them).  A scalar load per step instead cost a wait for
  // all of the wave's loads each step.
  const bool shared_list = MASK && a.ml.Hm == 1;
  int32_t lreg_v[2] = {};   // unused without a mask
  int win_h = -1, win_base = -128;
  auto win_load = [&](int h, int base) __attribute__((always_inline)) {
    const int32_t* l = kv_list(h);
    const int cnt = l[0];
#pragma unroll
    for (int w = 0; w < 2; ++w) {
      const int pos = base + 64 * w + lane;
      lreg_v[w] = pos < cnt ? l[1 + pos] : 0;
    }
    // consumed here, inside the (rarely taken) branch: otherwise the loads
    // are still pending where the branch rejoins, and every step waits there
    // for all of the wave's loads before reading the window
    asm volatile("" : "+v"(lreg_v[0]), "+v"(lreg_v[1]));
    win_h = h;
    win_base = base;
  };
  // List cursor (MASK): head h, position idx in that head's list of cnt
  // steps; seek() moves past exhausted and empty lists.  list_at(c): the
  // query step at the cursor (c.h < h_end).
  struct Cursor { int h, idx, cnt; const int32_t* lst; };
  auto seek = [&](Cursor& c) __attribute__((always_inline)) {
    while (c.idx >= c.cnt && c.h < h_end) {
      ++c.h;
      c.idx = 0;
      if (c.h < h_end) { c.lst = kv_list(c.h); c.cnt = c.lst[0]; }
    }
  };
  auto list_at = [&](const Cursor& c) __attribute__((always_inline)) -> int {
    const int base = c.idx & ~127;
    if (base != win_base || (c.h != win_h && !shared_list)) win_load(c.h, base);
    const int r = c.idx - win_base;
    const int lo = __builtin_amdgcn_readlane(lreg_v[0], r & 63);
    const int hi = __builtin_amdgcn_readlane(lreg_v[1], r & 63);
    return r < 64 ? lo : hi;
  };
  auto cursor0 = [&]() __attribute__((always_inline)) -> Cursor {
    Cursor c{h_first, 0, 0, nullptr};
    if constexpr (MASK) {
      c.lst = kv_list(h_first);
      c.cnt = c.lst[0];
      seek(c);
    }
    return c;
  };

  // ---- LDS addresses -----------------------------------------------------------
  const uint32_t lds0 = (uint32_t)(uintptr_t)(FA_LDS char*)smem;
  // ds_read_b128 (A of S / dP): row l32, logical chunk 2 ds + hf.  dO: + DOFF.
  uint32_t ab[DS];
#pragma unroll
  for (int ds = 0; ds < DS; ++ds) ab[ds] = opaque(lds0 + l32 * ROWB + (((2 * ds + hf) ^ swz_q<D>(l32)) * 16));
  // transpose reads (A of dV^T / dK^T): rows 16 c + 4 hf + rr (+8 for hi),
  // columns 32 nb + tr_col; the swizzle of those rows does not depend on c.
  const int rr = (lane >> 2) & 3;
  const int tr_col = ((lane >> 4) & 1) * 16 + (lane & 3) * 4;
  uint32_t at[2][NB];
#pragma unroll
  for (int hi = 0; hi < 2; ++hi)
#pragma unroll
    for (int nb = 0; nb < NB; ++nb) {
      const int row = 4 * hf + rr + 8 * hi, col = nb * 32 + tr_col;
      at[hi][nb] = opaque(lds0 + row * ROWB + (((col >> 3) ^ swz_q<D>(row)) * 16) + (col & 7) * 2);
    }
  // LSE / -Delta of rows 8 gi + 4 hf .. +3
  const uint32_t al = opaque(lds0 + LOFF + hf * 16);
  // second bases, 64 KB up (six buffers): a static offset off >= 64 KB is
  // reached as base2 + (off - 64 KB), keeping it in the DS immediate
  constexpr uint32_t kHi = 65536;
  uint32_t ab2[SIX ? DS : 1], at2[2][SIX ? NB : 1];
  if constexpr (SIX) {
#pragma unroll
    for (int ds = 0; ds < DS; ++ds) ab2[ds] = opaque(ab[ds] + kHi);
#pragma unroll
    for (int hi = 0; hi < 2; ++hi)
#pragma unroll
      for (int nb = 0; nb < NB; ++nb) at2[hi][nb] = opaque(at[hi][nb] + kHi);
  }
  auto lds_at = [](uint32_t lo, uint32_t hi, uint32_t off) __attribute__((always_inline)) -> uint32_t {
    return off >= kHi ? hi + (off - kHi) : lo + off;
  };

  // ---- tile staging ------------------------------------------------------------
  // chunk u of thread t: tile row r = idx / CH, logical chunk c = idx % CH
  // (idx = t + 256 u): coalesced rows in, swizzled position out.
  uint32_t gq[UQ], gd[UQ], sw[UQ], sw2[SIX ? UQ : 1];
#pragma unroll
  for (int u = 0; u < UQ; ++u) {
    const int idx = tid + u * kKvWaves * 64, r = idx / CH, c = idx % CH;
    gq[u] = (uint32_t)(r * a.qst * 2 + c * 16);
    gd[u] = (uint32_t)(r * a.dst * 2 + c * 16);
    sw[u] = opaque(lds0 + r * ROWB + ((c ^ swz_q<D>(r)) * 16));
    if constexpr (SIX) sw2[u] = opaque(sw[u] + kHi);
  }
  // two staging sets (tiles j+3, j+4 in flight during iteration j): [set]
  u32x4 stq[2][UQ], std_[2][UQ];
  float stl[2] = {0.f, 0.f}, std_l[2] = {0.f, 0.f};  // staged LSE / Delta of row l32 (wave 0)
  int st_rows[2] = {0, 0};                             // valid rows of the staged tile
  // Loads address a head through one descriptor whose records end after row
  // Tq - 1; a tile's first row is reached with the scalar offset, which the
  // range check includes, so rows past Tq read as zeros.  Padding steps use
  // descriptors without records.  State: next tile ld_it (head ld_h, first
  // row ld_qs), scalar byte offsets of that row in Q, dO and LSE/Delta.
  const uint32_t q_rec = (uint32_t)((int64_t)(Tq - 1) * a.qst * 2 + ROWB);
  const uint32_t d_rec = (uint32_t)((int64_t)(Tq - 1) * a.dst * 2 + ROWB);
  const uint32_t inc_q = (uint32_t)(kStep * a.qst * 2), inc_d = (uint32_t)(kStep * a.dst * 2);
  const uint32_t so_q0 = (uint32_t)qfirst * (uint32_t)a.qst * 2, so_d0 = (uint32_t)qfirst * (uint32_t)a.dst * 2;
  int ld_it = 0, ld_h = kvh * a.G + g0, ld_qs = qfirst;
  uint32_t so_q = so_q0, so_d = so_d0, so_l = (uint32_t)qfirst * 4;
  Cursor ldc = cursor0();
  const T* q_head = (const T*)a.q + b * a.qsb + (int64_t)ld_h * a.qsh;
  const T* d_head = (const T*)a.dout + b * a.dsb + (int64_t)ld_h * a.dsh;
  const float* l_head = a.lse + ((int64_t)b * a.Hq + ld_h) * Tq;
  const float* e_head = a.delta + ((int64_t)b * a.Hq + ld_h) * Tq;
  // Without a mask the descriptors change only at a head switch (the rows
  // advance through the scalar offsets), so they are kept across steps and
  // rebuilt there, with no records once the heads are exhausted (padding
  // steps): the loads cost no scalar work per step.
  auto rs_of = [&](const void* base, uint32_t rec, bool lv) __attribute__((always_inline)) {
    return __builtin_amdgcn_make_buffer_rsrc((void*)base, (short)0, lv ? (int)rec : 0, 0x00020000);
  };
  const bool live0 = n > 0;
  auto rq_c = rs_of(q_head, q_rec, live0), rd_c = rs_of(d_head, d_rec, live0);
  auto rl_c = rs_of(l_head, (uint32_t)Tq * 4, live0), re_c = rs_of(e_head, (uint32_t)Tq * 4, live0);
  // Mask words of the steps in flight (MASK): the transposed-bits word of
  // step t at this lane's key as loaded, with the step's tile (four steps
  // ahead), into slot t % 4; shifted by 4 hf (bit 8 gi + t' = row
  // 8 gi + 4 hf + t' of the step) and zeroed past the last step when used.
  // Loaded unconditionally (padding steps read the head's first words) and
  // used only four steps later: a conditional load whose result is used at
  // once made the compiler wait for all of the wave's loads right there.
  uint32_t mq[MASK ? 4 : 1] = {};
  // ... and the step's position, ((head - h_first) << psh) | (first row / 32),
  // read by the dS-store / score position four steps later (one list cursor
  // only).  psh bits hold every step index; the host's B Hq Tq < 2^31 keeps
  // the head part below 2^27.
  int pq[MASK ? 4 : 1] = {};
  const int psh = 32 - __builtin_clz((uint32_t)max(a.nq32 - 1, 1));
  auto load_next = [&](auto Sc, auto Qc) __attribute__((always_inline)) {
    constexpr int S = decltype(Sc)::value;
    constexpr int Q = decltype(Qc)::value;
    const bool live = ld_it < n;
    if constexpr (MASK) {
      // position the loads at the cursor's step (rows past Tq read as zeros)
      const int h_new = min(ldc.h, h_end - 1);
      ld_qs = live ? kStep * list_at(ldc) : 0;
      so_q = (uint32_t)ld_qs * (uint32_t)a.qst * 2;
      so_d = (uint32_t)ld_qs * (uint32_t)a.dst * 2;
      so_l = (uint32_t)ld_qs * 4;
      if (h_new != ld_h) {   // head pointers change only with the head
        ld_h = h_new;
        q_head = (const T*)a.q + b * a.qsb + (int64_t)ld_h * a.qsh;
        d_head = (const T*)a.dout + b * a.dsb + (int64_t)ld_h * a.dsh;
        l_head = a.lse + ((int64_t)b * a.Hq + ld_h) * Tq;
        e_head = a.delta + ((int64_t)b * a.Hq + ld_h) * Tq;
      }
      const uint32_t* bt = (const uint32_t*)(a.mws + a.ml.bitsT + mask_plane(a.ml, b, ld_h) * a.ml.pbitsT);
      mq[Q] = bt[((int64_t)(kc >> 5) * a.ml.wq + (ld_qs >> 5)) * 32 + (kc & 31)];
      pq[Q] = ((ld_h - h_first) << psh) | (ld_qs >> 5);
    }
    const auto rq = MASK ? rs_of(q_head, q_rec, live) : rq_c;
    const auto rd = MASK ? rs_of(d_head, d_rec, live) : rd_c;
#pragma unroll
    for (int u = 0; u < UQ; ++u) {
      stq[S][u] = __builtin_amdgcn_raw_buffer_load_b128(rq, gq[u], so_q, 0);
      std_[S][u] = __builtin_amdgcn_raw_buffer_load_b128(rd, gd[u], so_d, 0);
    }
    if (wv == 0) {  // lanes 0-31: LSE rows, 32-63: Delta rows
      const auto rl = MASK ? rs_of(l_head, (uint32_t)Tq * 4, live) : rl_c;
      const auto re = MASK ? rs_of(e_head, (uint32_t)Tq * 4, live) : re_c;
      stl[S] = __builtin_bit_cast(float, __builtin_amdgcn_raw_buffer_load_b32(rl, (uint32_t)l32 * 4, so_l, 0));
      std_l[S] = __builtin_bit_cast(float, __builtin_amdgcn_raw_buffer_load_b32(re, (uint32_t)l32 * 4, so_l, 0));
    }
    st_rows[S] = live ? min(kStep, Tq - ld_qs) : 0;
    ++ld_it;
    if constexpr (MASK) {
      if (live) {
        ++ldc.idx;
        seek(ldc);
      }
      return;
    }
    if constexpr (DESC) {
      ld_qs -= kStep;
      so_q -= inc_q;
      so_d -= inc_d;
      so_l -= kStep * 4;
    } else {
      ld_qs += kStep;
      so_q += inc_q;
      so_d += inc_d;
      so_l += kStep * 4;
    }
    if (DESC ? ld_qs < qstart : ld_qs >= rhi) {
      ++ld_h;
      ld_qs = qfirst;
      so_q = so_q0;
      so_d = so_d0;
      so_l = (uint32_t)qfirst * 4;
      q_head += a.qsh;
      d_head += a.dsh;
      l_head += Tq;
      e_head += Tq;
      const bool lv = ld_h < h_end;
      rq_c = rs_of(q_head, q_rec, lv);
      rd_c = rs_of(d_head, d_rec, lv);
      rl_c = rs_of(l_head, (uint32_t)Tq * 4, lv);
      re_c = rs_of(e_head, (uint32_t)Tq * 4, lv);
    }
  };
  auto store_tile = [&](int buf, auto Sc) __attribute__((always_inline)) {
    constexpr int S = decltype(Sc)::value;
#pragma unroll
    for (int u = 0; u < UQ; ++u) {
      const uint32_t qo = (uint32_t)(buf * QST), dof = (uint32_t)(buf * QST + DOFF);
      if constexpr (SIX) {
        lds_wr16(lds_at(sw[u], sw2[u], qo), stq[S][u]);
        lds_wr16(lds_at(sw[u], sw2[u], dof), std_[S][u]);
      } else {
        lds_wr16(sw[u] + qo, stq[S][u]);
        lds_wr16(sw[u] + dof, std_[S][u]);
      }
    }
    if (wv == 0) {
      // rows past the tile's end: LSE = +inf (P = 0 whatever S is), -Delta = 0
      const bool ok = l32 < st_rows[S];
      const float v = hf == 0 ? (ok ? stl[S] : kPosInf) : (ok ? -std_l[S] : 0.f);
      lds_wrf(lds0 + LOFF + buf * LBUF + lane * 4, v);
    }
  };

  // ---- step being computed: head it_h, first row it_qs (advanced per step) -----------
  int it_h = kvh * a.G + g0, it_qs = qfirst;
  Cursor itc = cursor0();
  if constexpr (MASK) {
    it_h = min(itc.h, h_end - 1);
    it_qs = n > 0 ? kStep * list_at(itc) : 0;
  }

  // ---- score of a step (lane's 16 query rows at its key) -----------------------
  // One range-checked buffer per step from its first row (the host keeps 32
  // rows below 4 GiB): rows past Tq read 0 (their P is 0: LSE = +inf); the
  // lane's offset (row 4 hf, key kc) is loop-invariant and element (g, t),
  // row 8 g + 4 hf + t, adds 8 g + t rows as a scalar offset.  Iteration j
  // loads step j+1's elements one by one, each right after step j's has been
  // used, so they get an iteration to arrive.
  float sreg[SCORE ? 16 : 1];
  const uint32_t s_lane = SCORE ? (uint32_t)(((int64_t)4 * hf * a.ssq + kc) * 4) : 0u;
  const uint32_t s_row = (uint32_t)a.ssq * 4u;
  auto score_rs = [&](int h, int qs, bool live) __attribute__((always_inline)) {
    const uint32_t nrec = live ? (uint32_t)(((int64_t)min(Tq - qs, 32) - 1) * a.ssq * 4 + (int64_t)Tk * 4) : 0u;
    return __builtin_amdgcn_make_buffer_rsrc((void*)(a.score + b * a.ssb + (int64_t)h * a.ssh + (int64_t)qs * a.ssq),
                                             (short)0, (int)nrec, 0x00020000);
  };
  auto load_s = [&](const __amdgpu_buffer_rsrc_t& rs, int i) __attribute__((always_inline)) {
    sreg[i] = __builtin_bit_cast(float, __builtin_amdgcn_raw_buffer_load_b32(
                                            rs, s_lane, (uint32_t)(8 * (i >> 2) + (i & 3)) * s_row, 0));
  };

  // ---- dS tiles for the dQ kernel --------------------------------------------------
  // dS of each step (this wave's 32 keys x the step's 32 rows) is stored as
  // tile row "key" = 64 bytes, 16 bytes per lane and chunk c: the lane's
  // packed values of rows 16 c + 4 hf + {0..3, 8..11}.  Stores of step j-1
  // are issued in iteration j; a descriptor with no records drops them
  // (padding steps, tiles above the causal diagonal, keys past Tk, no dS).
  // it_ptr: tile of (it_h, step it_qs / 32) and this wave's keys (a running
  // pointer: no 64-bit multiply per step).
  const int kb32 = __builtin_amdgcn_readfirstlane(kw0) >> 5;
  const int64_t ds_u0 = a.ds_p0;                 // first dS plane (b Hq + h) of the workspace
  const int64_t ds_r0 = ds_row(a.q32_lo, a.nk32, CAUSAL);   // first tile of the launch's steps in a plane
  const bool ds_on = a.ds != nullptr && kb32 < a.nk32;
  // tile bytes are chunk-major (chunk c of key row k at c 512 + k 16): store t
  // writes chunks 2 t + hf, i.e. one contiguous kilobyte of whole lines
  const uint32_t ds_vo = (uint32_t)(hf * 512 + l32 * 16);
  const int64_t ds_h0 = ((int64_t)b * a.Hq + it_h - ds_u0) * a.ds_plane + ds_row(qfirst >> 5, a.nk32, CAUSAL) - ds_r0 + kb32;
  const uint16_t* it_ptr = (const uint16_t*)a.ds + ds_h0 * 1024 * NPART;
  auto ds_rs = __builtin_amdgcn_make_buffer_rsrc((void*)a.ds, (short)0, 0, 0x00020000);
  // descriptor of step j's tile, then advance (it_h, it_qs, it_tile) to step j+1
  auto next_step = [&](int j, uint32_t mreg, int pos_next) __attribute__((always_inline)) {
    const int s = it_qs >> 5;
    if constexpr (MASK) {
      // tiles of blocks without a kept entry are neither stored nor read: the
      // block holds one iff a lane's transposed mask word (of this step; the
      // lanes of half 0 hold the whole words of the 32 keys) is not 0 -- the
      // block state the dQ kernel reads, without a scalar load
      const bool any = __builtin_amdgcn_ballot_w64(mreg != 0u) != 0;
      const bool ok = ds_on && j < n && (!CAUSAL || kb32 <= s) && any;
      const int64_t tile = ((int64_t)b * a.Hq + it_h - ds_u0) * a.ds_plane + ds_row(s, a.nk32, CAUSAL) - ds_r0 + kb32;
      ds_rs = __builtin_amdgcn_make_buffer_rsrc((void*)((uint16_t*)a.ds + tile * 1024 * NPART), (short)0,
                                                ok ? 2048 * NPART : 0, 0x00020000);
      // step j+1 as the load cursor queued it (padding steps: row 0 of the
      // last head)
      it_h = h_first + (pos_next >> psh);
      it_qs = kStep * (pos_next & ((1 << psh) - 1));
      return;
    }
    const bool ok = ds_on && j < n && (!CAUSAL || kb32 <= s);
    ds_rs = __builtin_amdgcn_make_buffer_rsrc((void*)it_ptr, (short)0, ok ? 2048 * NPART : 0, 0x00020000);
    if constexpr (DESC) {
      it_qs -= kStep;
      it_ptr -= (int64_t)min(s, a.nk32) * 1024 * NPART;   // row s-1 holds min(s, nk32) tiles
    } else {
      it_qs += kStep;
      it_ptr += (int64_t)(CAUSAL ? min(s + 1, a.nk32) : a.nk32) * 1024 * NPART;
    }
    if (DESC ? it_qs < qstart : it_qs >= rhi) {
      ++it_h;
      it_qs = qfirst;
      it_ptr = (const uint16_t*)a.ds + (ds_h0 + (int64_t)(it_h - (kvh * a.G + g0)) * a.ds_plane) * 1024 * NPART;
    }
  };

  // ---- accumulators ---------------------------------------------------------------
  f32x16 dkt[NB], dvt[NB];   // dK^T / dV^T [32 nb + 8 (i/4) + 4 hf + i%4][key]
#pragma unroll
  for (int nb = 0; nb < NB; ++nb) { dkt[nb] = f32x16{}; dvt[nb] = f32x16{}; }
  f32x16 sacc[2], pacc[2];   // S / dP of steps j (parity) ; lane: [q = 8 (i/4) + 4 hf + i%4][key]
  V8 ppk[2][2], dspk[2][2];  // P / dS packed: [parity][c], k-slot (hf, t) <-> row 16 c + 4 hf + t%4 + 8 (t/4)
  V8 ppl[PREC ? 2 : 1][2], dsl[PREC ? 2 : 1][2];   // their rounding residuals (PREC)
  V8 ppl2[PREC ? 2 : 1][2];                        // P's second residual (PREC)
#pragma unroll
  for (int x = 0; x < 2; ++x) {
    sacc[x] = f32x16{}; pacc[x] = f32x16{};
#pragma unroll
    for (int c = 0; c < 2; ++c) { ppk[x][c] = V8{}; dspk[x][c] = V8{}; }
  }
#pragma unroll
  for (int x = 0; x < (PREC ? 2 : 1); ++x)
#pragma unroll
    for (int c = 0; c < 2; ++c) { ppl[x][c] = V8{}; dsl[x][c] = V8{}; ppl2[x][c] = V8{}; }

  // S/dP of step j+1 (tile in buffer BUF+1) and dV/dK of step j-1 (buffer
  // BUF-1) -- one interleaved MFMA stream, with the P/dS VALU work of step j
  // (buffer BUF) threaded through it.  EDGE: some (row, key) of the step is
  // masked (causal diagonal or a mask).
  auto iter = [&](auto BUFc, auto EDGEc, int j, uint32_t mreg, int pos_next) __attribute__((always_inline)) {
    // j: step whose P/dS is computed now; S/dP of j+1; dV/dK of j-1
    constexpr int BUF = decltype(BUFc)::value;          // buffer of step j
    constexpr bool EDGE = decltype(EDGEc)::value != 0;
    constexpr int BN1 = (BUF + 1) % NBUF, BM1 = (BUF + NBUF - 1) % NBUF;
    constexpr int PJ = BUF & 1, PN = PJ ^ 1;            // parities of j and j +- 1
    const int dkq = key - (it_qs + 4 * hf);              // causal: keep iff dkq <= 8 gi + t

    // score buffer of step j+1 (its position: queued with its tile with a
    // mask, else the next row step / head)
    int hn = 0, qn = 0;
    if constexpr (SCORE) {
      if constexpr (MASK) {
        hn = h_first + (pos_next >> psh);
        qn = kStep * (pos_next & ((1 << psh) - 1));
      } else {
        hn = it_h;
        qn = DESC ? it_qs - kStep : it_qs + kStep;
        if (DESC ? qn < qstart : qn >= rhi) { ++hn; qn = qfirst; }
      }
    }
    const auto srs_next = score_rs(min(hn, h_end - 1), qn, SCORE && j + 1 < n);
    // operand reads for the two MFMA streams, AHEAD ops ahead
    auto rd_sd = [&](int t) __attribute__((always_inline)) -> u32x4 {   // t: ds = t/2, Q (even) / dO (odd)
      const uint32_t off = (uint32_t)((t & 1) * DOFF + BN1 * QST);
      if constexpr (SIX) return lds_rd16(lds_at(ab[t >> 1], ab2[t >> 1], off));
      else return lds_rd16(ab[t >> 1] + off);
    };
    auto rd_tr = [&](int t) __attribute__((always_inline)) -> V8 {       // t: c = t / (2 NB), nb, dO (even) / Q (odd)
      const int c = t / (2 * NB), nb = (t / 2) % NB, isq = t & 1;
      const uint32_t off = (uint32_t)((isq ? 0 : DOFF) + BM1 * QST + 16 * c * ROWB);
      if constexpr (SIX)
        return cat_tr<T>(lds_rdtr(lds_at(at[0][nb], at2[0][nb], off)), lds_rdtr(lds_at(at[1][nb], at2[1][nb], off)));
      else return cat_tr<T>(lds_rdtr(at[0][nb] + off), lds_rdtr(at[1][nb] + off));
    };
    constexpr int NOP = 2 * DS;                          // == 4 * NB: ops per stream
    // -Delta of the rows of step j+1: initial accumulator of its dP chain
    f32x16 nd_next;
#pragma unroll
    for (int gi = 0; gi < 4; ++gi) {
      const f32x4 d4 = lds_rdf4(al + BN1 * LBUF + kStep * 4 + gi * 32);
#pragma unroll
      for (int t = 0; t < 4; ++t) nd_next[gi * 4 + t] = d4[t];
    }
    // operand reads in flight per stream: at head dim 64 two keep the plain
    // kernel at 190 VGPRs + 64 AGPRs, i.e. two waves per SIMD (two
    // workgroups per CU), 17 % faster than one wave with four
    constexpr int AHEAD = D == 64 ? 2 : 4;
    u32x4 xs[AHEAD];
    V8 xt[AHEAD];
#pragma unroll
    for (int t = 0; t < AHEAD; ++t) { xs[t] = rd_sd(t); xt[t] = rd_tr(t); }

    // P / dS of step j, element by element (lane entry i: row 8 (i/4) + 4 hf + i%4),
    // in two halves one slot apart: exp, then mask / dS / packing.
    f32x4 l4[2];                           // LSE of rows group gi (double-buffered by gi parity)
    auto read_l = [&](int gi) __attribute__((always_inline)) { l4[gi & 1] = lds_rdf4(al + BUF * LBUF + gi * 32); };
    auto elem_exp = [&](int i) __attribute__((always_inline)) -> float {
      const int gi = i >> 2, t = i & 3;
      float sv = sacc[PJ][i];
      if constexpr (SCORE) sv += sreg[i];
      float p = exp2_fast(fmaf(sv, c2, -l4[gi & 1][t]));
      asm volatile("" : "+v"(p));
      return p;
    };
    // keep word of the step (EDGE): bit 8 gi + t <-> entry (gi, t); causal
    // keeps the bit positions from dkq on.  An entry then costs a
    // sign-extended bit extract and an AND (a dropped p becomes +0).
    uint32_t keepw = ~0u;
    if constexpr (EDGE) {
      if constexpr (MASK) keepw = mreg;
      if constexpr (CAUSAL) keepw &= dkq <= 0 ? ~0u : (dkq >= 32 ? 0u : ~0u << dkq);
    }
    auto elem_fin = [&](int i, float p) __attribute__((always_inline)) {
      const int gi = i >> 2, t = i & 3;
      if constexpr (EDGE) {
        const uint32_t m = (uint32_t)((int32_t)(keepw << (31 - (8 * gi + t))) >> 31);
        p = __builtin_bit_cast(float, __builtin_bit_cast(uint32_t, p) & m);
      }
      sacc[PJ][i] = p;
      pacc[PJ][i] = p * pacc[PJ][i];   // P (dP - Delta); the factor scale goes into dK
      if constexpr (PREC) {
        // per pair of entries: the packed 16-bit words and their residuals
        if ((i & 1) == 1) {
          const int c = i >> 3, k = (i >> 1) & 3;
          uint32_t ph, pl, pl2, dh, dl;
          split3<T>(sacc[PJ][i - 1], sacc[PJ][i], &ph, &pl, &pl2);
          split2<T>(pacc[PJ][i - 1], pacc[PJ][i], &dh, &dl);
          u32x4 w0 = as_u32x4<T>(ppk[PJ][c]), w1 = as_u32x4<T>(ppl[PJ][c]), w4 = as_u32x4<T>(ppl2[PJ][c]);
          u32x4 w2 = as_u32x4<T>(dspk[PJ][c]), w3 = as_u32x4<T>(dsl[PJ][c]);
          w0[k] = ph; w1[k] = pl; w4[k] = pl2; w2[k] = dh; w3[k] = dl;
          ppk[PJ][c] = as_vec8<T>(w0); ppl[PJ][c] = as_vec8<T>(w1); ppl2[PJ][c] = as_vec8<T>(w4);
          dspk[PJ][c] = as_vec8<T>(w2); dsl[PJ][c] = as_vec8<T>(w3);
          asm volatile("" : "+v"(ppk[PJ][c]), "+v"(ppl[PJ][c]), "+v"(dspk[PJ][c]), "+v"(dsl[PJ][c]));
          asm volatile("" : "+v"(ppl2[PJ][c]));
        } else {
          asm volatile("" : "+v"(sacc[PJ][i]), "+v"(pacc[PJ][i]));
        }
      } else if ((i & 7) == 7) {
        const int c = i >> 3;
        ppk[PJ][c] = pack8<T>(sacc[PJ][8 * c + 0], sacc[PJ][8 * c + 1], sacc[PJ][8 * c + 2], sacc[PJ][8 * c + 3],
                              sacc[PJ][8 * c + 4], sacc[PJ][8 * c + 5], sacc[PJ][8 * c + 6], sacc[PJ][8 * c + 7]);
        dspk[PJ][c] = pack8<T>(pacc[PJ][8 * c + 0], pacc[PJ][8 * c + 1], pacc[PJ][8 * c + 2], pacc[PJ][8 * c + 3],
                               pacc[PJ][8 * c + 4], pacc[PJ][8 * c + 5], pacc[PJ][8 * c + 6], pacc[PJ][8 * c + 7]);
        asm volatile("" : "+v"(ppk[PJ][c]), "+v"(dspk[PJ][c]));
      } else {
        // keep the element's work in its slot (its result is first used later)
        asm volatile("" : "+v"(sacc[PJ][i]), "+v"(pacc[PJ][i]));
      }
    };

    // Slot t (own scheduling region): MFMAs of op t of both streams, the
    // operand reads of op t + AHEAD, the exp of elements of slot t and the
    // rest of the elements of slot t-1 (16/NOP elements per slot).
    constexpr int EPS = 16 / NOP;
    float pe[2][EPS];
    read_l(0);
#pragma unroll
    for (int t = 0; t < NOP; ++t) {
      // stream 1: S / dP of step j+1 (ds = t/2)
      if ((t & 1) == 0) sacc[PN] = mfma32(as_vec8<T>(xs[t % AHEAD]), kf[t >> 1], (t >> 1) == 0 ? f32x16{} : sacc[PN]);
      else pacc[PN] = mfma32(as_vec8<T>(xs[t % AHEAD]), vf[t >> 1], (t >> 1) == 0 ? nd_next : pacc[PN]);
      // dS of step j-1 out to its tile (non-temporal: read once, by the dQ kernel)
      if (t < 2) __builtin_amdgcn_raw_buffer_store_b128(__builtin_bit_cast(u32x4, dspk[PN][t]), ds_rs, ds_vo + 1024 * t, 0, 2);
      if constexpr (PREC) {   // the residual tile follows the tile
        if (t >= 2 && t < 4)
          __builtin_amdgcn_raw_buffer_store_b128(__builtin_bit_cast(u32x4, dsl[PN][t - 2]), ds_rs,
                                                 ds_vo + 2048 + 1024 * (t - 2), 0, 2);
      }
      // stream 2: dV / dK of step j-1 (c, nb)
      {
        const int c = t / (2 * NB), nb = (t / 2) % NB;
        if ((t & 1) == 0) {
          mfma_acc(dvt[nb], xt[t % AHEAD], ppk[PN][c]);
          if constexpr (PREC) {
            mfma_acc(dvt[nb], xt[t % AHEAD], ppl[PN][c]);
            mfma_acc(dvt[nb], xt[t % AHEAD], ppl2[PN][c]);
          }
        } else {
          mfma_acc(dkt[nb], xt[t % AHEAD], dspk[PN][c]);
          if constexpr (PREC) mfma_acc(dkt[nb], xt[t % AHEAD], dsl[PN][c]);
        }
      }
      if (t + AHEAD < NOP) { xs[t % AHEAD] = rd_sd(t + AHEAD); xt[t % AHEAD] = rd_tr(t + AHEAD); }
#pragma unroll
      for (int e = 0; e < EPS; ++e) {
        const int i = t * EPS + e;
        if ((i & 3) == 1 && i + 3 < 16) read_l((i >> 2) + 1);   // LSE of the next row group
        pe[t & 1][e] = elem_exp(i);
        if constexpr (SCORE) load_s(srs_next, i);   // step j+1's element i
      }
      if (t > 0) {
#pragma unroll
        for (int e = 0; e < EPS; ++e) elem_fin((t - 1) * EPS + e, pe[(t - 1) & 1][e]);
      }
      __builtin_amdgcn_sched_barrier(0);
    }
#pragma unroll
    for (int e = 0; e < EPS; ++e) elem_fin((NOP - 1) * EPS + e, pe[(NOP - 1) & 1][e]);
    if constexpr (CAUSAL && !MASK) {
      // Causal without a mask: P and dS leave the step only packed (dV, dK, the
      // dS tile), so the entries above the diagonal are cleared there, with a
      // 32-bit AND per pair of 16-bit entries, on the steps where some key of
      // this wave lies above some row (bit pattern AND, so an overflowed p of a
      // dropped entry goes too).  Entry i: row 8 (i/4) + 4 hf + i%4, kept iff
      // dkq <= 8 (i/4) + i%4.
      if (kw0 + 31 > it_qs) {
#pragma unroll
        for (int c = 0; c < 2; ++c) {
          u32x4 mk;
#pragma unroll
          for (int k = 0; k < 4; ++k) {
            const int i0 = 8 * c + 2 * k, i1 = i0 + 1;
            mk[k] = (dkq <= 8 * (i0 >> 2) + (i0 & 3) ? 0x0000ffffu : 0u) |
                    (dkq <= 8 * (i1 >> 2) + (i1 & 3) ? 0xffff0000u : 0u);
          }
          ppk[PJ][c] = __builtin_bit_cast(V8, __builtin_bit_cast(u32x4, ppk[PJ][c]) & mk);
          dspk[PJ][c] = __builtin_bit_cast(V8, __builtin_bit_cast(u32x4, dspk[PJ][c]) & mk);
          if constexpr (PREC) {
            ppl[PJ][c] = __builtin_bit_cast(V8, __builtin_bit_cast(u32x4, ppl[PJ][c]) & mk);
            ppl2[PJ][c] = __builtin_bit_cast(V8, __builtin_bit_cast(u32x4, ppl2[PJ][c]) & mk);
            dsl[PJ][c] = __builtin_bit_cast(V8, __builtin_bit_cast(u32x4, dsl[PJ][c]) & mk);
          }
        }
      }
    }
    // next step's dS descriptor and position
    next_step(j, mreg, pos_next);
  };

  // ---- prologue --------------------------------------------------------------------
  // The last buffer is read as step -1 (with P = dS = 0): zero it.
#pragma unroll
  for (int u = 0; u < UQ; ++u) {
    constexpr uint32_t zo = (NBUF - 1) * QST;
    if constexpr (SIX) {
      lds_wr16(lds_at(sw[u], sw2[u], zo), u32x4{0, 0, 0, 0});
      lds_wr16(lds_at(sw[u], sw2[u], zo + DOFF), u32x4{0, 0, 0, 0});
    } else {
      lds_wr16(sw[u] + zo, u32x4{0, 0, 0, 0});
      lds_wr16(sw[u] + zo + DOFF, u32x4{0, 0, 0, 0});
    }
  }
  load_next(IC<0>{}, IC<0>{}); store_tile(0, IC<0>{});   // tile 0
  load_next(IC<1>{}, IC<1>{}); store_tile(1, IC<1>{});   // tile 1
  if constexpr (SIX) {
    load_next(IC<0>{}, IC<0>{}); store_tile(2, IC<0>{}); // tile 2
    load_next(IC<1>{}, IC<0>{});                         // tile 3 staged (set 1)
    load_next(IC<0>{}, IC<0>{});                         // tile 4 staged (set 0)
  } else {
    load_next(IC<0>{}, IC<2>{});                         // tile 2 staged (set 0)
    load_next(IC<1>{}, IC<3>{});                         // tile 3 staged (set 1)
  }
  if constexpr (SCORE) {
    const auto rs0 = score_rs(it_h, it_qs, n > 0);
#pragma unroll
    for (int i = 0; i < 16; ++i) load_s(rs0, i);
  }
  lds_barrier();
  // S / dP of step 0 (parity 0); the dP chain starts from -Delta
  f32x16 nd0;
#pragma unroll
  for (int gi = 0; gi < 4; ++gi) {
    const f32x4 d4 = lds_rdf4(al + kStep * 4 + gi * 32);
#pragma unroll
    for (int t = 0; t < 4; ++t) nd0[gi * 4 + t] = d4[t];
  }
#pragma unroll
  for (int ds = 0; ds < DS; ++ds) {
    sacc[0] = mfma32(as_vec8<T>(lds_rd16(ab[ds])), kf[ds], ds == 0 ? f32x16{} : sacc[0]);
    pacc[0] = mfma32(as_vec8<T>(lds_rd16(ab[ds] + DOFF)), vf[ds], ds == 0 ? nd0 : pacc[0]);
  }

  // ---- main loop: iteration j computes P/dS(j), S/dP(j+1), dV/dK(j-1) ---------------
  // j runs over [0, nr) with nr = n + 1 rounded up to a multiple of NBUF: the
  // iterations past n - 1 work on zero tiles whose rows carry LSE = +inf, so
  // their P and dS are exactly 0 and they add nothing, while iteration n
  // contributes dV/dK(n-1).  NBUF copies of the body with static buffers and
  // a single loop exit keep the accumulators in fixed registers (an exit
  // after each copy made the register allocator spill).
  // Staging first: buffer (j+AHD)%NBUF is not read in iteration j, so tile
  // j+AHD (loaded two iterations earlier) is written while the MFMA stream
  // runs, and the loads of tile j+AHD+2 get two iterations of latency.
  auto step = [&](auto BUFc, int j) __attribute__((always_inline)) {
    constexpr int BUF = decltype(BUFc)::value;
    constexpr int SET = (BUF + AHD) & 1;              // staging set of tiles j+AHD and j+AHD+2
    store_tile((BUF + AHD) % NBUF, IC<SET>{});      // tile j+AHD
    // mask word of step j (loaded with tile j), before slot BUF is refilled
    const uint32_t mcur = MASK && j < n ? mq[MASK ? BUF % 4 : 0] >> (4 * hf) : 0u;
    const int pnext = pq[MASK ? (BUF + 1) % 4 : 0];   // position of step j+1 (loaded with tile j+1)
    load_next(IC<SET>{}, IC<BUF % 4>{});            // tile j+AHD+2 (with a mask: j+4, its word into slot BUF)
    // with a mask the keep test runs per entry on every step (a second copy of
    // the body for steps without dropped entries would not fit the register
    // budget); causal alone clears packed entries on the diagonal steps
    iter(BUFc, IC<MASK ? 1 : 0>{}, j, mcur, pnext);
    if constexpr (!SIX || (BUF & 1) != 0) lds_barrier();
  };
  if constexpr (SIX) {
    int nr = n > 0 ? (n + 6) / 6 * 6 : 0;
    asm volatile("" : "+s"(nr));   // hide the trip count (uniform: scalar register)
    for (int j = 0; j < nr; j += 6) {
      step(IC<0>{}, j);
      step(IC<1>{}, j + 1);
      step(IC<2>{}, j + 2);
      step(IC<3>{}, j + 3);
      step(IC<4>{}, j + 4);
      step(IC<5>{}, j + 5);
    }
  } else {
    int nr = n > 0 ? (n + 4) & ~3 : 0;
    asm volatile("" : "+s"(nr));
    for (int j = 0; j < nr; j += 4) {
      step(IC<0>{}, j);
      step(IC<1>{}, j + 1);
      step(IC<2>{}, j + 2);
      step(IC<3>{}, j + 3);
    }
  }

  mfma_acc_drain();   // before the epilogue reads the AGPR accumulators

  // ---- epilogue: dK, dV (dV of a kv-head with a dead row is NaN) ---------------------
  const bool dead = a.dead[b * a.Hk + kvh] != 0;
  const float nanv = __builtin_nanf("");
  lds_barrier();
  if (a.split == 1 && (a.acc_mode == 0 || a.acc_mode == 3)) {
    // stage [key][d] through LDS (wave-private rows), then coalesced 16-byte stores
    T* stg = (T*)smem + wave * 32 * OS;
    auto put = [&](const f32x16 (&acc)[NB], bool nan_out, T* dst, int64_t dstt) __attribute__((always_inline)) {
#pragma unroll
      for (int nb = 0; nb < NB; ++nb)
#pragma unroll
        for (int gi = 0; gi < 4; ++gi) {
          const int d = nb * 32 + gi * 8 + hf * 4;
          const u32x2 v = nan_out ? pack4<T>(nanv, nanv, nanv, nanv)
                                  : pack4<T>(acc[nb][gi * 4 + 0], acc[nb][gi * 4 + 1], acc[nb][gi * 4 + 2], acc[nb][gi * 4 + 3]);
          lds_write8(stg + l32 * OS + d, v);
        }
      asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
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
        if (kw0 + r < Tk) gstore16(dst + (int64_t)(kw0 + r) * dstt + c * 8, ov[u]);
      }
      asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
    };
    if (a.acc_mode == 3) {
      // last row range: the fp32 sums of the earlier ranges join (dK's scaled)
      if (key < Tk) {
#pragma unroll
        for (int nb = 0; nb < NB; ++nb)
#pragma unroll
          for (int gi = 0; gi < 4; ++gi) {
            const int64_t o = (((int64_t)b * Tk + key) * a.Hk + kvh) * D + nb * 32 + gi * 8 + hf * 4;
            const f32x4 k4 = *(const f32x4*)(a.dk_accum + o), v4 = *(const f32x4*)(a.dv_accum + o);
#pragma unroll
            for (int t = 0; t < 4; ++t) {
              dkt[nb][gi * 4 + t] = dkt[nb][gi * 4 + t] * scale + k4[t];
              dvt[nb][gi * 4 + t] += v4[t];
            }
          }
      }
    } else {
#pragma unroll
      for (int nb = 0; nb < NB; ++nb) dkt[nb] *= scale;
    }
    put(dkt, false, (T*)a.dk + b * a.dksb + kvh * a.dksh, a.dkst);
    put(dvt, dead, (T*)a.dv + b * a.dvsb + kvh * a.dvsh, a.dvst);
  } else {
    // fp32 slabs [split][B, Tk, Hk, D]: one per head-group split, summed in a
    // fixed order later; or, over row ranges, the running sums (acc_mode 1
    // writes them, 2 adds to them, in launch order)
    const int64_t slab = (int64_t)sp * a.B * Tk * a.Hk * D;
    const bool add = a.acc_mode == 2;
    if (key < Tk) {
#pragma unroll
      for (int nb = 0; nb < NB; ++nb)
#pragma unroll
        for (int gi = 0; gi < 4; ++gi) {
          const int d = nb * 32 + gi * 8 + hf * 4;
          const int64_t o = slab + (((int64_t)b * Tk + key) * a.Hk + kvh) * D + d;
          f32x4 k4, v4;
#pragma unroll
          for (int t = 0; t < 4; ++t) { k4[t] = dkt[nb][gi * 4 + t] * scale; v4[t] = dead ? nanv : dvt[nb][gi * 4 + t]; }
          if (add) {
            k4 += *(const f32x4*)(a.dk_accum + o);
            v4 += *(const f32x4*)(a.dv_accum + o);
          }
          *(f32x4*)(a.dk_accum + o) = k4;
          *(f32x4*)(a.dv_accum + o) = v4;
        }
    }
  }
}

template <typename T, int D, bool CAUSAL>
hipError_t launch_t(const BwdArgs& a, hipStream_t s) {
  const dim3 grid((unsigned)(a.nbk * a.nkt * a.nsp)), block(kKvWaves * 64);
  const bool m = a.mask != nullptr, sc = a.score != nullptr;
  if (m && sc) hipLaunchKernelGGL((dkdv2_kernel<T, D, CAUSAL, true, true>), grid, block, 0, s, a);
  else if (m) hipLaunchKernelGGL((dkdv2_kernel<T, D, CAUSAL, true, false>), grid, block, 0, s, a);
  else if (sc) hipLaunchKernelGGL((dkdv2_kernel<T, D, CAUSAL, false, true>), grid, block, 0, s, a);
  else hipLaunchKernelGGL((dkdv2_kernel<T, D, CAUSAL, false, false>), grid, block, 0, s, a);
  return hipGetLastError();
}

}  // namespace

int dkdv2_block_keys() { return kKvKeys; }

hipError_t launch_bwd_dkdv2(const BwdArgs& a, int D, int dtype, bool causal, hipStream_t s) {
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
