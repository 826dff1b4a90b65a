// FlashAttention-2 forward for gfx950 (MI355X) with optional 4D keep-mask and
// 4D fp32 score.  Restates the maths of the reference's TileLang forward
// (python/fa2.py:22-139) as a hand-written wave64 MFMA kernel.
//
// Work decomposition: one workgroup of 8 waves per (256 query rows, query
// head, batch); each wave owns 32 query rows and walks the key axis in tiles
// of 64 keys.  Per tile and wave:
//   S^T[key, q] = K Q^T        32x32x16 MFMA, A = K rows from LDS, B = Q
//                              fragment resident in registers
//   online softmax in base 2   each lane owns one query row (32 keys of it),
//                              the other half of the row sits in lane ^ 32
//   O^T[d, q] += V^T P^T       A = V^T via ds_read_b64_tr_b16 from the
//                              row-major V tile, B = P straight from the S^T
//                              accumulator registers (no LDS round trip)
//
// Softmax costs about as many VALU cycles as the two GEMMs cost MFMA cycles,
// so the two must overlap.  The waves form two groups (0-3, 4-7) that run the
// same step sequence one phase apart:
//   M(p): S(p) = K(p) Q^T and O += V(p-1)^T P(p-1)      (MFMA phase)
//   V(p): softmax of S(p) -> P(p)                        (VALU phase)
// Waves w and w+4 share a SIMD, so while one issues MFMAs the other issues
// VALU work; a workgroup barrier ends every pair of phases (every second pair
// with four K/V buffers).  The MFMA wave runs at a raised issue priority so
// that the softmax wave fills the gaps.
//
// K/V staging: three or four LDS buffers each for K and V.  In its softmax
// phase each wave writes its share of the tiles loaded one phase pair earlier (16 bytes
// per lane per chunk, held in registers meanwhile) and loads its share of the
// next ones, with buffer loads whose per-lane offsets are loop-invariant and
// whose tile base sits in scalar registers; rows past the end of the keys are
// zero-filled by the buffer range check.  (Direct global->LDS loads were
// measured slower here: their issue stalls once ~32 KB per CU are in flight.)
// Rows are stored unpadded with an XOR swizzle of their 16-byte chunks, chosen
// per tile kind so that the K reads (ds_read_b128, 16 rows per bank cycle) and
// the V reads (ds_read_b64_tr_b16, 4 rows x 4 chunks per bank cycle) are
// conflict-free.
//
// Softmax fast path: p = exp2(s c - m_run) with the running maximum m_run
// left unchanged, and the row sum taken over the fp32 p with plain adds
// (v_dot2 would issue to the matrix pipe, where it waits behind the other
// wave's MFMAs and delays them).  Only
// when some p exceeds 2^8 (the lane's partial sum tells, conservatively) or
// m_run is still -inf does the slow path compute the tile maximum, rescale
// O and l, and redo P.  That is exact (O and l always share one reference)
// and removes the max reduction and the rescale from almost every tile.
// m_run is the maximum of the row's first tile holding a kept key, m0, and
// afterwards moves only in whole steps (m0 + k, the tile maximum rounded up
// to that grid): the 16-bit P that enters the PV product is then
// round(2^frac(s c - m0)) times a power of two whichever m0 + k was current
// -- the same values as against the row's final maximum taken to that grid
// (the rescale factors are powers of two, so they add no rounding either).
#include "fa_common.h"
#include "fa_kernels.h"

namespace fa {
namespace {

constexpr int kWaves = 8;               // two groups of four
constexpr int kBM = kWaves * 32;        // query rows per workgroup
constexpr int kBN = 64;                 // keys per tile
constexpr int kThreads = kWaves * 64;
constexpr float kFastSumMax = 256.0f;   // lane partial sum bound of the fast path

template <int N> struct IC { static constexpr int value = N; };

// Chunk swizzles (16-byte chunks of a 2*D-byte tile row).
//  K: 16 lanes read one chunk of 16 consecutive rows -> 16 distinct bank groups.
//  V: 32 lanes read 4 chunks (4 m .. 4 m + 3) of 4 rows (4 r0 .. 4 r0 + 3).
template <int D> __device__ __forceinline__ int swz_k(int r) {
  return D == 128 ? (r & 15) : ((r >> 1) & 7);
}
template <int D> __device__ __forceinline__ int swz_v(int r) {
  return D == 128 ? ((r & 3) << 2) : (((r >> 1) & 1) << 2);
}

template <typename T>
__device__ __forceinline__ u32x2 pack4(float x0, float x1, float x2, float x3) {
  typedef T T4 __attribute__((ext_vector_type(4)));
  T4 v;
  v[0] = (T)x0; v[1] = (T)x1; v[2] = (T)x2; v[3] = (T)x3;
  return __builtin_bit_cast(u32x2, v);
}

// Hides x's value from the optimiser (keeps an address in one register).
__device__ __forceinline__ uint32_t opaque(uint32_t x) {
  asm volatile("" : "+v"(x));
  return x;
}
__device__ __forceinline__ u32x4 lds_read16_at(uint32_t addr) {
  return *(const FA_LDS u32x4*)(uintptr_t)addr;
}
__device__ __forceinline__ s16x4 lds_read_tr_at(uint32_t addr) {
  return __builtin_amdgcn_ds_read_tr16_b64_v4i16((FA_LDS s16x4*)(uintptr_t)addr);
}

__device__ __forceinline__ void lds_write16_at(uint32_t addr, u32x4 v) {
  *(FA_LDS u32x4*)(uintptr_t)addr = v;
}

// Workgroup barrier that waits for this wave's LDS traffic only.
__device__ __forceinline__ void lds_barrier() {
  __builtin_amdgcn_sched_barrier(0);
  asm volatile("s_waitcnt lgkmcnt(0)\n\ts_barrier" ::: "memory");
  __builtin_amdgcn_sched_barrier(0);
}
template <typename T, int D, bool CAUSAL, bool MASK, bool SCORE>
__global__ __launch_bounds__(kThreads, 1) void fwd_kernel(const FwdArgs a) {
  using V8 = typename Vec8<T>::type;
  constexpr int BM = kBM, BN = kBN;
  constexpr int DS = D / 16;            // k-steps of S^T
  constexpr int NB = D / 32;            // 32-wide d blocks of O^T
  constexpr int CH = D / 8;             // 16-byte chunks per row
  constexpr int ROWB = 2 * D;           // bytes per tile row
  constexpr int TILEB = BN * ROWB;      // bytes per K or V tile
  constexpr int NI = TILEB / 1024;      // 1 KB slots (64 lanes x 16 bytes) per tile
  constexpr int IPW = NI / kWaves;      // ... staged by each wave
  constexpr int RPI = 1024 / ROWB;      // tile rows per slot
  constexpr int NSTG = 2 * IPW;         // staging registers (x 16 bytes) per lane: K + V
  // With a score at head dim 128 the registers are short (the score of the
  // next tile, P and its residual): each wave's Q rows live in LDS instead of
  // 32 registers (swizzled like K rows, read as the S MFMA's B operand).
  constexpr bool QLDS = SCORE && D == 128;
  // LDS buffers per tile kind: with four, a workgroup barrier every second
  // phase pair suffices; causal workgroups (short, ragged key ranges) run
  // faster with three and a barrier every pair; with Q in LDS three fit.
  constexpr int NBUF = CAUSAL || QLDS ? 3 : 4;
  constexpr int KOFF = 0, VOFF = NBUF * TILEB;
  static_assert(NI % kWaves == 0 && IPW >= 1, "staging split");
  static_assert(NBUF * TILEB <= 65536, "buffer + row offsets fit the 16-bit DS immediate");
  constexpr int OS = D + 8;             // epilogue O staging stride (elements)
  static_assert(kWaves * 32 * OS * 2 <= 2 * NBUF * TILEB, "O staging fits in the K/V buffers");
  static_assert(BM == kFwdRows && BN == kFwdKeys, "prepared-mask lists are built for this tile shape");
  // With a mask or a score, P enters O += P V as two 16-bit halves (the
  // rounded value and its rounding residual, one more MFMA each): rows that
  // see few keys (packed documents, steep position biases) would otherwise
  // carry the 16-bit rounding of their few large weights into O.
  constexpr bool PREC = MASK || SCORE;
  constexpr int QOFF = 2 * NBUF * TILEB;                 // Q rows (QLDS): 32 per wave
  constexpr int QBYTES = QLDS ? kWaves * 32 * ROWB : 0;
  __shared__ __attribute__((aligned(1024))) char smem[2 * NBUF * TILEB + QBYTES];

  // ---- which (batch, head, query tile) -------------------------------------
  // Logical order (b, kv-head, [query tile rank, head in group]), with a
  // mask (kv-head, b, ...) so that batches of different mask density mix
  // on every XCD; with the XCD remap each XCD works on few kv-heads (K/V stay
  // in its L2), and the longest workgroups are dispatched first: rank r is
  // query tile nqt-1-r (causal work grows with the tile), with a mask the
  // tile with the r-th most live key tiles.
  const int nblk = a.B * a.Hq * a.nqt;
  const int W = xcd_remap(blockIdx.x, nblk);
  const int per_kv = a.G * a.nqt;
  const int bk = W / per_kv;
  const int rem = W - bk * per_kv;
  const int qt_rank = rem / a.G;
  const int g = rem - qt_rank * a.G;
  const int b = MASK ? bk % a.B : bk / a.Hk, kvh = MASK ? bk / a.B : bk - b * a.Hk;
  const int h = kvh * a.G + g;
  const int qt = MASK ? mask_order(a.ml, a.mws, mask_plane(a.ml, b, h), 0)[qt_rank] : a.nqt - 1 - qt_rank;

  const int tid = threadIdx.x, lane = tid & 63;
  // D = 64: the softmax phase is over twice the MFMA phase, and the two
  // groups run in step (no phase offset), which measured 6 % faster there;
  // D = 128 needs the offset (in step it ran 3x slower)
  const int wave = tid >> 6, grp = D == 128 ? wave >> 2 : 0;
  const int l32 = lane & 31, hf = lane >> 5;
  const int q0 = qt * BM, q0w = q0 + wave * 32;
  const int qrow = q0w + l32;
  const int Tq = a.Tq, Tk = a.Tk;

  const T* __restrict__ qp = (const T*)a.q + b * a.qsb + h * a.qsh;
  const T* __restrict__ kp = (const T*)a.k + b * a.ksb + kvh * a.ksh;
  const T* __restrict__ vp = (const T*)a.v + b * a.vsb + kvh * a.vsh;

  // ---- Q fragment: lane holds Q[qrow][16 ds + 8 hf + 0..7] -------------------
  V8 qf[QLDS ? 1 : DS];
  auto load_q = [&]() __attribute__((always_inline)) {
    const uint32_t neg = a.qsign < 0.f ? 0x80008000u : 0u;
    const T* src = qp + (int64_t)min(qrow, Tq - 1) * a.qst + hf * 8;
#pragma unroll
    for (int ds = 0; ds < DS; ++ds) {
      u32x4 x = gload16(src + ds * 16);
      x ^= neg;
      qf[QLDS ? 0 : ds] = as_vec8<T>(x);
    }
  };

  // Key tiles of the workgroup: 0 .. nt-1, or with a mask the live tiles of
  // the prepared list (ascending; bit 31: every entry of the tile is kept).
  const int qrow_c = min(qrow, Tq - 1);  // clamped row for mask/score reads
  const int32_t* flist = nullptr;
  const uint32_t* mbits = nullptr;
  if constexpr (MASK) {
    const int pm = mask_plane(a.ml, b, h);
    flist = (const int32_t*)(a.mws + a.ml.lfwd + pm * a.ml.plfwd) + (int64_t)qt * (1 + a.ml.nft);
    mbits = (const uint32_t*)(a.mws + a.ml.bits + pm * a.ml.pbits) + (int64_t)qrow_c * a.ml.wk;
  }
  const int kv_end = CAUSAL ? min(Tk, q0 + BM) : Tk;
  // with a mask: count and first two entries in one scalar load (the words
  // past a short list are still inside the workspace; only used when valid)
  int32_t fl[3] = {0, 0, 0};
  if constexpr (MASK) {
#pragma unroll
    for (int i = 0; i < 3; ++i) fl[i] = flist[i];
  }
  const int nt = MASK ? fl[0] : (kv_end + BN - 1) / BN;
  // tiles of this wave (opaque: keeps the per-pair guards dynamic, so that
  // every instantiation gets the same control flow and register assignment);
  // with a mask every wave walks the whole list (causality is applied per key)
  const int nt_w = (int)opaque((uint32_t)(CAUSAL && !MASK ? min(nt, (min(Tk, q0w + 32) + BN - 1) / BN) : nt));
  // List entries: a window of 128 positions sits in two registers (lane i
  // of ents[w] holds position ebase + 64 w + i) and is read with readlane,
  // so that walking the list costs no memory waits in the pipeline; it moves
  // by 64 positions when a pair would read past it (a pair reads positions
  // p .. p+3).
  constexpr bool ENTV = MASK;
  constexpr bool MPRE = MASK && !SCORE;   // mask bits fetched a pair ahead (no registers to spare with a score)
  int32_t ents[2] = {};   // unused without a mask
  int ebase = 0;
  // range-checked loads (positions past the row read 0): no wait on the count
  const auto rl = __builtin_amdgcn_make_buffer_rsrc((void*)flist, (short)0, MASK ? (1 + a.ml.nft) * 4 : 0, 0x00020000);
  auto fill_ents = [&](int base) __attribute__((always_inline)) {
#pragma unroll
    for (int w = 0; w < 2; ++w)
      ents[w] = (int32_t)__builtin_amdgcn_raw_buffer_load_b32(rl, (uint32_t)(1 + base + 64 * w + lane) * 4, 0, 0);
    ebase = base;
  };
  if constexpr (ENTV) fill_ents(0);
  auto move_ents = [&](int p) __attribute__((always_inline)) {   // before pair p's reads
    if constexpr (ENTV) {
      if (p + 3 >= ebase + 128) {
        fill_ents(ebase + 64);
        // consumed inside the branch: loads still pending where it rejoins
        // would make every pair wait for all of the wave's loads
        asm volatile("" : "+v"(ents[0]), "+v"(ents[1]));
      }
    }
  };
  auto ent_at = [&](int p) __attribute__((always_inline)) -> int32_t {
    const int r = p - ebase;
    const int32_t lo = __builtin_amdgcn_readlane(ents[0], r & 63);
    const int32_t hi = __builtin_amdgcn_readlane(ents[1], r & 63);
    return r < 64 ? lo : hi;
  };
  // key tile at list position p < nt
  auto tile_at = [&](int p) __attribute__((always_inline)) -> int {
    if constexpr (MASK) return ent_at(p) & 0x7fffffff;
    else return p;
  };

  const uint32_t lds0 = (uint32_t)(uintptr_t)(FA_LDS char*)smem;

  // ---- K/V staging ------------------------------------------------------------
  // Slot n of a tile (wave w stages n = w IPW .. + IPW-1): lane l -> tile row
  // r = n RPI + l / CH, logical chunk c = l % CH (1 KB of whole rows, read
  // coalesced), written at physical chunk c ^ swz(r) of row r.
  uint32_t goff_k[IPW], goff_v[IPW], soff_k[IPW], soff_v[IPW];
#pragma unroll
  for (int u = 0; u < IPW; ++u) {
    const int r = (wave * IPW + u) * RPI + lane / CH, c = lane % CH;
    goff_k[u] = (uint32_t)(r * a.kst * 2) + (uint32_t)(c * 16);
    goff_v[u] = (uint32_t)(r * a.vst * 2) + (uint32_t)(c * 16);
    soff_k[u] = opaque(lds0 + KOFF + r * ROWB + ((c ^ swz_k<D>(r)) * 16));
    soff_v[u] = opaque(lds0 + VOFF + r * ROWB + ((c ^ swz_v<D>(r)) * 16));
  }
  // Tile at list position p: rows [t BN, min(Tk, t BN + BN)) of t = tile_at(p);
  // p >= nt gives an empty range (the loads return zeros).
  // Key tile t (valid: rows [t BN, min(Tk, t BN + BN)); else an empty range:
  // the loads return zeros).
  auto rsrc_tile = [&](const T* base, int64_t st, int t, bool valid) __attribute__((always_inline)) {
    uint32_t nrec = 0;
    const T* tb = base;
    if (valid) {
      const int64_t rows = min(Tk - t * BN, BN);
      nrec = (uint32_t)min_i64((rows - 1) * st * 2 + ROWB, 0xfffffff0);
      tb = base + (int64_t)t * BN * st;
    }
    return __builtin_amdgcn_make_buffer_rsrc((void*)tb, (short)0, (int)nrec, 0x00020000);
  };
  auto rsrc_of = [&](const T* base, int64_t st, int p) __attribute__((always_inline)) {
    return p < nt ? rsrc_tile(base, st, tile_at(p), true) : rsrc_tile(base, st, 0, false);
  };
  u32x4 stg[NSTG];   // K slots, then V slots, of the next batch
  // Without a mask, list position = key tile, and the batch descriptors come
  // from running tile pointers and three record counts (full tile, the last
  // partial tile, none) instead of a 64-bit multiply per tile: the loads are
  // issued in the softmax phase, whose instruction issue bounds the step.
  const int nt_full = min(nt, Tk / BN);   // tiles [0, nt_full) are whole
  auto nrec_of = [&](int64_t st) __attribute__((always_inline)) -> uint32_t {
    return (uint32_t)min_i64((int64_t)(BN - 1) * st * 2 + ROWB, 0xfffffff0);
  };
  const uint32_t nrec_k = nrec_of(a.kst), nrec_v = nrec_of(a.vst);
  const uint32_t tail_k = (uint32_t)((int64_t)(Tk - nt_full * BN - 1) * a.kst * 2 + ROWB);
  const uint32_t tail_v = (uint32_t)((int64_t)(Tk - nt_full * BN - 1) * a.vst * 2 + ROWB);
  const T* kb_run = kp + (int64_t)2 * BN * a.kst;   // K(p+2) of the batch loaded next
  const T* vb_run = vp + (int64_t)BN * a.vst;       // V(p+1)
  auto rsrc_run = [&](const T* tb, uint32_t full, uint32_t tail, int t) __attribute__((always_inline)) {
    const uint32_t nrec = t < nt_full ? full : (t < nt ? tail : 0u);
    return __builtin_amdgcn_make_buffer_rsrc((void*)tb, (short)0, (int)nrec, 0x00020000);
  };
  // Descriptors of the batch of pair p: K(p+2) -> K buffer (p+2)%3, V(p+1) ->
  // V buffer (p+1)%3.  Called once per pair, in pair order, outside the
  // per-group branches (the running pointers stay in scalar registers).
  struct Rs2 { __amdgpu_buffer_rsrc_t k, v; };
  auto batch_rsrc = [&](int p) __attribute__((always_inline)) -> Rs2 {
    if constexpr (MASK) {
      return Rs2{rsrc_of(kp, a.kst, p + 2), rsrc_of(vp, a.vst, p + 1)};
    } else {
      const Rs2 r{rsrc_run(kb_run, nrec_k, tail_k, p + 2), rsrc_run(vb_run, nrec_v, tail_v, p + 1)};
      kb_run += (int64_t)BN * a.kst;
      vb_run += (int64_t)BN * a.vst;
      return r;
    }
  };
  auto load_batch = [&](const Rs2& r) __attribute__((always_inline)) {
#pragma unroll
    for (int u = 0; u < IPW; ++u) {
      stg[u] = __builtin_amdgcn_raw_buffer_load_b128(r.k, goff_k[u], 0, 0);
      stg[IPW + u] = __builtin_amdgcn_raw_buffer_load_b128(r.v, goff_v[u], 0, 0);
    }
  };
  auto store_batch = [&](int kbuf, int vbuf) __attribute__((always_inline)) {
#pragma unroll
    for (int u = 0; u < IPW; ++u) {
      lds_write16_at(soff_k[u] + kbuf * TILEB, stg[u]);
      lds_write16_at(soff_v[u] + vbuf * TILEB, stg[IPW + u]);
    }
  };
  // Prologue tiles K(0), K(1), V(0) of list positions 0 and 1 (from the
  // scalar-loaded first entries), straight to LDS: the loads of all three
  // first, then the LDS writes (the compiler does not move a buffer load
  // above an LDS store, so interleaved they waited for each tile in turn).
  auto put_tiles = [&]() __attribute__((always_inline)) {
    const int t0 = MASK ? (fl[1] & 0x7fffffff) : 0, t1 = MASK ? (fl[2] & 0x7fffffff) : 1;
    const auto rk0 = rsrc_tile(kp, a.kst, t0, 0 < nt), rk1 = rsrc_tile(kp, a.kst, t1, 1 < nt);
    const auto rv0 = rsrc_tile(vp, a.vst, t0, 0 < nt);
    u32x4 xk0[IPW], xk1[IPW], xv0[IPW];
#pragma unroll
    for (int u = 0; u < IPW; ++u) {
      xk0[u] = __builtin_amdgcn_raw_buffer_load_b128(rk0, goff_k[u], 0, 0);
      xk1[u] = __builtin_amdgcn_raw_buffer_load_b128(rk1, goff_k[u], 0, 0);
      xv0[u] = __builtin_amdgcn_raw_buffer_load_b128(rv0, goff_v[u], 0, 0);
    }
#pragma unroll
    for (int u = 0; u < IPW; ++u) {
      lds_write16_at(soff_k[u], xk0[u]);
      lds_write16_at(soff_k[u] + TILEB, xk1[u]);
      lds_write16_at(soff_v[u], xv0[u]);
    }
  };

  // ---- per-lane LDS read addresses -------------------------------------------
  // Byte addresses of buffer 0 of each kind; the buffer, k-block and key-row
  // offsets are compile-time immediates (< 64 KB) added per read.  opaque()
  // keeps the compiler from moving the region base into those immediates.
  // K (A operand of S^T): lane reads row 32 kb + l32, logical chunk 2 ds + hf.
  // With a score (registers short) one address: chunk 2 ds + hf of row l32
  // sits at 16 ((2 ds) ^ (hf ^ swz)) within the row, i.e. at kaddr0 ^ (32 ds)
  // (row starts are 256-byte aligned), one XOR per read instead of a register
  // per ds.
  constexpr bool KXOR = SCORE;
  uint32_t kaddr[KXOR ? 1 : DS];
  if constexpr (KXOR) {
    kaddr[0] = opaque(lds0 + KOFF + l32 * ROWB + ((hf ^ swz_k<D>(l32)) * 16));
  } else {
#pragma unroll
    for (int ds = 0; ds < DS; ++ds)
      kaddr[ds] = opaque(lds0 + KOFF + l32 * ROWB + (((2 * ds + hf) ^ swz_k<D>(l32)) * 16));
  }
  static_assert(ROWB % 256 == 0 || ROWB == 128, "row starts aligned for the XOR addressing");
  // Q rows in LDS (QLDS): chunk 2 ds + hf of row l32 at qaddr ^ (32 ds)
  uint32_t qaddr = 0;
  if constexpr (QLDS) qaddr = opaque(lds0 + QOFF + (wave * 32 + l32) * ROWB + ((hf ^ swz_k<D>(l32)) * 16));
  auto put_q = [&]() __attribute__((always_inline)) {
    const uint32_t neg = a.qsign < 0.f ? 0x80008000u : 0u;
    const T* src = qp + (int64_t)min(qrow, Tq - 1) * a.qst + hf * 8;
    u32x4 x[DS];
#pragma unroll
    for (int ds = 0; ds < DS; ++ds) x[ds] = gload16(src + ds * 16) ^ neg;
#pragma unroll
    for (int ds = 0; ds < DS; ++ds) lds_write16_at(qaddr ^ (uint32_t)(32 * ds), x[ds]);
  };
  // V (A operand of O^T via the transpose read): lane addresses key row
  // 32 (kk/2) + 16 (kk%2) + tr_row (+8), columns 32 nb + tr_col .. +3.
  const int tr_row = 4 * hf + ((lane >> 2) & 3);
  const int tr_col = ((lane >> 4) & 1) * 16 + (lane & 3) * 4;
  // (with a score one address again: chunk 4 nb + tr_col / 8 of the row at
  // vaddr0 ^ (64 nb), as for K)
  uint32_t vaddr[KXOR ? 1 : NB];
#pragma unroll
  for (int nb = 0; nb < (KXOR ? 1 : NB); ++nb) {
    const int c = nb * 32 + tr_col;
    vaddr[nb] = opaque(lds0 + VOFF + tr_row * ROWB + ((((c >> 3) ^ swz_v<D>(tr_row))) * 16) + (c & 7) * 2);
  }

  // Score of the wave's rows through one buffer descriptor from the wave's
  // first (clamped) row, whose range ends with the wave's last row: lane
  // offset = its row + 16 bytes per half-wave (+ the tile's keys); keys past
  // Tk read the next row or, past the last row, zeros (never kept: they are
  // masked below).  The host keeps the range below 2^32 bytes.
  const int srow0 = min(q0 + 32 * __builtin_amdgcn_readfirstlane(wave), Tq - 1);   // wave-uniform
  const __amdgpu_buffer_rsrc_t srs = __builtin_amdgcn_make_buffer_rsrc(
      SCORE ? (void*)(a.score + b * a.ssb + h * a.ssh + (int64_t)srow0 * a.ssq) : nullptr, (short)0,
      SCORE ? (int)(((int64_t)min(Tq - 1 - srow0, 31) * a.ssq + Tk) * 4) : 0, 0x00020000);
  const uint32_t soff_row = (uint32_t)((int64_t)(qrow_c - srow0) * a.ssq * 4) + hf * 16;
  const float c2 = a.scale_log2;

  f32x16 oacc[NB];
#pragma unroll
  for (int nb = 0; nb < NB; ++nb) oacc[nb] = f32x16{};
  f32x16 sacc[2] = {f32x16{}, f32x16{}};
  V8 pk[4];                        // P(p) packed, B operand of the next M step
  V8 pkl[PREC ? 4 : 1];            // ... and its rounding residual, P - pk (PREC)
#pragma unroll
  for (int kk = 0; kk < 4; ++kk) pk[kk] = V8{};
#pragma unroll
  for (int kk = 0; kk < (PREC ? 4 : 1); ++kk) pkl[kk] = V8{};
  // mask bits of the tile in flight as loaded: word kb holds keys 32 kb ..
  // 32 kb + 31 of this lane's row (used, shifted by 4 hf, only when mpart).
  // Loaded unconditionally (every listed tile's words exist) and used only
  // in the softmax phase: a conditional load whose result is used at once
  // made the compiler wait for all of the wave's loads right there.
  uint32_t mreg[2] = {~0u, ~0u};
  int tile_cur = 0;                // key tile of the tile in flight
  bool mpart = false;              // the tile in flight has dropped entries
  // Mask without a score: the list entry and mask bits of position p+1 are
  // loaded at the start of M(p) (the "next" set) and become current at the
  // start of M(p+1), so the softmax phase never waits for them.
  uint32_t mreg_nx[2] = {~0u, ~0u};
  int tile_nx = 0;
  bool mpart_nx = false;
  auto fetch_mask = [&](int p) __attribute__((always_inline)) {   // position p < nt_w -> next set
    const int e = p == 0 ? fl[1] : ent_at(p);
    tile_nx = e & 0x7fffffff;
    mpart_nx = e >= 0;
    const u32x2 w = *(const u32x2*)(mbits + 2 * tile_nx);
    mreg_nx[0] = w[0];
    mreg_nx[1] = w[1];
  };
  // With a mask and a score: position p's list entry and mask bits, loaded
  // at the start of M(p) and used in V(p).
  auto fetch_cur = [&](int p) __attribute__((always_inline)) {     // position p < nt_w
    const int e = ent_at(p);
    tile_cur = e & 0x7fffffff;
    mpart = e >= 0;
    const u32x2 w = *(const u32x2*)(mbits + 2 * tile_cur);
    mreg[0] = w[0];
    mreg[1] = w[1];
  };
  // Score of the next tile: the initial accumulator of its S chain (S = Score
  // + K Q^T, the score added before the scale as in the reference).  Loaded
  // in M(p) right after the first two MFMAs have taken tile p's score (in the
  // prologue for position 0), into the same registers: the loads get the rest
  // of M(p) and all of V(p) to arrive (issued at the start of V(p), the S
  // forward ran 7-9 % slower).
  f32x16 sc[SCORE ? 2 : 1];
  sc[0] = f32x16{};
  auto fetch_score = [&](int p) __attribute__((always_inline)) {   // position p < nt_w
    const int t = MASK ? (ent_at(p) & 0x7fffffff) : p;
    const uint32_t so = soff_row + (uint32_t)(t * BN * 4);   // range-checked: in the lane offset
#pragma unroll
    for (int kb = 0; kb < 2; ++kb)
#pragma unroll
      for (int gi = 0; gi < 4; ++gi) {
        const f32x4 x = __builtin_bit_cast(f32x4, __builtin_amdgcn_raw_buffer_load_b128(srs, so + (kb * 32 + gi * 8) * 4, 0, 0));
#pragma unroll
        for (int t4 = 0; t4 < 4; ++t4) sc[kb][gi * 4 + t4] = x[t4];
      }
  };
  float m_run = kNegInf, l_run = 0.f;

  // ---- M(p): S(p) = K(p) Q^T and O += V(p-1)^T P(p-1) ---------------------------
  // S(p) is computed (and later discarded) also when p >= nt_w, and PV(p-1)
  // also when p == 0 (P = 0 against a zeroed V buffer): one straight-line body.
  auto m_step = [&](auto KBc, int p) __attribute__((always_inline)) {
    constexpr int KB = decltype(KBc)::value;
    constexpr uint32_t kb_lds = KB * TILEB;                      // K(p), relative to K buffer 0
    constexpr uint32_t vb_lds = ((KB + NBUF - 1) % NBUF) * TILEB;  // V(p-1), relative to V buffer 0
    if constexpr (MPRE) {
      // position p's set (fetched in M(p-1) or the prologue) becomes current;
      // fetch position p+1's
      tile_cur = tile_nx;
      mpart = mpart_nx;
      mreg[0] = mreg_nx[0];
      mreg[1] = mreg_nx[1];
      if (p + 1 < nt_w) fetch_mask(p + 1);
    }
    if constexpr (MASK && SCORE) {
      if (p < nt_w) fetch_cur(p);
    }
    if constexpr (SCORE) {
      // a negative scale is folded into Q and the score's sign (rare: the
      // wait for the score loads happens here only then)
      if (a.qsign < 0.f) {
        sc[0] = -sc[0];
        sc[1] = -sc[1];
      }
    }
    __builtin_amdgcn_s_setprio(2);
    // The two independent chains interleaved, S op t = (kb = t%2, ds = t/2),
    // PV op t = (kk = t/NB, nb = t%NB); operands are read from LDS AHEAD op
    // pairs before their MFMAs.
    constexpr int NOP = 2 * DS;   // == 4 * NB
    constexpr int AHEAD = SCORE ? 2 : 3;
    auto rd_s = [&](int t) __attribute__((always_inline)) -> u32x4 {
      const uint32_t ka = KXOR ? (kaddr[0] ^ (uint32_t)(32 * (t >> 1))) : kaddr[t >> 1];
      return lds_read16_at(ka + kb_lds + (uint32_t)((t & 1) * 32 * ROWB));
    };
    auto rd_pv = [&](int t) __attribute__((always_inline)) -> V8 {
      const int kk = t / NB, nb = t % NB;
      const uint32_t row = (kk >> 1) * 32 + 16 * (kk & 1);
      const uint32_t va = KXOR ? (vaddr[0] ^ (uint32_t)(64 * nb)) : vaddr[nb];
      const uint32_t base = va + vb_lds + row * ROWB;
      return cat_tr<T>(lds_read_tr_at(base), lds_read_tr_at(base + 8 * ROWB));
    };
    u32x4 kq[AHEAD];
    V8 vq[AHEAD];
    u32x4 qv[2];   // Q chunks ds and ds + 1 (QLDS)
#pragma unroll
    for (int t = 0; t < AHEAD; ++t) {
      kq[t] = rd_s(t);
      vq[t] = rd_pv(t);
    }
    if constexpr (QLDS) qv[0] = lds_read16_at(qaddr);
    __builtin_amdgcn_sched_group_barrier(0x100, 3 * AHEAD + (QLDS ? 1 : 0), 0);
#pragma unroll
    for (int t = 0; t < NOP; ++t) {
      const int kb = t & 1, ds = t >> 1;
      const V8 qb = QLDS ? as_vec8<T>(qv[ds & 1]) : qf[QLDS ? 0 : ds];
      sacc[kb] = mfma32(as_vec8<T>(kq[t % AHEAD]), qb, ds == 0 ? (SCORE ? sc[kb] : f32x16{}) : sacc[kb]);
      oacc[t % NB] = mfma32(vq[t % AHEAD], pk[t / NB], oacc[t % NB]);
      if constexpr (PREC) oacc[t % NB] = mfma32(vq[t % AHEAD], pkl[t / NB], oacc[t % NB]);
      if (t + AHEAD < NOP) {
        kq[t % AHEAD] = rd_s(t + AHEAD);
        vq[t % AHEAD] = rd_pv(t + AHEAD);
      }
      // Q chunk ds + 1, two ops before its first use (its slot last served ds - 1)
      const bool qrd = QLDS && kb == 0 && ds + 1 < DS;
      if (qrd) qv[(ds + 1) & 1] = lds_read16_at(qaddr ^ (uint32_t)(32 * (ds + 1)));
      __builtin_amdgcn_sched_group_barrier(0x008, PREC ? 3 : 2, 0);
      if (t + AHEAD < NOP) {
        if (qrd) __builtin_amdgcn_sched_group_barrier(0x100, 4, 0);
        else __builtin_amdgcn_sched_group_barrier(0x100, 3, 0);
      } else if (qrd) {
        __builtin_amdgcn_sched_group_barrier(0x100, 1, 0);
      }
      if constexpr (SCORE) {
        // the score of tile p is in the S chains now: its registers take the
        // next tile's (position p + 1; past the list, a harmless valid read)
        if (t == 1) {
          fetch_score(p + 1);
          __builtin_amdgcn_sched_group_barrier(0x020, 8, 0);
        }
      }
    }
    __builtin_amdgcn_s_setprio(0);
  };

  // P = exp2(S c - m) packed into pk; returns the lane's partial row sum.
  auto make_p = [&](float mneg) __attribute__((always_inline)) -> float {
    float lsum = 0.f;
#pragma unroll
    for (int kk = 0; kk < 4; ++kk) {
      const int kb = kk >> 1, c = kk & 1;
      float x[8];
#pragma unroll
      for (int t = 0; t < 8; ++t) x[t] = exp2_fast(fmaf(sacc[kb][8 * c + t], c2, mneg));
      pk[kk] = pack8<T>(x[0], x[1], x[2], x[3], x[4], x[5], x[6], x[7]);
      if constexpr (PREC) {
        // residual of each rounded p (exact in fp32), itself rounded: pk + pkl
        // carries p to about 16 significant bits
        float r[8];
#pragma unroll
        for (int t = 0; t < 8; ++t) r[t] = x[t] - (float)(T)x[t];
        pkl[kk] = pack8<T>(r[0], r[1], r[2], r[3], r[4], r[5], r[6], r[7]);
      }
      lsum += ((x[0] + x[1]) + (x[2] + x[3])) + ((x[4] + x[5]) + (x[6] + x[7]));
    }
    return lsum;
  };

  // ---- V(p): softmax of S(p) -> P(p) ----------------------------------------------
  // lane's entry (kb, e) is key 64 p + 32 kb + 8 (e/4) + 4 hf + e%4 of row qrow;
  // key slot t of k-step kk (= 2 kb + c) <-> key 32 kb + 16 c + 4 hf + t%4 + 8 (t/4)
  auto v_step = [&](int p, auto&& stage) __attribute__((always_inline)) {
    const int k0 = (MASK ? tile_cur : p) * BN;
    if constexpr (SCORE) {
      // (fetched in M(p))
    }
    const bool edge = (MASK && mpart) || a.zero_scale || (k0 + BN > Tk) || (CAUSAL && k0 + BN - 1 > q0w);
    if (edge) {
      // Keep word of each 32-key half: bit 8 gi + t <-> key k0 + 32 kb +
      // 8 gi + 4 hf + t; keys at or past Tk (causal: past the row) are a
      // suffix of the bit positions.  Each entry then costs a sign-extended
      // bit extract and one bitwise select against -inf (scale 0: against 0
      // for the kept logits, in a copy of its own).
      const int lim = CAUSAL ? min(Tk, qrow + 1) : Tk;
      auto apply = [&](auto ZEROc) __attribute__((always_inline)) {
#pragma unroll
        for (int kb = 0; kb < 2; ++kb) {
          const int n = lim - (k0 + 32 * kb + 4 * hf);
          uint32_t keepw = n >= 32 ? ~0u : (n <= 0 ? 0u : (1u << n) - 1u);
          if constexpr (MASK) keepw &= mpart ? mreg[kb] >> (4 * hf) : ~0u;
#pragma unroll
          for (int gi = 0; gi < 4; ++gi)
#pragma unroll
            for (int t = 0; t < 4; ++t) {
              const uint32_t m = (uint32_t)((int32_t)(keepw << (31 - (8 * gi + t))) >> 31);
              // (through a float copy: this compiler's bit_cast of a vector
              // element operand reads element 0)
              const float f = decltype(ZEROc)::value ? 0.f : sacc[kb][gi * 4 + t];
              const uint32_t sv = __builtin_bit_cast(uint32_t, f);
              sacc[kb][gi * 4 + t] = __builtin_bit_cast(float, (sv & m) | (0xff800000u & ~m));
              asm volatile("" : "+v"(keepw));   // one entry at a time (no 32 live masks)
            }
        }
      };
      if constexpr (MASK || SCORE || CAUSAL) {
        if (a.zero_scale) apply(IC<1>{});
        else apply(IC<0>{});
      } else {
        // no mask, score or causality: only the last, partial key tile and
        // scale 0 come here (per-entry selects: the plain kernel's register
        // assignment stays as it is without the keep-word code)
#pragma unroll
        for (int kb = 0; kb < 2; ++kb)
#pragma unroll
          for (int gi = 0; gi < 4; ++gi) {
            const int kk = k0 + kb * 32 + gi * 8 + hf * 4;
#pragma unroll
            for (int t = 0; t < 4; ++t) {
              const float sv = sacc[kb][gi * 4 + t];
              sacc[kb][gi * 4 + t] = kk + t < Tk ? (a.zero_scale ? 0.f : sv) : kNegInf;
            }
          }
      }
    }
    // The mask/score registers are consumed: loads issued from here on do not
    // delay this wave's next wait for them.
    stage();
    // Fast path against the current m_run (+inf offset while m_run is -inf,
    // which makes the sum inf or NaN and forces the slow path).
    float lsum = make_p(-m_run);
    if (wave_any(!(lsum <= kFastSumMax))) {
      float mx = kNegInf;
#pragma unroll
      for (int kb = 0; kb < 2; ++kb)
#pragma unroll
        for (int e = 0; e < 16; ++e) mx = fmaxf(mx, sacc[kb][e]);
      mx = half_max(mx);
      // the row's first tile with a kept key sets the reference maximum m0
      // (its largest p is exactly 1); later tiles raise it in whole steps:
      // p = exp2(s c - m0 - k) has the same mantissa for every integer k, so P
      // rounds to the same 16-bit values whichever maximum was current (and
      // alpha below is an exact power of two)
      const float mc = mx * c2;
      const float m_new = m_run == kNegInf ? mc : m_run + fmaxf(0.f, ceilf(mc - m_run));
      const float alpha = (m_run == kNegInf) ? 0.f : exp2_fast(m_run - m_new);
      l_run *= alpha;
#pragma unroll
      for (int nb = 0; nb < NB; ++nb)
#pragma unroll
        for (int e = 0; e < 16; ++e) oacc[nb][e] *= alpha;
      m_run = m_new;
      lsum = make_p(m_run == kNegInf ? 0.f : -m_run);
    }
    l_run += lsum;
  };

  // ---- prologue: zero the last V buffer (read as V(-1) with P = 0), K(0),
  // K(1), V(0) to LDS, batch 0 (K(2), V(1)) into the staging registers.
  {
    char* z = smem + VOFF + (NBUF - 1) * TILEB;
#pragma unroll
    for (int u = 0; u < TILEB / (kThreads * 16); ++u) lds_write16(z + (tid + u * kThreads) * 16, u32x4{0, 0, 0, 0});
  }
  if constexpr (QLDS) put_q();
  else load_q();
  if constexpr (MPRE) {
    if (nt_w > 0) fetch_mask(0);
  }
  if constexpr (SCORE) {
    if (nt_w > 0) fetch_score(0);
  }
  put_tiles();   // K(0), K(1), V(0)
  load_batch(batch_rsrc(0));
  lds_barrier();

  // ---- main loop over phase pairs p = 0 .. nt ------------------------------------
  // pair p: phase 2p   group 0: M(p)   group 1: V(p-1)
  //         phase 2p+1 group 0: V(p)   group 1: M(p)
  // In its softmax phase of pair p each wave stores its share of batch p
  // (K(p+2), V(p+1), loaded during pair p-1) and loads its share of batch
  // p+1 (pair p writes K buffer (p+2)%NBUF and V buffer (p+1)%NBUF).  With
  // three buffers those were last read in pair p-1 and a barrier ends every
  // pair; with four they were last read in pair p-2 and a barrier ends every
  // odd pair.  Either way a barrier lies between each write and the first
  // read, in pair p+2.  The two phases of a pair are not separated by a
  // barrier (the waves of a SIMD settle into the alternation by themselves,
  // and a phase that ends early does not wait).
  auto pair = [&](auto KBc, int p) __attribute__((always_inline)) {
    constexpr int KB = decltype(KBc)::value;   // p % NBUF
    constexpr bool BAR = NBUF == 3 || (KB & 1) != 0;
    move_ents(p);
    const Rs2 rs = batch_rsrc(p + 1);
    auto stage = [&]() __attribute__((always_inline)) {
      store_batch((KB + 2) % NBUF, (KB + 1) % NBUF);
      load_batch(rs);
    };
    if (grp == 0) {
      if (p <= nt_w) m_step(KBc, p);
    } else {
      if (p >= 1 && p - 1 < nt_w) v_step(p - 1, stage);
      else stage();
    }
    // D = 64 (one group: M then V in every wave): the phases are scheduled
    // apart, which keeps the live registers of one phase at a time (150
    // instead of 239 without a score; with a score 256 and spills before)
    if constexpr (D == 64) __builtin_amdgcn_sched_barrier(0);
    if (grp == 0) {
      if (p < nt_w) v_step(p, stage);
      else stage();
    } else {
      if (p <= nt_w) m_step(KBc, p);
    }
    if constexpr (BAR) lds_barrier();
  };
  for (int p = 0; p <= nt; p += NBUF) {
    pair(IC<0>{}, p);
    if (p + 1 > nt) break;
    pair(IC<1>{}, p + 1);
    if (p + 2 > nt) break;
    pair(IC<2>{}, p + 2);
    if constexpr (NBUF == 4) {
      if (p + 3 > nt) break;
      pair(IC<3>{}, p + 3);
    }
  }
  if constexpr (NBUF == 4) lds_barrier();   // all waves are done with the K/V buffers

  // ---- epilogue: O = acc / l (NaN for a row with no kept key), LSE ----------------
  const float l_tot = half_sum(l_run);
  const float inv = 1.0f / l_tot;
  T* os = (T*)smem + wave * 32 * OS;  // wave-private staging, K/V buffers are free now
#pragma unroll
  for (int nb = 0; nb < NB; ++nb)
#pragma unroll
    for (int gi = 0; gi < 4; ++gi) {
      const int d = nb * 32 + gi * 8 + hf * 4;
      lds_write8(os + l32 * OS + d,
                 pack4<T>(oacc[nb][gi * 4 + 0] * inv, oacc[nb][gi * 4 + 1] * inv, oacc[nb][gi * 4 + 2] * inv,
                          oacc[nb][gi * 4 + 3] * inv));
    }
  asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");  // wave-private region: no barrier needed
  T* op = (T*)a.o + b * a.osb + h * a.osh;
  // all staging reads first (one wait), then the row-guarded stores
  constexpr int NU = 32 * CH / 64;
  u32x4 ov[NU];
#pragma unroll
  for (int u = 0; u < NU; ++u) {
    const int idx = lane + u * 64;
    ov[u] = lds_read16(os + (idx / CH) * OS + (idx % CH) * 8);
  }
#pragma unroll
  for (int u = 0; u < NU; ++u) {
    const int idx = lane + u * 64;
    const int r = idx / CH, c = idx % CH;
    const int qr = q0w + r;
    if (qr < Tq) gstore16(op + (int64_t)qr * a.ost + c * 8, ov[u]);
  }
  if (hf == 0 && qrow < Tq)
    a.lse[((int64_t)b * a.Hq + h) * Tq + qrow] = (l_tot > 0.f) ? m_run + log2_fast(l_tot) : kPosInf;
  if constexpr (PREC) {
    // O's rounding residual (fp32 O minus O as stored, rounded), through the
    // same wave-private staging rows: Delta = rowsum(dO (O + residual)) then
    // sees O to about 16 significant bits
    if (a.olo) {
#pragma unroll
      for (int nb = 0; nb < NB; ++nb)
#pragma unroll
        for (int gi = 0; gi < 4; ++gi) {
          const int d = nb * 32 + gi * 8 + hf * 4;
          float r[4];
#pragma unroll
          for (int t = 0; t < 4; ++t) {
            const float o = oacc[nb][gi * 4 + t] * inv;
            r[t] = o - (float)(T)o;
          }
          lds_write8(os + l32 * OS + d, pack4<T>(r[0], r[1], r[2], r[3]));
        }
      asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
      T* lp = (T*)a.olo + b * a.olsb + h * a.olsh;
#pragma unroll
      for (int u = 0; u < NU; ++u) {
        const int idx = lane + u * 64;
        ov[u] = lds_read16(os + (idx / CH) * OS + (idx % CH) * 8);
      }
#pragma unroll
      for (int u = 0; u < NU; ++u) {
        const int idx = lane + u * 64;
        const int r = idx / CH, c = idx % CH;
        const int qr = q0w + r;
        if (qr < Tq) gstore16(lp + (int64_t)qr * a.olst + c * 8, ov[u]);
      }
    }
  }
}

template <typename T, int D, bool CAUSAL>
hipError_t launch_fwd_t(const FwdArgs& a, hipStream_t s) {
  const dim3 grid((unsigned)(a.B * a.Hq * a.nqt)), block(kThreads);
  const bool m = a.mask != nullptr, sc = a.score != nullptr;
  if (m && sc) hipLaunchKernelGGL((fwd_kernel<T, D, CAUSAL, true, true>), grid, block, 0, s, a);
  else if (m) hipLaunchKernelGGL((fwd_kernel<T, D, CAUSAL, true, false>), grid, block, 0, s, a);
  else if (sc) hipLaunchKernelGGL((fwd_kernel<T, D, CAUSAL, false, true>), grid, block, 0, s, a);
  else hipLaunchKernelGGL((fwd_kernel<T, D, CAUSAL, false, false>), grid, block, 0, s, a);
  return hipGetLastError();
}

template <typename T, int D>
hipError_t launch_fwd_d(const FwdArgs& a, bool causal, hipStream_t s) {
  return causal ? launch_fwd_t<T, D, true>(a, s) : launch_fwd_t<T, D, false>(a, s);
}

}  // namespace

int fwd_block_rows() { return kBM; }

hipError_t launch_fwd(const FwdArgs& a, int D, int dtype, bool causal, hipStream_t s) {
  if (dtype == 0) {
    if (D == 128) return launch_fwd_d<bf16, 128>(a, causal, s);
    if (D == 64) return launch_fwd_d<bf16, 64>(a, causal, s);
  } else {
    if (D == 128) return launch_fwd_d<f16, 128>(a, causal, s);
    if (D == 64) return launch_fwd_d<f16, 64>(a, causal, s);
  }
  return hipErrorInvalidValue;
}

}  // namespace fa
