// Attention kernels for head dims above 128 on gfx950 (MI355X): instances at
// head dim 256 (the host zero-pads other head dims in (128, 256], which is
// exact).  The reference's TileLang kernels take the head dim as a
// compile-time constant of any size (python/fa2.py:33); these restate their
// maths (forward python/fa2.py:22-139, backward :181-302 / :305-426) with
// tiles that operands of 512 bytes per row fit:
//
//   fwd_wide_kernel  one workgroup of 4 waves (one per SIMD, 512 registers
//                    each) per (128 query rows, query head, batch).  Each wave
//                    owns 32 rows: its Q fragment (64 registers) and its O^T
//                    accumulator (128) stay in registers while it walks the
//                    keys in tiles of 32:
//                      S^T = K Q^T     16 MFMAs, A = K rows from LDS
//                      online softmax  base 2, O and l rescaled only when a
//                                      row's maximum grows
//                      O^T += V^T P^T  16 MFMAs, A = V^T by transpose reads,
//                                      B = P straight from the S registers
//                    K/V tiles are double-buffered in LDS (rows padded so that
//                    the K row reads and the V transpose reads spread over the
//                    banks), staged through registers one tile ahead.
//   kv_wide_kernel   one workgroup of 4 waves per (128 keys, kv-head, batch
//                    [, head-group split]).  Each wave owns 32 keys with their
//                    K (and V) fragments in registers and walks the query rows
//                    of every head of its group in steps of 32 (Q/dO tiles
//                    double-buffered in LDS).  Two launches:
//                      WHICH 0 (dV)  S = Q K^T, P = exp2(S c - LSE),
//                                    dV^T += dO^T P
//                      WHICH 1 (dK)  S, dP = dO V^T - Delta, dS = P (dP - Delta),
//                                    dK^T += Q^T dS  (times scale at the end)
//                    A wave holding both accumulators (256 registers) and both
//                    fragments (128) beside its working set would not fit the
//                    register file at this head dim, so the dK launch
//                    recomputes S.
// dQ comes from the recompute kernel of fa_bwd.hip (dq_kernel), Delta and the
// backward's LSE from its preprocess kernel.  Conventions as in the head-dim
// 64/128 kernels: masked entries get P = 0 by select after the exp; rows past
// Tq carry LSE = +inf (P = 0); keys past Tk read key Tk-1 (finite) and are
// masked; with a mask or a score, P and dS enter their products in several
// 16-bit parts (P to fp32 precision in dV, dS to about 16 bits; P_hi + P_lo
// in O) and the forward writes O's rounding residual when asked.
#include "fa_common.h"
#include "fa_kernels.h"

namespace fa {
namespace {

constexpr int kWD = 256;         // head dim of these instances
constexpr int kWRows = 128;      // forward: query rows per workgroup
constexpr int kWKeys = 32;       // forward: keys per tile
constexpr int kWKvKeys = 128;    // dK/dV: keys per workgroup (4 waves x 32), 32-row steps
constexpr int kWDqRows = 128;    // dQ: query rows per workgroup (4 waves x 32), 32-key tiles
constexpr float kWLift = 8.f;    // forward: largest exponent of p against the running maximum


template <typename T>
__device__ __forceinline__ u32x2 pack4w(float x0, float x1, float x2, float x3) {
  typedef T T4 __attribute__((ext_vector_type(4)));
  T4 v;
  v[0] = (T)x0; v[1] = (T)x1; v[2] = (T)x2; v[3] = (T)x3;
  return __builtin_bit_cast(u32x2, v);
}

// ---------------------------------------------------------------------------
// forward
// ---------------------------------------------------------------------------
template <typename T, bool CAUSAL, bool MASK, bool SCORE>
__global__ __launch_bounds__(256, 1) void fwd_wide_kernel(const FwdArgs a) {
  using V8 = typename Vec8<T>::type;
  constexpr int D = kWD, DS = D / 16, NB = D / 32, CH = D / 8;
  constexpr int BM = kWRows, BN = kWKeys;
  // padded row strides (elements): K rows are read 16 bytes per lane over 16
  // rows (a stride of 4 mod 64 banks), V by 4-row transpose reads of 64
  // bytes per row (16 mod 64): both conflict-free
  constexpr int KS = D + 8, VS = D + 32;
  constexpr int KT = BN * KS, VT = BN * VS;
  constexpr int U = BN * CH / 256;      // 16-byte chunks per thread per tile and kind
  constexpr int OS = D + 8;             // epilogue staging stride
  static_assert(4 * 32 * OS <= 2 * (KT + VT), "O staging fits in the tile buffers");
  constexpr bool PREC = MASK || SCORE;
  // two K buffers, then two V buffers
  __shared__ __attribute__((aligned(16))) T smem[2 * (KT + VT)];

  // Causal: query tiles longest first (rank r = tile nqt-1-r), the rank
  // varying slowest so that every XCD (blocks go round-robin over the 8)
  // gets an equal share of each length.  Otherwise (equal work) logical
  // order (batch, kv-head, tile, head in group) contiguous per XCD, so each
  // XCD's L2 serves few kv-heads' K/V.
  int b, h, qt;
  if constexpr (CAUSAL) {
    const int bh = a.B * a.Hq;
    const int r = blockIdx.x / bh, i = blockIdx.x - r * bh;
    b = i / a.Hq;
    h = i - b * a.Hq;
    qt = a.nqt - 1 - r;
  } else {
    const int W = xcd_remap(blockIdx.x, a.B * a.Hq * a.nqt);
    const int per_kv = a.G * a.nqt;
    const int bk = W / per_kv, rem = W - bk * per_kv;
    qt = rem / a.G;
    b = bk / a.Hk;
    h = (bk - b * a.Hk) * a.G + (rem - qt * a.G);
  }
  const int kvh = h / a.G;

  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int l32 = lane & 31, hf = lane >> 5;
  const int Tq = a.Tq, Tk = a.Tk;
  const int q0 = qt * BM, q0w = q0 + wave * 32, qrow = q0w + l32;
  const int qrow_c = min(qrow, Tq - 1);
  const float c2 = a.scale_log2;

  // Q fragment (B of S^T): lane holds Q[qrow][16 ds + 8 hf .. +7]; a negative
  // scale is folded into Q's sign (and the score's)
  V8 qf[DS];
  {
    const uint32_t neg = a.qsign < 0.f ? 0x80008000u : 0u;
    const T* src = (const T*)a.q + b * a.qsb + h * a.qsh + (int64_t)qrow_c * a.qst + hf * 8;
#pragma unroll
    for (int ds = 0; ds < DS; ++ds) qf[ds] = as_vec8<T>(gload16(src + ds * 16) ^ neg);
  }
  // The fragment stays in AGPRs (MFMA reads its operands there too): 64
  // VGPRs that the pipelined loop needs, which the compiler otherwise shuffles
  // through AGPRs every iteration.
#pragma unroll
  for (int ds = 0; ds < DS; ++ds) asm volatile("" : "+a"(qf[ds]));
  const T* __restrict__ kp = (const T*)a.k + b * a.ksb + kvh * a.ksh;
  const T* __restrict__ vp = (const T*)a.v + b * a.vsb + kvh * a.vsh;
  const uint32_t* mbits = nullptr;
  if constexpr (MASK) {
    const int pm = mask_plane(a.ml, b, h);
    mbits = (const uint32_t*)(a.mws + a.ml.bits + pm * a.ml.pbits) + (int64_t)qrow_c * a.ml.wk;
  }
  // score rows of the wave through one range-checked buffer from its first
  // row (the host keeps 32 rows below 4 GiB); keys past Tk read the next row
  // or zeros and are masked
  const int srow0 = min(q0 + 32 * __builtin_amdgcn_readfirstlane(wave), Tq - 1);
  const __amdgpu_buffer_rsrc_t srs = __builtin_amdgcn_make_buffer_rsrc(
      SCORE ? (void*)(a.score + b * a.ssb + h * a.ssh + (int64_t)srow0 * a.ssq) : nullptr, (short)0,
      SCORE ? (int)(((int64_t)min(Tq - 1 - srow0, 31) * a.ssq + Tk) * 4) : 0, 0x00020000);
  const uint32_t soff_row = (uint32_t)((int64_t)(qrow_c - srow0) * a.ssq * 4) + hf * 16;

  const int kv_end = CAUSAL ? min(Tk, q0 + BM) : Tk;
  const int nt = (kv_end + BN - 1) / BN;

  // staging: chunk u of thread t is row idx / CH, chunk idx % CH of a tile
  // (idx = t + 256 u), loaded through a descriptor from the tile's first key
  // whose records end after key Tk-1 (keys past Tk read zeros: their P is 0),
  // with loop-invariant lane offsets
  u32x4 kreg[U], vreg[U];
  uint32_t goff_k[U], goff_v[U];
#pragma unroll
  for (int u = 0; u < U; ++u) {
    const int idx = tid + u * 256, r = idx / CH, c = idx % CH;
    goff_k[u] = (uint32_t)(r * a.kst * 2 + c * 16);
    goff_v[u] = (uint32_t)(r * a.vst * 2 + c * 16);
  }
  auto tile_rs = [&](const T* base, int64_t st, int t) __attribute__((always_inline)) {
    const int rows = min(Tk - t * BN, BN);
    const uint32_t nrec = rows > 0 ? (uint32_t)((int64_t)(rows - 1) * st * 2 + 2 * D) : 0u;
    return __builtin_amdgcn_make_buffer_rsrc((void*)(base + (rows > 0 ? (int64_t)t * BN * st : 0)), (short)0,
                                             (int)nrec, 0x00020000);
  };
  auto load_k = [&](int t) __attribute__((always_inline)) {
    const auto rs = tile_rs(kp, a.kst, t);
#pragma unroll
    for (int u = 0; u < U; ++u) kreg[u] = __builtin_amdgcn_raw_buffer_load_b128(rs, goff_k[u], 0, 0);
  };
  auto load_v = [&](int t) __attribute__((always_inline)) {
    const auto rs = tile_rs(vp, a.vst, t);
#pragma unroll
    for (int u = 0; u < U; ++u) vreg[u] = __builtin_amdgcn_raw_buffer_load_b128(rs, goff_v[u], 0, 0);
  };
  auto kbuf = [&](int t) __attribute__((always_inline)) { return smem + (t & 1) * KT; };
  auto vbuf = [&](int t) __attribute__((always_inline)) { return smem + 2 * KT + (t & 1) * VT; };
  auto store_k = [&](int t) __attribute__((always_inline)) {
#pragma unroll
    for (int u = 0; u < U; ++u) {
      const int idx = tid + u * 256, r = idx / CH, c = idx % CH;
      lds_write16(kbuf(t) + r * KS + c * 8, kreg[u]);
    }
  };
  auto store_v = [&](int t) __attribute__((always_inline)) {
#pragma unroll
    for (int u = 0; u < U; ++u) {
      const int idx = tid + u * 256, r = idx / CH, c = idx % CH;
      lds_write16(vbuf(t) + r * VS + c * 8, vreg[u]);
    }
  };
  // score of tile t (the initial accumulator of its S chain) and the mask
  // word of tile t (bit 8 gi + i%4 <-> entry i, after the 4 hf shift)
  auto score_of = [&](int t, f32x16& sc) __attribute__((always_inline)) {
#pragma unroll
    for (int gi = 0; gi < 4; ++gi) {
      const f32x4 x = __builtin_bit_cast(
          f32x4, __builtin_amdgcn_raw_buffer_load_b128(srs, soff_row + (uint32_t)(t * BN + gi * 8) * 4, 0, 0));
#pragma unroll
      for (int e = 0; e < 4; ++e) sc[gi * 4 + e] = a.qsign < 0.f ? -x[e] : x[e];
    }
  };
  auto mask_of = [&](int t) __attribute__((always_inline)) -> uint32_t {
    if constexpr (MASK) return mbits[min(t * BN, Tk - 1) >> 5] >> (4 * hf);
    else return ~0u;
  };

  f32x16 oacc[NB];
#pragma unroll
  for (int nb = 0; nb < NB; ++nb) oacc[nb] = f32x16{};
  float m_run = kNegInf, l_run = 0.f;
  // transpose-read lane pattern: rows 4 hf + (lane / 4) % 4 (+8), columns
  // 16 ((lane / 16) % 2) + 4 (lane % 4) of each 32-column block
  const int tr_row = 4 * hf + ((lane >> 2) & 3);
  const int tr_col = ((lane >> 4) & 1) * 16 + (lane & 3) * 4;

  // Iteration j (0 .. nt): O += V(j-1)^T P(j-1) with the masking and row
  // maximum of tile j threaded through it, the rescale when a maximum grows,
  // then S(j+1) = K(j+1) Q^T with the exp, row sum and packing of P(j)
  // threaded through it -- one MFMA stream with the softmax VALU work in its
  // gaps.  Staging: K(j+2) and V(j) are loaded at the start of iteration j
  // and written at its end (K buffer j%2, last read in iteration j-1 by
  // S(j); V buffer j%2, last read in iteration j-1 by PV(j-2)), then a
  // barrier.  Past the tiles (iteration nt, S of tile nt) the work runs on
  // stale buffers and is discarded: every entry of a tile t >= nt (or wholly
  // above a causal wave's rows) is dropped, so its P is 0.
  V8 pk[2], pkl[PREC ? 2 : 1];
#pragma unroll
  for (int c = 0; c < 2; ++c) pk[c] = V8{};
#pragma unroll
  for (int c = 0; c < (PREC ? 2 : 1); ++c) pkl[c] = V8{};
  f32x16 sc = f32x16{}, s_cur;
  uint32_t mw_cur = mask_of(0), mw_nx = mask_of(1);
  // prologue: K(0), K(1) and a zeroed V buffer 1 (read as V(-1) with P = 0)
  load_k(0);
  store_k(0);
  load_k(1);
  store_k(1);
#pragma unroll
  for (int u = 0; u < U; ++u) {
    const int idx = tid + u * 256, r = idx / CH, c = idx % CH;
    lds_write16(vbuf(1) + r * VS + c * 8, u32x4{0, 0, 0, 0});
  }
  if constexpr (SCORE) score_of(0, sc);
  __syncthreads();
  {
    const T* ks = kbuf(0);
    s_cur = sc;
#pragma unroll
    for (int ds = 0; ds < DS; ++ds) s_cur = mfma32(as_vec8<T>(lds_read16(ks + l32 * KS + ds * 16 + hf * 8)), qf[ds], s_cur);
  }
  if constexpr (SCORE) score_of(1, sc);

  constexpr int AH = 3;   // LDS operand reads in flight per MFMA stream
#pragma nounroll
  for (int j = 0; j <= nt; ++j) {
    load_k(j + 2);
    load_v(j);
    const int k0 = j * BN;
    // Dropped entries of tile j to -inf (kept ones to 0 with scale 0) on the
    // tiles that have any: keep word bit 8 gi + e <-> entry 4 gi + e, key
    // k0 + 8 gi + 4 hf + e (keys below Tk, and up to the row when causal, are
    // a prefix of the bit positions); no bit past the tiles or for a tile
    // wholly above a causal wave's rows.
    {
      const bool live = j < nt && (!CAUSAL || k0 <= q0w + 31);
      const bool edge = !live || MASK || a.zero_scale || (k0 + BN > Tk) || (CAUSAL && k0 + BN - 1 > q0w);
      if (edge) {
        const int lim = CAUSAL ? min(Tk, qrow + 1) : Tk;
        const int nk = lim - (k0 + 4 * hf);
        uint32_t keepw = !live || nk <= 0 ? 0u : (nk >= 32 ? ~0u : (1u << nk) - 1u);
        if constexpr (MASK) keepw &= mw_cur;
#pragma unroll
        for (int i = 0; i < 16; ++i) {
          const bool keep = (keepw >> (8 * (i >> 2) + (i & 3))) & 1u;
          s_cur[i] = keep ? (a.zero_scale ? 0.f : s_cur[i]) : kNegInf;
        }
      }
    }

    // ---- block 1: PV(j-1) || maximum of tile j --------------------------------------
    float mx = kNegInf;
    {
      const T* vs = vbuf(j - 1);
      auto rd_v = [&](int t) __attribute__((always_inline)) -> V8 {   // t: c = t / NB, nb = t % NB
        const int row = 16 * (t / NB) + tr_row, col = (t % NB) * 32 + tr_col;
        return cat_tr<T>(lds_read_tr(vs + row * VS + col), lds_read_tr(vs + (row + 8) * VS + col));
      };
      V8 vq[AH];
#pragma unroll
      for (int t = 0; t < AH; ++t) vq[t] = rd_v(t);
#pragma unroll
      for (int t = 0; t < 2 * NB; ++t) {
        const int c = t / NB, nb = t % NB;
        oacc[nb] = mfma32(vq[t % AH], pk[c], oacc[nb]);
        if constexpr (PREC) oacc[nb] = mfma32(vq[t % AH], pkl[c], oacc[nb]);
        if (t + AH < 2 * NB) vq[t % AH] = rd_v(t + AH);
        mx = fmaxf(mx, s_cur[t]);
        __builtin_amdgcn_sched_group_barrier(0x008, PREC ? 2 : 1, 0);
        if (t + AH < 2 * NB) __builtin_amdgcn_sched_group_barrier(0x100, 2, 0);
        __builtin_amdgcn_sched_group_barrier(0x002, 1, 0);
      }
    }
    // The running maximum moves only when a row's maximum exceeds it by more
    // than kWLift (p stays below 2^kWLift meanwhile: O and l are fp32): the
    // rescale (O in AGPRs, read, scaled and written back) is rare.
    const float mt = half_max(mx) * c2;   // the row's largest logit of tile j (scaled)
    if (wave_any(mt > m_run + kWLift)) {
      const float m_new = fmaxf(m_run, mt);
      const float alpha = m_run == kNegInf ? 0.f : exp2_fast(m_run - m_new);
      l_run *= alpha;
#pragma unroll
      for (int nb = 0; nb < NB; ++nb) oacc[nb] *= alpha;
      m_run = m_new;
    }
    const float mneg = m_run == kNegInf ? 0.f : -m_run;

    // ---- block 2: S(j+1) || P(j) ---------------------------------------------------
    {
      const T* ks = kbuf(j + 1);
      auto rd_k = [&](int ds) __attribute__((always_inline)) -> u32x4 {
        return lds_read16(ks + l32 * KS + ds * 16 + hf * 8);
      };
      u32x4 kq[AH];
#pragma unroll
      for (int t = 0; t < AH; ++t) kq[t] = rd_k(t);
      f32x16 s_nxt = sc;
      float p[16], lsum = 0.f;
#pragma unroll
      for (int ds = 0; ds < DS; ++ds) {
        s_nxt = mfma32(as_vec8<T>(kq[ds % AH]), qf[ds], s_nxt);
        if (ds + AH < DS) kq[ds % AH] = rd_k(ds + AH);
        p[ds] = exp2_fast(fmaf(s_cur[ds], c2, mneg));
        lsum += p[ds];
        if ((ds & 7) == 7) {
          const int c = ds >> 3;
          pk[c] = pack8<T>(p[8 * c + 0], p[8 * c + 1], p[8 * c + 2], p[8 * c + 3], p[8 * c + 4], p[8 * c + 5],
                           p[8 * c + 6], p[8 * c + 7]);
          if constexpr (PREC) {
            float r[8];
#pragma unroll
            for (int e = 0; e < 8; ++e) r[e] = p[8 * c + e] - (float)(T)p[8 * c + e];
            pkl[c] = pack8<T>(r[0], r[1], r[2], r[3], r[4], r[5], r[6], r[7]);
          }
        }
        __builtin_amdgcn_sched_group_barrier(0x008, 1, 1);
        if (ds + AH < DS) __builtin_amdgcn_sched_group_barrier(0x100, 1, 1);
        __builtin_amdgcn_sched_group_barrier(0x002, PREC ? 5 : 3, 1);
      }
      l_run += lsum;
      s_cur = s_nxt;
    }
    // score / mask word of tile j+2 (the S chain above has taken tile j+1's)
    if constexpr (SCORE) score_of(j + 2, sc);
    mw_cur = mw_nx;
    mw_nx = mask_of(j + 2);
    store_k(j + 2);
    store_v(j);
    __syncthreads();
  }

  // ---- epilogue: O = acc / l (NaN for a row with no kept key), LSE ---------------
  const float l_tot = half_sum(l_run);
  const float inv = 1.0f / l_tot;
  T* os = smem + wave * 32 * OS;   // wave-private rows; the loop ended with a barrier
  constexpr int NU = 32 * CH / 64;
  auto put_rows = [&](bool resid, T* dst, int64_t sb, int64_t st, int64_t sh) __attribute__((always_inline)) {
#pragma unroll
    for (int nb = 0; nb < NB; ++nb)
#pragma unroll
      for (int gi = 0; gi < 4; ++gi) {
        float v[4];
#pragma unroll
        for (int t = 0; t < 4; ++t) {
          const float o = oacc[nb][gi * 4 + t] * inv;
          v[t] = resid ? o - (float)(T)o : o;
        }
        lds_write8(os + l32 * OS + nb * 32 + gi * 8 + hf * 4, pack4w<T>(v[0], v[1], v[2], v[3]));
      }
    asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
    u32x4 ov[NU];
#pragma unroll
    for (int u = 0; u < NU; ++u) {
      const int idx = lane + u * 64;
      ov[u] = lds_read16(os + (idx / CH) * OS + (idx % CH) * 8);
    }
    T* op = dst + b * sb + h * sh;
#pragma unroll
    for (int u = 0; u < NU; ++u) {
      const int idx = lane + u * 64, r = idx / CH, c = idx % CH;
      if (q0w + r < Tq) gstore16(op + (int64_t)(q0w + r) * st + c * 8, ov[u]);
    }
    asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
  };
  put_rows(false, (T*)a.o, a.osb, a.ost, a.osh);
  if (hf == 0 && qrow < Tq)
    a.lse[((int64_t)b * a.Hq + h) * Tq + qrow] = (l_tot > 0.f) ? m_run + log2_fast(l_tot) : kPosInf;
  if constexpr (PREC) {
    if (a.olo) put_rows(true, (T*)a.olo, a.olsb, a.olst, a.olsh);
  }
}

// ---------------------------------------------------------------------------
// dV (WHICH 0) / dK (WHICH 1)
// ---------------------------------------------------------------------------
template <typename T, bool CAUSAL, bool MASK, bool SCORE, int WHICH>
__global__ __launch_bounds__(256, 1) void kv_wide_kernel(const BwdArgs a) {
  using V8 = typename Vec8<T>::type;
  constexpr int D = kWD, DS = D / 16, NB = D / 32, CH = D / 8;
  constexpr bool DK = WHICH == 1;
  // padded row stride of the Q / dO tiles (row reads and transpose reads)
  constexpr int QS = D + 40;
  constexpr int QT = 32 * QS;
  constexpr int U = 32 * CH / 256;      // 16-byte chunks per thread per tile and kind
  constexpr int OS = D + 8;
  static_assert(4 * 32 * OS <= 4 * QT, "epilogue staging fits in the tile buffers");
  constexpr bool PREC = MASK || SCORE;
  __shared__ __attribute__((aligned(16))) T smem[4 * QT];          // [buf][Q | dO]
  __shared__ __attribute__((aligned(16))) float lsd[2][2][32];     // [buf][LSE | -Delta][row]

  const int nblk = a.nbk * a.nkt * a.split;
  const int W = xcd_remap(blockIdx.x, nblk);
  const int per_bk = a.split * a.nkt;
  const int bkl = W / per_bk;
  const int bk = a.bk0 + bkl;
  const int rem = W - bkl * per_bk;
  const int sp = rem / a.nkt;
  const int kt = rem - sp * a.nkt;    // ascending: causal work shrinks with the block
  const int b = bk / a.Hk, kvh = bk - b * a.Hk;

  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int l32 = lane & 31, hf = lane >> 5;
  const int Tq = a.Tq, Tk = a.Tk;
  const int kt0 = kt * kWKvKeys, kw0 = kt0 + wave * 32;
  const int key = kw0 + l32, kc = min(key, Tk - 1);
  const float c2 = a.scale_log2;

  // K (and V) fragments, B of S = Q K^T and dP = dO V^T: lane holds
  // K[key][16 ds + 8 hf .. +7]
  V8 kf[DS], vf[DK ? DS : 1];
  {
    const T* kp = (const T*)a.k + b * a.ksb + kvh * a.ksh + (int64_t)kc * a.kst + hf * 8;
    const T* vp = (const T*)a.v + b * a.vsb + kvh * a.vsh + (int64_t)kc * a.vst + hf * 8;
#pragma unroll
    for (int ds = 0; ds < DS; ++ds) {
      kf[ds] = as_vec8<T>(gload16(kp + ds * 16));
      if constexpr (DK) vf[ds] = as_vec8<T>(gload16(vp + ds * 16));
    }
  }
  // The fragments stay in AGPRs (MFMA reads its operands there too); the
  // dK or dV accumulator takes 128 VGPRs (results in VGPRs: this file is
  // built with VGPR-form MFMAs).
#pragma unroll
  for (int ds = 0; ds < DS; ++ds) {
    asm volatile("" : "+a"(kf[ds]));
    if constexpr (DK) asm volatile("" : "+a"(vf[ds]));
  }

  // steps: (head of the group split, 32-row step from qstart), rows above the
  // key block are masked when causal
  const int gsz = a.G / a.split;
  const int h_first = kvh * a.G + sp * gsz;
  const int qstart = CAUSAL ? (kt0 / 32) * 32 : 0;
  const int nst = qstart < Tq ? (Tq - qstart + 31) / 32 : 0;
  const int n = gsz * nst;

  // staging of step j: Q / dO rows (past Tq: row Tq-1, whose P is 0 there),
  // LSE (+inf past Tq) and -Delta (0 past Tq) of its rows
  u32x4 qreg[U], dreg[U];
  float lreg = 0.f;
  auto load_step = [&](int j) __attribute__((always_inline)) {
    const int hh = h_first + j / nst, qs = qstart + 32 * (j % nst);
    const T* qh = (const T*)a.q + b * a.qsb + (int64_t)hh * a.qsh;
    const T* dh = (const T*)a.dout + b * a.dsb + (int64_t)hh * a.dsh;
#pragma unroll
    for (int u = 0; u < U; ++u) {
      const int idx = tid + u * 256, r = idx / CH, c = idx % CH;
      const int qq = min(qs + r, Tq - 1);
      qreg[u] = gload16(qh + (int64_t)qq * a.qst + c * 8);
      dreg[u] = gload16(dh + (int64_t)qq * a.dst + c * 8);
    }
    if (tid < 64) {
      const int qq = qs + l32;
      const int64_t ri = ((int64_t)b * a.Hq + hh) * Tq + qq;
      lreg = hf == 0 ? (qq < Tq ? a.lse[ri] : kPosInf) : (qq < Tq ? -a.delta[ri] : 0.f);
    }
  };
  auto store_step = [&](int buf) __attribute__((always_inline)) {
    T* qs_ = smem + buf * 2 * QT;
    T* ds_ = qs_ + QT;
#pragma unroll
    for (int u = 0; u < U; ++u) {
      const int idx = tid + u * 256, r = idx / CH, c = idx % CH;
      lds_write16(qs_ + r * QS + c * 8, qreg[u]);
      lds_write16(ds_ + r * QS + c * 8, dreg[u]);
    }
    if (tid < 64) lsd[buf][hf][l32] = lreg;
  };

  f32x16 acc[NB];   // dV^T or dK^T [32 nb + 8 (i/4) + 4 hf + i%4][key]
#pragma unroll
  for (int nb = 0; nb < NB; ++nb) acc[nb] = f32x16{};
  const int tr_row = 4 * hf + ((lane >> 2) & 3);
  const int tr_col = ((lane >> 4) & 1) * 16 + (lane & 3) * 4;
  const uint32_t s_lane = SCORE ? (uint32_t)(((int64_t)4 * hf * a.ssq + kc) * 4) : 0u;
  const uint32_t s_row = (uint32_t)a.ssq * 4u;

  if (n > 0) {
    load_step(0);
    store_step(0);
  }
  __syncthreads();
  for (int j = 0; j < n; ++j) {
    const bool more = j + 1 < n;
    if (more) load_step(j + 1);
    const int buf = j & 1;
    const int hh = h_first + j / nst, qs = qstart + 32 * (j % nst);
    const T* qt_ = smem + buf * 2 * QT;
    const T* dt_ = qt_ + QT;
    // causal: a step wholly above the wave's keys adds nothing
    const bool active = !CAUSAL || qs + 31 >= kw0;
    if (active) {
      // lane entry i: row qs + 8 (i/4) + 4 hf + i%4 at key `key`
      f32x16 s = f32x16{};
      if constexpr (SCORE) {
        const uint32_t nrec = (uint32_t)(((int64_t)min(Tq - qs, 32) - 1) * a.ssq * 4 + (int64_t)Tk * 4);
        const auto rs = __builtin_amdgcn_make_buffer_rsrc(
            (void*)(a.score + b * a.ssb + (int64_t)hh * a.ssh + (int64_t)qs * a.ssq), (short)0, (int)nrec, 0x00020000);
#pragma unroll
        for (int i = 0; i < 16; ++i)
          s[i] = __builtin_bit_cast(float, __builtin_amdgcn_raw_buffer_load_b32(
                                               rs, s_lane, (uint32_t)(8 * (i >> 2) + (i & 3)) * s_row, 0));
      }
      uint32_t mw = ~0u;
      if constexpr (MASK) {
        const uint32_t* bt = (const uint32_t*)(a.mws + a.ml.bitsT + mask_plane(a.ml, b, hh) * a.ml.pbitsT);
        mw = bt[((int64_t)(kc >> 5) * a.ml.wq + (qs >> 5)) * 32 + (kc & 31)] >> (4 * hf);
      }
#pragma unroll
      for (int ds = 0; ds < DS; ++ds)
        s = mfma32(as_vec8<T>(lds_read16(qt_ + l32 * QS + ds * 16 + hf * 8)), kf[ds], s);
      f32x16 dp = f32x16{};
      if constexpr (DK) {
#pragma unroll
        for (int gi = 0; gi < 4; ++gi) {
          const f32x4 d4 = *(const f32x4*)&lsd[buf][1][8 * gi + 4 * hf];
#pragma unroll
          for (int t = 0; t < 4; ++t) dp[gi * 4 + t] = d4[t];
        }
#pragma unroll
        for (int ds = 0; ds < DS; ++ds)
          dp = mfma32(as_vec8<T>(lds_read16(dt_ + l32 * QS + ds * 16 + hf * 8)), vf[ds], dp);
      }
      float p[16];
#pragma unroll
      for (int gi = 0; gi < 4; ++gi) {
        const f32x4 l4 = *(const f32x4*)&lsd[buf][0][8 * gi + 4 * hf];
#pragma unroll
        for (int t = 0; t < 4; ++t) {
          const int i = gi * 4 + t, row = qs + 8 * gi + 4 * hf + t;
          const float sv = a.zero_scale ? 0.f : s[i];
          float pv = exp2_fast(fmaf(sv, c2, -l4[t]));
          bool keep = key < Tk;
          if constexpr (CAUSAL) keep = keep && key <= row;
          if constexpr (MASK) keep = keep && ((mw >> (8 * gi + t)) & 1u);
          pv = keep ? pv : 0.f;
          p[i] = DK ? pv * dp[i] : pv;   // dK: dS = P (dP - Delta) (scale applied at the end)
        }
      }
      // packed per 16-row step c: slot t <-> row 16 c + 8 (t/4) + 4 hf + t%4;
      // P in three parts (dV), dS in two (dK) with a mask or a score
      constexpr int NP = PREC ? (DK ? 2 : 3) : 1;
      V8 pk[2][NP];
#pragma unroll
      for (int c = 0; c < 2; ++c) {
        if constexpr (PREC) {
          u32x4 w[NP];
#pragma unroll
          for (int k = 0; k < 4; ++k) {
            uint32_t x0, x1, x2 = 0;
            if constexpr (DK) split2<T>(p[8 * c + 2 * k], p[8 * c + 2 * k + 1], &x0, &x1);
            else split3<T>(p[8 * c + 2 * k], p[8 * c + 2 * k + 1], &x0, &x1, &x2);
            w[0][k] = x0;
            w[1][k] = x1;
            if constexpr (NP == 3) w[NP - 1][k] = x2;
          }
#pragma unroll
          for (int x = 0; x < NP; ++x) pk[c][x] = as_vec8<T>(w[x]);
        } else {
          pk[c][0] = pack8<T>(p[8 * c + 0], p[8 * c + 1], p[8 * c + 2], p[8 * c + 3], p[8 * c + 4], p[8 * c + 5],
                              p[8 * c + 6], p[8 * c + 7]);
        }
      }
      // dV^T += dO^T P (A = dO^T) / dK^T += Q^T dS (A = Q^T), transpose reads
      const T* at = DK ? qt_ : dt_;
#pragma unroll
      for (int c = 0; c < 2; ++c) {
        const int row = 16 * c + tr_row;
#pragma unroll
        for (int nb = 0; nb < NB; ++nb) {
          const int col = nb * 32 + tr_col;
          const V8 av = cat_tr<T>(lds_read_tr(at + row * QS + col), lds_read_tr(at + (row + 8) * QS + col));
#pragma unroll
          for (int x = 0; x < NP; ++x) acc[nb] = mfma32(av, pk[c][x], acc[nb]);
        }
      }
    }
    if (more) store_step((j + 1) & 1);
    __syncthreads();
  }

  // ---- epilogue: dK (times scale) or dV (NaN for a kv-head with a dead row) --------
  const bool nan_out = !DK && a.dead[b * a.Hk + kvh] != 0;
  const float nanv = __builtin_nanf("");
  const float mul = DK ? a.scale : 1.f;
  if (a.split == 1) {
    T* stg = smem + wave * 32 * OS;   // wave-private rows; the loop ended with a barrier
#pragma unroll
    for (int nb = 0; nb < NB; ++nb)
#pragma unroll
      for (int gi = 0; gi < 4; ++gi) {
        const u32x2 v = nan_out ? pack4w<T>(nanv, nanv, nanv, nanv)
                                : pack4w<T>(acc[nb][gi * 4 + 0] * mul, acc[nb][gi * 4 + 1] * mul,
                                            acc[nb][gi * 4 + 2] * mul, acc[nb][gi * 4 + 3] * mul);
        lds_write8(stg + l32 * OS + nb * 32 + gi * 8 + hf * 4, v);
      }
    asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
    constexpr int NU = 32 * CH / 64;
    u32x4 ov[NU];
#pragma unroll
    for (int u = 0; u < NU; ++u) {
      const int idx = lane + u * 64;
      ov[u] = lds_read16(stg + (idx / CH) * OS + (idx % CH) * 8);
    }
    T* dst = DK ? (T*)a.dk + b * a.dksb + kvh * a.dksh : (T*)a.dv + b * a.dvsb + kvh * a.dvsh;
    const int64_t dstt = DK ? a.dkst : a.dvst;
#pragma unroll
    for (int u = 0; u < NU; ++u) {
      const int idx = lane + u * 64, r = idx / CH, c = idx % CH;
      if (kw0 + r < Tk) gstore16(dst + (int64_t)(kw0 + r) * dstt + c * 8, ov[u]);
    }
  } else {
    // head-group split: fp32 slabs [split][B, Tk, Hk, D], summed in a fixed order later
    const int64_t slab = (int64_t)sp * a.B * Tk * a.Hk * D;
    float* dst = DK ? a.dk_accum : a.dv_accum;
    if (key < Tk) {
#pragma unroll
      for (int nb = 0; nb < NB; ++nb)
#pragma unroll
        for (int gi = 0; gi < 4; ++gi) {
          const int d = nb * 32 + gi * 8 + hf * 4;
          const int64_t o = slab + (((int64_t)b * Tk + key) * a.Hk + kvh) * D + d;
          f32x4 v4;
#pragma unroll
          for (int t = 0; t < 4; ++t) v4[t] = nan_out ? nanv : acc[nb][gi * 4 + t] * mul;
          *(f32x4*)(dst + o) = v4;
        }
    }
  }
}

// ---------------------------------------------------------------------------
// dQ (recomputed): dQ = scale sum_k dS K, dS = P (dP - Delta)
// ---------------------------------------------------------------------------
// Chunk swizzle of the unpadded 512-byte rows of the dQ kernel's K and V
// tiles: chunk c of row r sits at chunk c ^ swz(r) (low four bits), so that
// 16 rows read at one chunk (ds_read_b128) and 4 rows x 4 chunks
// (ds_read_b64_tr_b16) both hit 64 distinct banks.
__device__ __forceinline__ int swz_w(int r) { return ((r & 3) << 2) | ((r >> 2) & 3); }

// 16 bytes per lane from a buffer straight into LDS: lane l's bytes land at
// lds_addr + 16 l (lds_addr wave-uniform).  (A plain device function: inside
// the kernel template the builtin kept its host-side stub from being emitted.)
__device__ __forceinline__ void lds_dma16(__amdgpu_buffer_rsrc_t rs, uint32_t lds_addr, uint32_t voff) {
  __builtin_amdgcn_raw_ptr_buffer_load_lds(rs, (FA_LDS void*)(uintptr_t)lds_addr, 16, voff, 0, 0, 0);
}

template <typename T, bool CAUSAL, bool MASK, bool SCORE>
__global__ __launch_bounds__(256, 1) void dq_wide_kernel(const BwdArgs a) {
  using V8 = typename Vec8<T>::type;
  constexpr int D = kWD, DS = D / 16, NB = D / 32, CH = D / 8;
  constexpr int BM = kWDqRows, BN = kWKeys;
  constexpr int TILEB = BN * D * 2;       // bytes of one K or V tile (32 rows of 512 bytes)
  // K tile t is read as rows by S(t) in iteration t-1 and transposed by
  // dQ(t) in iteration t+1, and written in iteration t-2: four buffers; V tile
  // t only by dP(t) in iteration t-1: two
  constexpr int NKB = 4, NVB = 2;
  constexpr int KOFF = 0, VOFF = NKB * TILEB;
  constexpr int OS = D + 8;               // epilogue staging stride (elements)
  static_assert(4 * 32 * OS * 2 <= (NKB + NVB) * TILEB, "dQ staging fits in the tile buffers");
  constexpr bool PREC = MASK || SCORE;
  __shared__ __attribute__((aligned(1024))) char smem[(NKB + NVB) * TILEB];

  // blocks as in the forward: causal longest first across all XCDs
  int b, h, qt;
  if constexpr (CAUSAL) {
    const int bh = a.B * a.Hq;
    const int r = blockIdx.x / bh, i = blockIdx.x - r * bh;
    b = i / a.Hq;
    h = i - b * a.Hq;
    qt = a.nqt - 1 - r;
  } else {
    const int W = xcd_remap(blockIdx.x, a.B * a.Hq * a.nqt);
    const int per_kv = a.G * a.nqt;
    const int bk = W / per_kv, rem = W - bk * per_kv;
    qt = rem / a.G;
    b = bk / a.Hk;
    h = (bk - b * a.Hk) * a.G + (rem - qt * a.G);
  }
  const int kvh = h / a.G;

  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int l32 = lane & 31, hf = lane >> 5;
  const int Tq = a.Tq, Tk = a.Tk;
  const int q0 = qt * BM, q0w = q0 + wave * 32, qrow = q0w + l32;
  const int qrow_c = min(qrow, Tq - 1);
  const float c2 = a.scale_log2;

  // Q and dO fragments (B of S^T = K Q^T and dP^T = V dO^T), kept in AGPRs;
  // rows past Tq read row Tq-1 (their LSE is +inf there: P = 0)
  V8 qf[DS], dof[DS];
  {
    const T* qs = (const T*)a.q + b * a.qsb + h * a.qsh + (int64_t)qrow_c * a.qst + hf * 8;
    const T* ds_ = (const T*)a.dout + b * a.dsb + h * a.dsh + (int64_t)qrow_c * a.dst + hf * 8;
#pragma unroll
    for (int ds = 0; ds < DS; ++ds) {
      qf[ds] = as_vec8<T>(gload16(qs + ds * 16));
      dof[ds] = as_vec8<T>(gload16(ds_ + ds * 16));
    }
  }
#pragma unroll
  for (int ds = 0; ds < DS; ++ds) asm volatile("" : "+a"(qf[ds]), "+a"(dof[ds]));
  const int64_t ri = ((int64_t)b * a.Hq + h) * Tq + qrow_c;
  const float lse_q = qrow < Tq ? a.lse[ri] : kPosInf;
  const float ndelta = qrow < Tq ? -a.delta[ri] : 0.f;

  const T* __restrict__ kp = (const T*)a.k + b * a.ksb + kvh * a.ksh;
  const T* __restrict__ vp = (const T*)a.v + b * a.vsb + kvh * a.vsh;
  const uint32_t* mbits = nullptr;
  if constexpr (MASK) {
    const int pm = mask_plane(a.ml, b, h);
    mbits = (const uint32_t*)(a.mws + a.ml.bits + pm * a.ml.pbits) + (int64_t)qrow_c * a.ml.wk;
  }
  const int srow0 = min(q0 + 32 * __builtin_amdgcn_readfirstlane(wave), Tq - 1);
  const __amdgpu_buffer_rsrc_t srs = __builtin_amdgcn_make_buffer_rsrc(
      SCORE ? (void*)(a.score + b * a.ssb + h * a.ssh + (int64_t)srow0 * a.ssq) : nullptr, (short)0,
      SCORE ? (int)(((int64_t)min(Tq - 1 - srow0, 31) * a.ssq + Tk) * 4) : 0, 0x00020000);
  const uint32_t soff_row = (uint32_t)((int64_t)(qrow_c - srow0) * a.ssq * 4) + hf * 16;

  const int kv_end = CAUSAL ? min(Tk, q0 + BM) : Tk;
  const int nt = (kv_end + BN - 1) / BN;

  // ---- staging: direct-to-LDS buffer loads --------------------------------------
  // Load u (0..3) of wave w writes the 1 KB of tile rows 8 w + 2 u, +1: lane l
  // lands at physical chunk l % 32 of row 8 w + 2 u + l / 32 and so fetches
  // logical chunk (l % 32) ^ swz(row); rows past Tk read zeros.
  const uint32_t lds0 = (uint32_t)(uintptr_t)(FA_LDS char*)smem;
  uint32_t goff_k[4], goff_v[4];
#pragma unroll
  for (int u = 0; u < 4; ++u) {
    const int r = 8 * wave + 2 * u + (lane >> 5), c = (lane & 31) ^ swz_w(r);
    goff_k[u] = (uint32_t)(r * a.kst * 2 + c * 16);
    goff_v[u] = (uint32_t)(r * a.vst * 2 + c * 16);
  }
  auto tile_rs = [&](const T* base, int64_t st, int t) __attribute__((always_inline)) {
    const int rows = min(Tk - t * BN, BN);
    const uint32_t nrec = rows > 0 ? (uint32_t)((int64_t)(rows - 1) * st * 2 + 2 * D) : 0u;
    return __builtin_amdgcn_make_buffer_rsrc((void*)(base + (rows > 0 ? (int64_t)t * BN * st : 0)), (short)0,
                                             (int)nrec, 0x00020000);
  };
  auto load_tiles = [&](int tk, int tv) __attribute__((always_inline)) {   // K(tk), V(tv)
    const auto rk = tile_rs(kp, a.kst, tk), rv = tile_rs(vp, a.vst, tv);
    const uint32_t dk = lds0 + KOFF + (tk & (NKB - 1)) * TILEB + 8 * wave * 512;
    const uint32_t dv = lds0 + VOFF + (tv & (NVB - 1)) * TILEB + 8 * wave * 512;
#pragma unroll
    for (int u = 0; u < 4; ++u) {
      lds_dma16(rk, dk + u * 1024, goff_k[u]);
      lds_dma16(rv, dv + u * 1024, goff_v[u]);
    }
  };
  auto loads_done = [&]() __attribute__((always_inline)) { asm volatile("s_waitcnt vmcnt(0)" ::: "memory"); };

  // ---- LDS read addresses ------------------------------------------------------
  // rows (A of S and dP): row l32, logical chunk 2 ds + hf -> byte
  // (row_base + 16 ((hf ^ swz(l32)))) ^ (32 ds) (row bases 512-aligned)
  const uint32_t arow = lds0 + l32 * 512 + 16 * (hf ^ swz_w(l32));
  // transposed (A of dQ^T = K^T dS^T): rows 16 c + tr_row (+8), columns
  // 32 nb + tr_col: byte (base + 16 ((tc ^ swz(row)))) ^ (64 nb) + c 8 KB
  const int tr_row = 4 * hf + ((lane >> 2) & 3);
  const int tr_col = ((lane >> 4) & 1) * 16 + (lane & 3) * 4;
  uint32_t atr[2];
#pragma unroll
  for (int hi = 0; hi < 2; ++hi) {
    const int r = tr_row + 8 * hi;
    atr[hi] = lds0 + r * 512 + 16 * ((tr_col >> 3) ^ swz_w(r)) + (tr_col & 7) * 2;
  }
  auto rd_row = [&](uint32_t buf, int ds) __attribute__((always_inline)) -> u32x4 {
    return *(const FA_LDS u32x4*)(uintptr_t)((arow ^ (uint32_t)(32 * ds)) + buf);
  };
  auto rd_tr = [&](uint32_t buf, int c, int nb) __attribute__((always_inline)) -> V8 {
    const uint32_t o = buf + (uint32_t)(c * 16 * 512);
    return cat_tr<T>(__builtin_amdgcn_ds_read_tr16_b64_v4i16((FA_LDS s16x4*)(uintptr_t)((atr[0] ^ (uint32_t)(64 * nb)) + o)),
                     __builtin_amdgcn_ds_read_tr16_b64_v4i16((FA_LDS s16x4*)(uintptr_t)((atr[1] ^ (uint32_t)(64 * nb)) + o)));
  };
  auto kbuf = [&](int t) __attribute__((always_inline)) { return (uint32_t)(KOFF + (t & (NKB - 1)) * TILEB); };
  auto vbuf = [&](int t) __attribute__((always_inline)) { return (uint32_t)(VOFF + (t & (NVB - 1)) * TILEB); };

  auto score_of = [&](int t, f32x16& sc) __attribute__((always_inline)) {
#pragma unroll
    for (int gi = 0; gi < 4; ++gi) {
      const f32x4 x = __builtin_bit_cast(
          f32x4, __builtin_amdgcn_raw_buffer_load_b128(srs, soff_row + (uint32_t)(t * BN + gi * 8) * 4, 0, 0));
#pragma unroll
      for (int e = 0; e < 4; ++e) sc[gi * 4 + e] = x[e];
    }
  };
  auto mask_of = [&](int t) __attribute__((always_inline)) -> uint32_t {
    if constexpr (MASK) return mbits[min(t * BN, Tk - 1) >> 5] >> (4 * hf);
    else return ~0u;
  };

  f32x16 acc[NB];    // dQ^T [32 nb + 8 (i/4) + 4 hf + i%4][q]
#pragma unroll
  for (int nb = 0; nb < NB; ++nb) acc[nb] = f32x16{};
  f32x16 nd;         // -Delta of the lane's row: initial accumulator of every dP chain
#pragma unroll
  for (int i = 0; i < 16; ++i) nd[i] = ndelta;
  V8 dk_[2], dkl[PREC ? 2 : 1];   // dS(j-1) packed per 16-key step (and its residual)
#pragma unroll
  for (int c = 0; c < 2; ++c) dk_[c] = V8{};
#pragma unroll
  for (int c = 0; c < (PREC ? 2 : 1); ++c) dkl[c] = V8{};
  f32x16 sc = f32x16{}, s_cur, dp_cur;
  uint32_t mw_cur = mask_of(0), mw_nx = mask_of(1);

  // prologue: K(0), V(0), K(1), V(1); K buffer 3 zeroed (read as K(-1) with dS = 0)
#pragma unroll
  for (int u = 0; u < TILEB / (256 * 16); ++u)
    *(FA_LDS u32x4*)(uintptr_t)(lds0 + KOFF + 3 * TILEB + (tid + u * 256) * 16) = u32x4{0, 0, 0, 0};
  load_tiles(0, 0);
  load_tiles(1, 1);
  if constexpr (SCORE) score_of(0, sc);
  loads_done();
  __syncthreads();
  s_cur = sc;
  dp_cur = nd;
#pragma unroll
  for (int ds = 0; ds < DS; ++ds) {
    s_cur = mfma32(as_vec8<T>(rd_row(kbuf(0), ds)), qf[ds], s_cur);
    dp_cur = mfma32(as_vec8<T>(rd_row(vbuf(0), ds)), dof[ds], dp_cur);
  }
  if constexpr (SCORE) score_of(1, sc);

  constexpr int AH = 3;
#pragma nounroll
  for (int j = 0; j <= nt; ++j) {
    load_tiles(j + 2, j + 2);
    const int k0 = j * BN;
    // keep word of tile j (bit 8 gi + e <-> entry 4 gi + e, key k0 + 8 gi + 4 hf
    // + e): keys below Tk and, causal, up to the row; none past the tiles
    uint32_t keepw;
    {
      const bool live = j < nt && (!CAUSAL || k0 <= q0w + 31);
      const int lim = CAUSAL ? min(Tk, qrow + 1) : Tk;
      const int nk = lim - (k0 + 4 * hf);
      keepw = !live || nk <= 0 ? 0u : (nk >= 32 ? ~0u : (1u << nk) - 1u);
      if constexpr (MASK) keepw &= mw_cur;
    }
    if (a.zero_scale) {
#pragma unroll
      for (int i = 0; i < 16; ++i) s_cur[i] = 0.f;
    }

    // ---- block 1: dQ(j-1) || P(j) ----------------------------------------------
    float p[16];
    {
      const uint32_t kb = kbuf(j - 1);
      V8 kq[AH];
#pragma unroll
      for (int t = 0; t < AH; ++t) kq[t] = rd_tr(kb, t / NB, t % NB);
#pragma unroll
      for (int t = 0; t < 2 * NB; ++t) {
        const int c = t / NB, nb = t % NB;
        acc[nb] = mfma32(kq[t % AH], dk_[c], acc[nb]);
        if constexpr (PREC) acc[nb] = mfma32(kq[t % AH], dkl[c], acc[nb]);
        if (t + AH < 2 * NB) kq[t % AH] = rd_tr(kb, (t + AH) / NB, (t + AH) % NB);
        // P of entry t: selected to 0 when dropped (whatever the exp gives)
        const float pv = exp2_fast(fmaf(s_cur[t], c2, -lse_q));
        p[t] = (keepw >> (8 * (t >> 2) + (t & 3))) & 1u ? pv : 0.f;
        __builtin_amdgcn_sched_group_barrier(0x008, PREC ? 2 : 1, 0);
        if (t + AH < 2 * NB) __builtin_amdgcn_sched_group_barrier(0x100, 2, 0);
        __builtin_amdgcn_sched_group_barrier(0x002, 4, 0);
      }
    }

    // ---- block 2: S(j+1), dP(j+1) || dS(j) ---------------------------------------
    {
      const uint32_t kb = kbuf(j + 1), vb = vbuf(j + 1);
      u32x4 xk[AH], xv[AH];
#pragma unroll
      for (int t = 0; t < AH; ++t) { xk[t] = rd_row(kb, t); xv[t] = rd_row(vb, t); }
      f32x16 s_nxt = sc, dp_nxt = nd;
      float dsv[16];
#pragma unroll
      for (int ds = 0; ds < DS; ++ds) {
        s_nxt = mfma32(as_vec8<T>(xk[ds % AH]), qf[ds], s_nxt);
        dp_nxt = mfma32(as_vec8<T>(xv[ds % AH]), dof[ds], dp_nxt);
        if (ds + AH < DS) { xk[ds % AH] = rd_row(kb, ds + AH); xv[ds % AH] = rd_row(vb, ds + AH); }
        dsv[ds] = p[ds] * dp_cur[ds];
        if ((ds & 7) == 7) {
          const int c = ds >> 3;
          if constexpr (PREC) {
            u32x4 wh, wl;
#pragma unroll
            for (int k = 0; k < 4; ++k) {
              uint32_t h2, l2;
              split2<T>(dsv[8 * c + 2 * k], dsv[8 * c + 2 * k + 1], &h2, &l2);
              wh[k] = h2;
              wl[k] = l2;
            }
            dk_[c] = as_vec8<T>(wh);
            dkl[c] = as_vec8<T>(wl);
          } else {
            dk_[c] = pack8<T>(dsv[8 * c + 0], dsv[8 * c + 1], dsv[8 * c + 2], dsv[8 * c + 3], dsv[8 * c + 4],
                              dsv[8 * c + 5], dsv[8 * c + 6], dsv[8 * c + 7]);
          }
        }
        __builtin_amdgcn_sched_group_barrier(0x008, 2, 1);
        if (ds + AH < DS) __builtin_amdgcn_sched_group_barrier(0x100, 2, 1);
        __builtin_amdgcn_sched_group_barrier(0x002, PREC ? 4 : 2, 1);
      }
      s_cur = s_nxt;
      dp_cur = dp_nxt;
    }
    if constexpr (SCORE) score_of(j + 2, sc);
    mw_cur = mw_nx;
    mw_nx = mask_of(j + 2);
    loads_done();
    __syncthreads();
  }

  // ---- epilogue: dQ = scale acc, through wave-private LDS rows ----------------------
  const float scale = a.scale;
  T* os = (T*)smem + wave * 32 * OS;
#pragma unroll
  for (int nb = 0; nb < NB; ++nb)
#pragma unroll
    for (int gi = 0; gi < 4; ++gi)
      lds_write8(os + l32 * OS + nb * 32 + gi * 8 + hf * 4,
                 pack4w<T>(acc[nb][gi * 4 + 0] * scale, acc[nb][gi * 4 + 1] * scale, acc[nb][gi * 4 + 2] * scale,
                           acc[nb][gi * 4 + 3] * scale));
  asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
  constexpr int NU = 32 * CH / 64;
  u32x4 ov[NU];
#pragma unroll
  for (int u = 0; u < NU; ++u) {
    const int idx = lane + u * 64;
    ov[u] = lds_read16(os + (idx / CH) * OS + (idx % CH) * 8);
  }
  T* dqp = (T*)a.dq + b * a.dqsb + h * a.dqsh;
#pragma unroll
  for (int u = 0; u < NU; ++u) {
    const int idx = lane + u * 64, r = idx / CH, c = idx % CH;
    if (q0w + r < Tq) gstore16(dqp + (int64_t)(q0w + r) * a.dqst + c * 8, ov[u]);
  }
}

template <typename T, bool CAUSAL>
hipError_t launch_dq_w(const BwdArgs& a, hipStream_t s) {
  const dim3 grid((unsigned)(a.B * a.Hq * a.nqt)), block(256);
  const bool m = a.mask != nullptr, sc = a.score != nullptr;
  if (m && sc) hipLaunchKernelGGL((dq_wide_kernel<T, CAUSAL, true, true>), grid, block, 0, s, a);
  else if (m) hipLaunchKernelGGL((dq_wide_kernel<T, CAUSAL, true, false>), grid, block, 0, s, a);
  else if (sc) hipLaunchKernelGGL((dq_wide_kernel<T, CAUSAL, false, true>), grid, block, 0, s, a);
  else hipLaunchKernelGGL((dq_wide_kernel<T, CAUSAL, false, false>), grid, block, 0, s, a);
  return hipGetLastError();
}

template <typename T, bool CAUSAL>
hipError_t launch_fwd_w(const FwdArgs& a, hipStream_t s) {
  const dim3 grid((unsigned)(a.B * a.Hq * a.nqt)), block(256);
  const bool m = a.mask != nullptr, sc = a.score != nullptr;
  if (m && sc) hipLaunchKernelGGL((fwd_wide_kernel<T, CAUSAL, true, true>), grid, block, 0, s, a);
  else if (m) hipLaunchKernelGGL((fwd_wide_kernel<T, CAUSAL, true, false>), grid, block, 0, s, a);
  else if (sc) hipLaunchKernelGGL((fwd_wide_kernel<T, CAUSAL, false, true>), grid, block, 0, s, a);
  else hipLaunchKernelGGL((fwd_wide_kernel<T, CAUSAL, false, false>), grid, block, 0, s, a);
  return hipGetLastError();
}

template <typename T, bool CAUSAL, int WHICH>
hipError_t launch_kv_w(const BwdArgs& a, hipStream_t s) {
  const dim3 grid((unsigned)(a.nbk * a.nkt * a.split)), block(256);
  const bool m = a.mask != nullptr, sc = a.score != nullptr;
  if (m && sc) hipLaunchKernelGGL((kv_wide_kernel<T, CAUSAL, true, true, WHICH>), grid, block, 0, s, a);
  else if (m) hipLaunchKernelGGL((kv_wide_kernel<T, CAUSAL, true, false, WHICH>), grid, block, 0, s, a);
  else if (sc) hipLaunchKernelGGL((kv_wide_kernel<T, CAUSAL, false, true, WHICH>), grid, block, 0, s, a);
  else hipLaunchKernelGGL((kv_wide_kernel<T, CAUSAL, false, false, WHICH>), grid, block, 0, s, a);
  return hipGetLastError();
}

template <typename T, bool CAUSAL>
hipError_t launch_kv_both(const BwdArgs& a, hipStream_t s) {
  const hipError_t e = launch_kv_w<T, CAUSAL, 0>(a, s);
  return e != hipSuccess ? e : launch_kv_w<T, CAUSAL, 1>(a, s);
}

}  // namespace

int fwd_wide_block_rows() { return kWRows; }
int dq_wide_block_rows() { return kWDqRows; }

hipError_t launch_bwd_dq_wide(const BwdArgs& a, int dtype, bool causal, hipStream_t s) {
  if (dtype == 0) return causal ? launch_dq_w<bf16, true>(a, s) : launch_dq_w<bf16, false>(a, s);
  return causal ? launch_dq_w<f16, true>(a, s) : launch_dq_w<f16, false>(a, s);
}
int kv_wide_block_keys() { return kWKvKeys; }

hipError_t launch_fwd_wide(const FwdArgs& a, int dtype, bool causal, hipStream_t s) {
  if (dtype == 0) return causal ? launch_fwd_w<bf16, true>(a, s) : launch_fwd_w<bf16, false>(a, s);
  return causal ? launch_fwd_w<f16, true>(a, s) : launch_fwd_w<f16, false>(a, s);
}

hipError_t launch_bwd_kv_wide(const BwdArgs& a, int dtype, bool causal, hipStream_t s) {
  if (dtype == 0) return causal ? launch_kv_both<bf16, true>(a, s) : launch_kv_both<bf16, false>(a, s);
  return causal ? launch_kv_both<f16, true>(a, s) : launch_kv_both<f16, false>(a, s);
}

}  // namespace fa
